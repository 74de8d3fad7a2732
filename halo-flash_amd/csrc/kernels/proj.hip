// Grouped Q8_0 projections with the activation prologue fused in (gfx950, wave64; MI355X-native, no reference
// kernel of this shape).
//
// One launch computes up to four Q8_0 x int8-activation products that share their input row(s) x [T][cols]
// (T <= NB tokens): the q|k|v, z and alpha|beta projections of a DeltaNet layer, the q|gate, k and v projections of
// an attention layer, or the C1 q/gate and kv pair. The reference issues one FlashNextGpu::MatVec per matrix
// (src/engine/flash_next_gpu.cpp:212-254), each after a separate quantize launch (halo_quantize_q8_rows,
// src/kernels/core.hip:3089-3101) and, for the first projections of a layer, after the RMSNorm launch.
//
// Prologue modes (kernel name letter):
//   q  x is already quantized (xq [T][cols] int8, xs [T][cols / 32]);
//   f  x [T][cols] fp32 is quantized in the prologue (amax / 127, round half to even);
//   n  x = RMSNorm(res + delta) * w, then quantized; block 0 writes res + delta to res_out (never the buffer it
//      reads) so the residual stream stays consistent without a separate norm launch;
//   g  x = per 128-value head RMSNorm(o) * w * sigmoid(z) (the DeltaNet output norm; z passed as delta), then
//      quantized.
// The row prologue is the canonical decomposition of common.h: the quantized bytes equal those of
// halo_quantize_q8_rows / halo_add_rmsnorm_q8 / halo_gated_rmsnorm_q8 for the same input.
//
// Work split: 256-thread blocks, LPR lanes per row, a task = 64 / LPR rows of one matrix, one task per wave (a
// grid of many small blocks keeps more loads in flight on MI355X than a persistent grid walking a task list: the
// dispatcher refills CUs as waves retire). Each wave's weight loads are issued before the prologue, after the
// prologue's own loads, so the HBM stream overlaps the norm and quantization; x is then read from LDS.
#include "common.h"

using halo::kWave;

namespace {

constexpr std::uint32_t kProjMaxCols = 4096;

template <int LPR>
struct RowLoad {
  int4 q[4];
  float s[4];
};

// The weight pieces of task `task` (P = 64 / LPR consecutive rows of one matrix) for this lane.
template <int LPR>
__device__ __forceinline__ void LoadTask(RowLoad<LPR>& w, std::uint32_t task, std::uint32_t o1, std::uint32_t o2,
                                         std::uint32_t o3, const std::int8_t* qs0, const std::uint16_t* d0,
                                         std::uint32_t rows0, const std::int8_t* qs1, const std::uint16_t* d1,
                                         std::uint32_t rows1, const std::int8_t* qs2, const std::uint16_t* d2,
                                         std::uint32_t rows2, const std::int8_t* qs3, const std::uint16_t* d3,
                                         std::uint32_t rows3, std::uint32_t cols) {
  constexpr int P = kWave / LPR;
  constexpr std::uint32_t kStep = LPR * 16;
  const std::uint32_t lane = threadIdx.x % kWave, nblk = cols / 32;
  const std::uint32_t m = task < o1 ? 0 : task < o2 ? 1 : task < o3 ? 2 : 3;
  const std::uint32_t lt = task - (m == 0 ? 0 : m == 1 ? o1 : m == 2 ? o2 : o3);
  const std::int8_t* qs = m == 0 ? qs0 : m == 1 ? qs1 : m == 2 ? qs2 : qs3;
  const std::uint16_t* d = m == 0 ? d0 : m == 1 ? d1 : m == 2 ? d2 : d3;
  const std::uint32_t rows = m == 0 ? rows0 : m == 1 ? rows1 : m == 2 ? rows2 : rows3;
  const std::uint32_t r = min(lt * P + lane / LPR, rows - 1);
  const std::int8_t* rowp = qs + static_cast<std::size_t>(r) * cols;
  const std::uint16_t* dp = d + static_cast<std::size_t>(r) * nblk;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const std::uint32_t c = (lane % LPR) * 16 + u * kStep;
    const bool ok = c < cols;
    const std::uint32_t cc = ok ? c : (lane % LPR) * 16;
    w.q[u] = __builtin_bit_cast(int4, __builtin_nontemporal_load(reinterpret_cast<const halo::V4i*>(rowp + cc)));
    const float sv = halo::F16(dp[cc / 32]);  // unconditional: a load under a branch costs a vmcnt(0) wait
    w.s[u] = ok ? sv : 0.0f;
  }
}

// The mode-n prologue of one row (n <= 2048) for waves 0-3 of a block without a block barrier: each wave loads
// the whole residual row and forms the sum of squares of all four waves itself, with the arithmetic of
// halo::LoadRow8 / RmsNormRow8W (lane l's partial j is thread l + 64 j's, GroupSum adds the same lanes in the same
// tree, the four wave sums are added in order: the same bits), then normalizes and quantizes its own chunk as
// thread threadIdx.x of the 256-thread layout. Block 0 writes res + delta to res_out and, with xq_out, the codes.
__device__ __forceinline__ void WideNormRow(const float* __restrict__ x, const float* __restrict__ delta,
                                            const float* __restrict__ nw, float* __restrict__ res_out,
                                            std::int8_t* __restrict__ xq_out, float* __restrict__ xs_out,
                                            std::uint32_t n, float eps, std::int8_t* lxq, float* lxs) {
  const std::uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  float v[4][8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const std::uint32_t c = lane + 64u * j, cc = min(c, n / 8 - 1);
    const float4 a = reinterpret_cast<const float4*>(x)[2 * cc], b = reinterpret_cast<const float4*>(x)[2 * cc + 1];
    const float* dsrc = delta != nullptr ? delta : x;
    const float on = delta != nullptr ? 1.0f : 0.0f;
    const float4 e = reinterpret_cast<const float4*>(dsrc)[2 * cc], f = reinterpret_cast<const float4*>(dsrc)[2 * cc + 1];
    const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}, dv[8] = {e.x, e.y, e.z, e.w, f.x, f.y, f.z, f.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) v[j][k] = c < n / 8 ? xv[k] + dv[k] * on : 0.0f;
  }
  halo::Row8<1> w8;
  halo::LoadRow8(nw, nullptr, n, w8);
  float ws[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[j][e], v[j][e], ss);
    ws[j] = halo::GroupSum(ss);
  }
  const float ss = ((ws[0] + ws[1]) + ws[2]) + ws[3];
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
  halo::Row8<1> row;
#pragma unroll
  for (int e = 0; e < 8; ++e) row.v[0][e] = wave == 0 ? v[0][e] : wave == 1 ? v[1][e] : wave == 2 ? v[2][e] : v[3][e];
  if (blockIdx.x == 0 && res_out != nullptr && delta != nullptr) halo::StoreRow8(res_out, n, row);
  if (threadIdx.x < n / 8)
#pragma unroll
    for (int e = 0; e < 8; ++e) row.v[0][e] = row.v[0][e] * scale * w8.v[0][e];
  halo::QuantRow8(row, n, lxq, lxs);
  if (blockIdx.x == 0 && xq_out != nullptr) halo::QuantRow8(row, n, xq_out, xs_out);
}

// The staged activation rows, one allocation per token count whatever the lanes per row, so a launch that runs two
// tilings (halo_proj_q8q2_*) holds one copy.
template <int NB>
__device__ __forceinline__ std::int8_t (&ProjLxq())[NB][kProjMaxCols] {
  __shared__ __attribute__((aligned(16))) std::int8_t a[NB][kProjMaxCols];
  return a;
}
template <int NB>
__device__ __forceinline__ float (&ProjLxs())[NB][kProjMaxCols / 32] {
  __shared__ float a[NB][kProjMaxCols / 32];
  return a;
}

template <int LPR, int NB, int kMode, int TPW, bool kWide = false>
__device__ __forceinline__ void ProjQ8(const float* __restrict__ x, const float* __restrict__ delta,
                                       const float* __restrict__ nw, float* __restrict__ res_out,
                                       const std::int8_t* __restrict__ xq_in, const float* __restrict__ xs_in,
                                       std::int8_t* __restrict__ xq_out, float* __restrict__ xs_out,
                                       const std::int8_t* qs0, const std::uint16_t* d0, float* y0,
                                       const std::int8_t* qs1, const std::uint16_t* d1, float* y1,
                                       const std::int8_t* qs2, const std::uint16_t* d2, float* y2,
                                       const std::int8_t* qs3, const std::uint16_t* d3, float* y3, std::uint32_t rows0,
                                       std::uint32_t rows1, std::uint32_t rows2, std::uint32_t rows3, std::uint32_t o1,
                                       std::uint32_t o2, std::uint32_t o3, std::uint32_t o4, std::uint32_t T,
                                       std::uint32_t cols, float eps, std::uint32_t bid) {
  auto& lxq = ProjLxq<NB>();
  auto& lxs = ProjLxs<NB>();
  __shared__ float red[4];
  constexpr int P = kWave / LPR;  // rows per task
  constexpr std::uint32_t kStep = LPR * 16;
  const std::uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, nblk = cols / 32;
  // TPW tasks per wave: block b covers tasks [W TPW b, W TPW (b + 1)), wave w the tasks W TPW b + W i + w (W waves)
  constexpr std::uint32_t kWaves = kWide ? 8 : 4;
  const std::uint32_t task0 = bid * kWaves * TPW + wave;
  // Order of issue: token 0's prologue inputs (L2 hits), then the weights of this wave's first two tasks (HBM),
  // so the prologue of token 0 waits only for its own loads while the weight stream is in flight.
  // 2048-column chunks of the row per 256 threads: cols <= 64 LPR, so one chunk unless LPR = 64
  constexpr int KC = LPR == 64 ? 2 : 1;
  static_assert(!kWide || (kMode == 2 && NB == 1 && KC == 1), "the 8-wave form: one token, RMSNorm prologue");
  halo::Row8<KC> row, aux;
  float w8[8];
  int4 xv = make_int4(0, 0, 0, 0);
  float xsv = 0.0f;
  auto load_token = [&](std::uint32_t b) {
    const std::size_t off = static_cast<std::size_t>(b) * cols;
    if constexpr (kMode == 0) {
      xv = reinterpret_cast<const int4*>(xq_in + off)[min(threadIdx.x, cols / 16 - 1)];
      xsv = xs_in[static_cast<std::size_t>(b) * nblk + min(threadIdx.x, nblk - 1)];
    } else {
      halo::LoadRow8(x + off, kMode == 2 && delta != nullptr ? delta + off : nullptr, cols, row);
      if constexpr (kMode == 2) {
        if (b == 0) halo::LoadRow8(nw, nullptr, cols, aux);
      }
      if constexpr (kMode == 3) {
        halo::LoadRow8(delta + off, nullptr, cols, aux);
        if (b == 0) {
          const float4 wa = reinterpret_cast<const float4*>(nw)[2 * (threadIdx.x % 16)],
                       wb = reinterpret_cast<const float4*>(nw)[2 * (threadIdx.x % 16) + 1];
          w8[0] = wa.x, w8[1] = wa.y, w8[2] = wa.z, w8[3] = wa.w, w8[4] = wb.x, w8[5] = wb.y, w8[6] = wb.z, w8[7] = wb.w;
        }
      }
    }
  };
  auto finish_token = [&](std::uint32_t b) {
    const std::size_t off = static_cast<std::size_t>(b) * cols;
    if constexpr (kMode == 0) {
      if (threadIdx.x < cols / 16) reinterpret_cast<int4*>(&lxq[b][0])[threadIdx.x] = xv;
      if (threadIdx.x < nblk) lxs[b][threadIdx.x] = xsv;
    } else {
      if constexpr (kMode == 2) {
        if (bid == 0 && res_out != nullptr && delta != nullptr) halo::StoreRow8(res_out + off, cols, row);
        halo::RmsNormRow8W(row, aux, cols, eps, red);
      }
      if constexpr (kMode == 3) halo::GatedNormRow8W(row, aux, w8, cols, eps);
      halo::QuantRow8(row, cols, &lxq[b][0], &lxs[b][0]);
      if (bid == 0 && xq_out != nullptr) halo::QuantRow8(row, cols, xq_out + off, xs_out + b * nblk);
    }
  };
  static_assert(kProjMaxCols / 16 <= 256, "one 16-byte piece of a quantized row per thread");
  RowLoad<LPR> cur[TPW];
  if constexpr (kMode == 2) HALO_PHASE(2, 0);
  if constexpr (kWide) {
    // 8 waves: waves 0-3 form the normalized, quantized row without a block barrier (WideNormRow) and only then
    // issue their weight loads; waves 4-7 issue theirs at once. A wave's loads issue in order and stall while the
    // weight stream is queued, so a prologue placed behind its own weight loads, or waiting at a barrier for waves
    // that are, would finish only once most of the stream is in flight.
    if (wave < 4) {
      WideNormRow(x, delta, nw, res_out, xq_out, xs_out, cols, eps, &lxq[0][0], &lxs[0][0]);
      HALO_PHASE(2, 1);
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i)
      LoadTask<LPR>(cur[i], min(task0 + kWaves * i, o4 - 1), o1, o2, o3, qs0, d0, rows0, qs1, d1, rows1, qs2, d2, rows2,
                    qs3, d3, rows3, cols);
  } else if constexpr (kMode == 0) {
    // quantized rows straight into LDS, issued before the weights: every token's row (wave w its 16-byte pieces
    // 64 w .. 64 w + 63, from clamped addresses; pieces past the row land in the row's unused tail) and, by waves 0
    // and 1, its scales (128 slots, those past nblk unused); a clamped token past T reloads the last. Register
    // staging let the compiler sink the row loads behind the weights, so the block waited for its weights before
    // its barrier.
    const std::uint32_t lx = static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>(&lxq[0][0]));
    const std::uint32_t ls = static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>(&lxs[0][0]));
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const std::uint32_t bb = min(static_cast<std::uint32_t>(b), T - 1);
      halo::DmaRow16(xq_in + static_cast<std::size_t>(bb) * cols, min(64 * wave + lane, cols / 16 - 1) * 16,
                     lx + b * kProjMaxCols + 64 * wave * 16);
      if (wave < 2)
        halo::DmaDword(xs_in + static_cast<std::size_t>(bb) * nblk + min(64 * wave + lane, nblk - 1),
                       ls + (b * (kProjMaxCols / 32) + 64 * wave) * 4);
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i)
      LoadTask<LPR>(cur[i], min(task0 + kWaves * i, o4 - 1), o1, o2, o3, qs0, d0, rows0, qs1, d1, rows1, qs2, d2, rows2,
                    qs3, d3, rows3, cols);
    // the rows and scales have landed; the weights (8 loads a task) stay in flight (the count of loads between the
    // DMAs and this wait is checked on the built code)
    halo::WaitVmem<8 * TPW>();
  } else {
  load_token(0);
  // The tasks' loads are unconditional (a load in a conditional block costs a vmcnt(0) wait at the join): a
  // wave past the end of the list reloads the last task and stores nothing.
#pragma unroll
  for (int i = 0; i < TPW; ++i)
    LoadTask<LPR>(cur[i], min(task0 + kWaves * i, o4 - 1), o1, o2, o3, qs0, d0, rows0, qs1, d1, rows1, qs2, d2, rows2,
                  qs3, d3, rows3, cols);
  finish_token(0);
  if constexpr (kMode == 2) HALO_PHASE(2, 1);
  for (std::uint32_t b = 1; b < T; ++b) {
    load_token(b);
    finish_token(b);
  }
  }
  __syncthreads();
  if constexpr (kMode == 2) HALO_PHASE(2, 2);
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const std::uint32_t task = task0 + kWaves * i;
    if (task >= o4) break;
    if constexpr (kMode == 2) {
      if (i == 1) HALO_PHASE(2, 3);
    }
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const std::uint32_t c = (lane % LPR) * 16 + u * kStep;
      if (c < cols) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int4 xq4 = *reinterpret_cast<const int4*>(&lxq[b][c]);
          const float part = lxs[b][c / 32] * static_cast<float>(halo::Dot16(cur[i].q[u], xq4));
          acc[b] += cur[i].s[u] * part;
        }
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = halo::GroupSum<LPR>(acc[b]);
    const std::uint32_t m = task < o1 ? 0 : task < o2 ? 1 : task < o3 ? 2 : 3;
    const std::uint32_t lt = task - (m == 0 ? 0 : m == 1 ? o1 : m == 2 ? o2 : o3);
    float* y = m == 0 ? y0 : m == 1 ? y1 : m == 2 ? y2 : y3;
    const std::uint32_t rows = m == 0 ? rows0 : m == 1 ? rows1 : m == 2 ? rows2 : rows3;
    const std::uint32_t r = lt * P + lane / LPR;
    if (r < rows && lane % LPR == 0)
#pragma unroll
      for (int b = 0; b < NB; ++b)
        if (b < static_cast<int>(T)) y[static_cast<std::size_t>(b) * rows + r] = acc[b];
  }
  if constexpr (kMode == 2) HALO_PHASE(2, 4);
}

}  // namespace

// grid (ceil(o_4 / (4 TPW))), block 256. The work is a list of tasks of 64 / LPR rows: matrix m (m < 4, rows_m = 0
// when absent) owns tasks [o_m, o_{m+1}) with o_0 = 0, o_4 = the total; block b computes tasks [4 TPW b, 4 TPW b +
// 4 TPW) (TPW tasks per wave, all loaded before the prologue, which runs once per block). y_m [T][rows_m].
// Weight rows are unpadded (qstride = cols), cols % 32 == 0, cols <= 64 * LPR, T <= NB.
#define HALO_PROJ_Q8(MODE, LETTER, LPR, NB, TPW)                                                                  \
  extern "C" __global__ void __launch_bounds__(256) halo_proj_q8##LETTER##_l##LPR##_b##NB##_t##TPW(              \
      const float* x, const float* delta, const float* nw, float* res_out, const std::int8_t* xq_in,           \
      const float* xs_in, std::int8_t* xq_out, float* xs_out, const std::int8_t* qs0, const std::uint16_t* d0,   \
      float* y0, const std::int8_t* qs1, const std::uint16_t* d1, float* y1, const std::int8_t* qs2,            \
      const std::uint16_t* d2, float* y2, const std::int8_t* qs3, const std::uint16_t* d3, float* y3,           \
      std::uint32_t rows0, std::uint32_t rows1, std::uint32_t rows2, std::uint32_t rows3, std::uint32_t o1,     \
      std::uint32_t o2, std::uint32_t o3, std::uint32_t o4, std::uint32_t T, std::uint32_t cols, float eps) {   \
    ProjQ8<LPR, NB, MODE, TPW>(x, delta, nw, res_out, xq_in, xs_in, xq_out, xs_out, qs0, d0, y0, qs1, d1, y1, qs2, \
                               d2, y2, qs3, d3, y3, rows0, rows1, rows2, rows3, o1, o2, o3, o4, T, cols, eps,   \
                               blockIdx.x);                                                                       \
  }
#define HALO_PROJ_Q8_T(MODE, LETTER, LPR, NB) \
  HALO_PROJ_Q8(MODE, LETTER, LPR, NB, 1) HALO_PROJ_Q8(MODE, LETTER, LPR, NB, 2) HALO_PROJ_Q8(MODE, LETTER, LPR, NB, 4)
#define HALO_PROJ_Q8_NB(MODE, LETTER, LPR)                                                                \
  HALO_PROJ_Q8_T(MODE, LETTER, LPR, 1) HALO_PROJ_Q8_T(MODE, LETTER, LPR, 2) HALO_PROJ_Q8_T(MODE, LETTER, LPR, 4) \
  HALO_PROJ_Q8_T(MODE, LETTER, LPR, 8)
#define HALO_PROJ_Q8_L(MODE, LETTER) \
  HALO_PROJ_Q8_NB(MODE, LETTER, 64) HALO_PROJ_Q8_NB(MODE, LETTER, 32) HALO_PROJ_Q8_NB(MODE, LETTER, 16)
// grid (ceil(o_4 / (8 TPW))), block 512: the mode-n kernel of one token, waves 4-7 streaming weights while waves 0-3
// form the normalized row (LPR <= 32, cols <= 2048); otherwise as above.
#define HALO_PROJ_Q8W(LPR, TPW)                                                                                    \
  extern "C" __global__ void __launch_bounds__(512) halo_proj_q8w_l##LPR##_t##TPW(                                \
      const float* x, const float* delta, const float* nw, float* res_out, const std::int8_t* xq_in,           \
      const float* xs_in, std::int8_t* xq_out, float* xs_out, const std::int8_t* qs0, const std::uint16_t* d0,   \
      float* y0, const std::int8_t* qs1, const std::uint16_t* d1, float* y1, const std::int8_t* qs2,            \
      const std::uint16_t* d2, float* y2, const std::int8_t* qs3, const std::uint16_t* d3, float* y3,           \
      std::uint32_t rows0, std::uint32_t rows1, std::uint32_t rows2, std::uint32_t rows3, std::uint32_t o1,     \
      std::uint32_t o2, std::uint32_t o3, std::uint32_t o4, std::uint32_t T, std::uint32_t cols, float eps) {   \
    ProjQ8<LPR, 1, 2, TPW, true>(x, delta, nw, res_out, xq_in, xs_in, xq_out, xs_out, qs0, d0, y0, qs1, d1, y1, qs2, \
                                 d2, y2, qs3, d3, y3, rows0, rows1, rows2, rows3, o1, o2, o3, o4, T, cols, eps, \
                                 blockIdx.x);                                                                     \
  }
HALO_PROJ_Q8W(32, 1)
HALO_PROJ_Q8W(32, 2)
HALO_PROJ_Q8W(32, 4)
HALO_PROJ_Q8W(16, 1)
HALO_PROJ_Q8W(16, 2)
HALO_PROJ_Q8W(16, 4)
#undef HALO_PROJ_Q8W
// grid (nb1 + ceil(o_3' / 4)), block 256: two grouped mode-q projections with their own quantized inputs in one
// launch. Blocks b < nb1 = ceil(o_2 / 4) run matrices 0 and 1 on (xq, xs, cols) with LPR1 lanes per row (tasks
// [0, o_2)); blocks b >= nb1 run matrix 2 on (xq2, xs2, cols2) with LPR2 (its own task list of o_3' tasks), each part
// exactly as halo_proj_q8q_l<LPR>_b<NB>_t1 (the same bits).
#define HALO_PROJ_Q8Q2(L1, L2, NB)                                                                                \
  extern "C" __global__ void __launch_bounds__(256) halo_proj_q8q2_l##L1##x##L2##_b##NB(                          \
      const std::int8_t* xq, const float* xs, const std::int8_t* qs0, const std::uint16_t* d0, float* y0,         \
      const std::int8_t* qs1, const std::uint16_t* d1, float* y1, std::uint32_t rows0, std::uint32_t rows1,       \
      std::uint32_t o1, std::uint32_t o2, std::uint32_t cols, const std::int8_t* xq2, const float* xs2,           \
      const std::int8_t* qs2, const std::uint16_t* d2, float* y2, std::uint32_t rows2, std::uint32_t o3,          \
      std::uint32_t cols2, std::uint32_t nb1, std::uint32_t T) {                                                  \
    if (blockIdx.x < nb1)                                                                                         \
      ProjQ8<L1, NB, 0, 1>(nullptr, nullptr, nullptr, nullptr, xq, xs, nullptr, nullptr, qs0, d0, y0, qs1, d1, y1,  \
                           qs0, d0, y0, qs0, d0, y0, rows0, rows1, 0, 0, o1, o2, o2, o2, T, cols, 0.0f, blockIdx.x); \
    else                                                                                                          \
      ProjQ8<L2, NB, 0, 1>(nullptr, nullptr, nullptr, nullptr, xq2, xs2, nullptr, nullptr, qs2, d2, y2, qs2, d2, y2, \
                           qs2, d2, y2, qs2, d2, y2, rows2, 0, 0, 0, o3, o3, o3, o3, T, cols2, 0.0f,               \
                           blockIdx.x - nb1);                                                                     \
  }
HALO_PROJ_Q8Q2(32, 64, 2)
HALO_PROJ_Q8Q2(32, 64, 4)
HALO_PROJ_Q8Q2(32, 64, 8)
HALO_PROJ_Q8Q2(32, 32, 4)
HALO_PROJ_Q8Q2(32, 32, 8)
HALO_PROJ_Q8Q2(64, 64, 4)
HALO_PROJ_Q8Q2(64, 64, 8)
#undef HALO_PROJ_Q8Q2
HALO_PROJ_Q8_L(0, q)
HALO_PROJ_Q8_L(1, f)
HALO_PROJ_Q8_L(2, n)
HALO_PROJ_Q8_L(3, g)
#undef HALO_PROJ_Q8_L
#undef HALO_PROJ_Q8_T
#undef HALO_PROJ_Q8_NB
#undef HALO_PROJ_Q8

// ---- grouped projections of up to 16 quantized token rows on int8 matrix cores -------------------------------
// The same products as halo_proj_q8q_* (mode q: xq [T][cols] int8, xs [T][cols / 32]) for T <= 16, where the VALU
// form's dot4 chains grow with T (four v_dot4 and two FMAs per 16 weight bytes and token). A block of 8 waves owns
// one task of 16 rows of one matrix; wave w the 64 S columns from 64 S w (S = cols / 512 steps of 64 columns, two
// Q8_0 blocks each) on v_mfma_i32_16x16x64_i8: A = the 16 token rows, B = the 16 weight rows, lane l supplying the
// 16 bytes at column 16 (l / 16) of the step for token / row l % 16, so each lane's weight load is one 16-byte piece
// of its row. The step's two Q8_0 blocks need separate integer sums (each has its own scales): two MFMAs share the
// weight operand, the activation operand holding only the first block's lanes (l / 16 < 2) in one and only the
// second block's in the other. D lane l holds tokens 4 (l / 16) + i of row l % 16; its fp32 epilogue per block is
// acc += d_w (s_x float(isum)), blocks in ascending order within the wave, then the 8 waves' partial sums are added
// in wave order through LDS. Each token's outputs depend on its own row only, so they carry the same bits whatever
// T. Small waves (8 per 16-row task, S <= 8 weight loads each, all issued first) keep the weight stream's requests in
// flight across the chip; the activation scales sit in LDS transposed ([block][token]). (Measured on the C1 q|gate +
// kv pair: 8 waves x 4 steps 7.5 us at 16 tokens, 16 x 2 8.3, 4 x 8 7.4; the int8 MFMAs themselves cost nothing
// measurable, the weight-scale loads 0.7 us, the activation loads 1.4 us at 16 tokens.)
namespace {
typedef int V4I32p __attribute__((ext_vector_type(4)));
constexpr std::uint32_t kMfmaWaves = 8;

template <int S>  // 64-column steps per wave: cols = 512 S
__device__ __forceinline__ void ProjQ8Mfma(const std::int8_t* __restrict__ xq, const float* __restrict__ xs,
                                           const std::int8_t* qs0, const std::uint16_t* d0, float* y0,
                                           const std::int8_t* qs1, const std::uint16_t* d1, float* y1,
                                           const std::int8_t* qs2, const std::uint16_t* d2, float* y2,
                                           const std::int8_t* qs3, const std::uint16_t* d3, float* y3,
                                           std::uint32_t rows0, std::uint32_t rows1, std::uint32_t rows2,
                                           std::uint32_t rows3, std::uint32_t o1, std::uint32_t o2, std::uint32_t o3,
                                           std::uint32_t T, std::uint32_t task) {
  constexpr std::uint32_t cols = 64 * kMfmaWaves * S, nblk = cols / 32, kThreads = 64 * kMfmaWaves;
  __shared__ __attribute__((aligned(16))) float sxt[nblk][16];
  __shared__ __attribute__((aligned(16))) float red[kMfmaWaves - 1][64][4];
  const std::uint32_t tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, g = lane / 16, li = lane % 16;
  const std::uint32_t m = task < o1 ? 0 : task < o2 ? 1 : task < o3 ? 2 : 3;
  const std::uint32_t lt = task - (m == 0 ? 0 : m == 1 ? o1 : m == 2 ? o2 : o3);
  const std::int8_t* qs = m == 0 ? qs0 : m == 1 ? qs1 : m == 2 ? qs2 : qs3;
  const std::uint16_t* d = m == 0 ? d0 : m == 1 ? d1 : m == 2 ? d2 : d3;
  float* y = m == 0 ? y0 : m == 1 ? y1 : m == 2 ? y2 : y3;
  const std::uint32_t rows = m == 0 ? rows0 : m == 1 ? rows1 : m == 2 ? rows2 : rows3;
  const std::uint32_t row = min(lt * 16 + li, rows - 1), tok = min(li, T - 1);
  const std::uint32_t c0 = wave * 64 * S;
  // the activation scales first (vmcnt counts in order: their wait must not include the weight stream)
  constexpr std::uint32_t kSx = (nblk * 16 + kThreads - 1) / kThreads;
  float sxr[kSx];
#pragma unroll
  for (std::uint32_t j = 0; j < kSx; ++j) {
    const std::uint32_t e = min(tid + kThreads * j, nblk * 16 - 1), b = e / 16, t = e % 16;
    sxr[j] = xs[static_cast<std::size_t>(min(t, T - 1)) * nblk + b];
  }
  __builtin_amdgcn_sched_barrier(0);
  const std::int8_t* wp = qs + static_cast<std::size_t>(row) * cols + c0 + 16 * g;
  const std::int8_t* xp = xq + static_cast<std::size_t>(tok) * cols + c0 + 16 * g;
  const std::uint16_t* dp = d + static_cast<std::size_t>(row) * nblk + c0 / 32;
  int4 w[S], x[S];
#pragma unroll
  for (int s = 0; s < S; ++s)
    w[s] = __builtin_bit_cast(int4, __builtin_nontemporal_load(reinterpret_cast<const halo::V4i*>(wp + 64 * s)));
  std::uint16_t dsv[2 * S];  // the wave's 2 S block scales of this row: 16-byte loads (8 bytes at S = 2)
  if constexpr (S >= 4) {
#pragma unroll
    for (int j = 0; j < S / 4; ++j) {
      const uint4 v = *reinterpret_cast<const uint4*>(dp + 8 * j);
      __builtin_memcpy(dsv + 8 * j, &v, 16);
    }
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(dp);
    __builtin_memcpy(dsv, &v, 8);
  }
#pragma unroll
  for (int s = 0; s < S; ++s) x[s] = *reinterpret_cast<const int4*>(xp + 64 * s);
  __builtin_amdgcn_sched_barrier(0);
  // unconditional stores (a thread past the table rewrites its last entry with the value it loaded for it): a
  // store under `e < nblk * 16` let the compiler sink that load into the branch, where it waited for the weights
#pragma unroll
  for (std::uint32_t j = 0; j < kSx; ++j) {
    const std::uint32_t e = min(tid + kThreads * j, nblk * 16 - 1), b = e / 16, t = e % 16;
    sxt[b][t] = t < T ? sxr[j] : 0.0f;
  }
  // nothing of the products moves above the barrier (a product hoisted there waits for the weights first)
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const bool first_half = g < 2;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int4 xv = x[s];
    const V4I32p xa = first_half ? V4I32p{xv.x, xv.y, xv.z, xv.w} : V4I32p{0, 0, 0, 0};
    const V4I32p xb = first_half ? V4I32p{0, 0, 0, 0} : V4I32p{xv.x, xv.y, xv.z, xv.w};
    const V4I32p wb = {w[s].x, w[s].y, w[s].z, w[s].w};
    const V4I32p zero = {0, 0, 0, 0};
    const V4I32p ia = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, wb, zero, 0, 0, 0);
    const V4I32p ib = __builtin_amdgcn_mfma_i32_16x16x64_i8(xb, wb, zero, 0, 0, 0);
    const std::uint32_t blk = c0 / 32 + 2 * s;
    const float dwa = halo::F16(dsv[2 * s]), dwb = halo::F16(dsv[2 * s + 1]);
    const float4 sa = *reinterpret_cast<const float4*>(&sxt[blk][4 * g]);
    const float4 sb = *reinterpret_cast<const float4*>(&sxt[blk + 1][4 * g]);
    const float sav[4] = {sa.x, sa.y, sa.z, sa.w}, sbv[4] = {sb.x, sb.y, sb.z, sb.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i] += dwa * (sav[i] * static_cast<float>(ia[i]));
      acc[i] += dwb * (sbv[i] * static_cast<float>(ib[i]));
    }
  }
  if (wave > 0)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave - 1][lane][i] = acc[i];
  __syncthreads();
  if (wave == 0) {
    const std::uint32_t r = lt * 16 + li;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = acc[i];
#pragma unroll
      for (std::uint32_t u = 0; u + 1 < kMfmaWaves; ++u) v += red[u][lane][i];
      const std::uint32_t t = 4 * g + i;
      if (r < rows && t < T) y[static_cast<std::size_t>(t) * rows + r] = v;
    }
  }
}
}  // namespace

// grid (o_4) (one 16-row task per block), block 512. Matrix m owns tasks [o_m, o_{m+1}) (16 rows each, o_0 = 0);
// y_m [T][rows_m]. cols = 512 S (the kernel name's c<cols / 1024>: 1024, 2048 or 4096), unpadded rows (qstride =
// cols), 1 <= T <= 16.
#define HALO_PROJ_Q8M(C, S)                                                                                        \
  extern "C" __global__ void __launch_bounds__(512) halo_proj_q8m_c##C(                                           \
      const std::int8_t* xq, const float* xs, const std::int8_t* qs0, const std::uint16_t* d0, float* y0,       \
      const std::int8_t* qs1, const std::uint16_t* d1, float* y1, const std::int8_t* qs2, const std::uint16_t* d2, \
      float* y2, const std::int8_t* qs3, const std::uint16_t* d3, float* y3, std::uint32_t rows0,                 \
      std::uint32_t rows1, std::uint32_t rows2, std::uint32_t rows3, std::uint32_t o1, std::uint32_t o2,          \
      std::uint32_t o3, std::uint32_t T) {                                                                        \
    ProjQ8Mfma<S>(xq, xs, qs0, d0, y0, qs1, d1, y1, qs2, d2, y2, qs3, d3, y3, rows0, rows1, rows2, rows3, o1, o2, o3, \
                  T, blockIdx.x);                                                                                 \
  }
HALO_PROJ_Q8M(1, 2)
HALO_PROJ_Q8M(2, 4)
HALO_PROJ_Q8M(4, 8)
#undef HALO_PROJ_Q8M

// grid (o_2 + o_3'), block 512: two of the above in one launch with their own quantized inputs: blocks b < o_2 run
// matrices 0 and 1 (2048 columns) on (xq, xs), blocks b >= o_2 matrix 2 (4096 columns) on (xq2, xs2), each exactly
// as halo_proj_q8m_c2 / _c4 (the same bits). 1 <= T <= 16.
extern "C" __global__ void __launch_bounds__(512) halo_proj_q8m2_c2x4(
    const std::int8_t* xq, const float* xs, const std::int8_t* qs0, const std::uint16_t* d0, float* y0,
    const std::int8_t* qs1, const std::uint16_t* d1, float* y1, std::uint32_t rows0, std::uint32_t rows1,
    std::uint32_t o1, std::uint32_t o2, const std::int8_t* xq2, const float* xs2, const std::int8_t* qs2,
    const std::uint16_t* d2, float* y2, std::uint32_t rows2, std::uint32_t T) {
  if (blockIdx.x < o2)
    ProjQ8Mfma<4>(xq, xs, qs0, d0, y0, qs1, d1, y1, qs0, d0, y0, qs0, d0, y0, rows0, rows1, 0, 0, o1, o2, o2, T,
                  blockIdx.x);
  else
    ProjQ8Mfma<8>(xq2, xs2, qs2, d2, y2, qs2, d2, y2, qs2, d2, y2, qs2, d2, y2, rows2, 0, 0, 0, 0xFFFFFFFFu,
                  0xFFFFFFFFu, 0xFFFFFFFFu, T, blockIdx.x - o2);
}
