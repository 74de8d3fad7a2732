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

template <int LPR, int NB, int kMode, int TPW>
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
                                       std::uint32_t cols, float eps) {
  __shared__ __attribute__((aligned(16))) std::int8_t lxq[NB][kProjMaxCols];
  __shared__ float lxs[NB][kProjMaxCols / 32];
  __shared__ float red[4];
  constexpr int P = kWave / LPR;  // rows per task
  constexpr std::uint32_t kStep = LPR * 16;
  const std::uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, nblk = cols / 32;
  // TPW tasks per wave: block b covers tasks [4 TPW b, 4 TPW (b + 1)), wave w the tasks 4 TPW b + 4 i + w
  const std::uint32_t task0 = blockIdx.x * (blockDim.x / kWave) * TPW + wave;
  // Order of issue: token 0's prologue inputs (L2 hits), then the weights of this wave's first two tasks (HBM),
  // so the prologue of token 0 waits only for its own loads while the weight stream is in flight.
  // 2048-column chunks of the row per 256 threads: cols <= 64 LPR, so one chunk unless LPR = 64
  constexpr int KC = LPR == 64 ? 2 : 1;
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
        if (blockIdx.x == 0 && res_out != nullptr && delta != nullptr) halo::StoreRow8(res_out + off, cols, row);
        halo::RmsNormRow8W(row, aux, cols, eps, red);
      }
      if constexpr (kMode == 3) halo::GatedNormRow8W(row, aux, w8, cols, eps);
      halo::QuantRow8(row, cols, &lxq[b][0], &lxs[b][0]);
      if (blockIdx.x == 0 && xq_out != nullptr) halo::QuantRow8(row, cols, xq_out + off, xs_out + b * nblk);
    }
  };
  static_assert(kProjMaxCols / 16 <= 256, "one 16-byte piece of a quantized row per thread");
  load_token(0);
  // The tasks' loads are unconditional (a load in a conditional block costs a vmcnt(0) wait at the join): a
  // wave past the end of the list reloads the last task and stores nothing.
  RowLoad<LPR> cur[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i)
    LoadTask<LPR>(cur[i], min(task0 + 4u * i, o4 - 1), o1, o2, o3, qs0, d0, rows0, qs1, d1, rows1, qs2, d2, rows2,
                  qs3, d3, rows3, cols);
  finish_token(0);
  for (std::uint32_t b = 1; b < T; ++b) {
    load_token(b);
    finish_token(b);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const std::uint32_t task = task0 + 4u * i;
    if (task >= o4) break;
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
                               d2, y2, qs3, d3, y3, rows0, rows1, rows2, rows3, o1, o2, o3, o4, T, cols, eps);   \
  }
#define HALO_PROJ_Q8_T(MODE, LETTER, LPR, NB) \
  HALO_PROJ_Q8(MODE, LETTER, LPR, NB, 1) HALO_PROJ_Q8(MODE, LETTER, LPR, NB, 2) HALO_PROJ_Q8(MODE, LETTER, LPR, NB, 4)
#define HALO_PROJ_Q8_NB(MODE, LETTER, LPR)                                                                \
  HALO_PROJ_Q8_T(MODE, LETTER, LPR, 1) HALO_PROJ_Q8_T(MODE, LETTER, LPR, 2) HALO_PROJ_Q8_T(MODE, LETTER, LPR, 4) \
  HALO_PROJ_Q8_T(MODE, LETTER, LPR, 8)
#define HALO_PROJ_Q8_L(MODE, LETTER) \
  HALO_PROJ_Q8_NB(MODE, LETTER, 64) HALO_PROJ_Q8_NB(MODE, LETTER, 32) HALO_PROJ_Q8_NB(MODE, LETTER, 16)
HALO_PROJ_Q8_L(0, q)
HALO_PROJ_Q8_L(1, f)
HALO_PROJ_Q8_L(2, n)
HALO_PROJ_Q8_L(3, g)
#undef HALO_PROJ_Q8_L
#undef HALO_PROJ_Q8_T
#undef HALO_PROJ_Q8_NB
#undef HALO_PROJ_Q8
