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
//      reads) so the residual stream stays consistent without a separate norm launch.
// The row prologue is the canonical decomposition of common.h: the quantized bytes equal those of
// halo_quantize_q8_rows / halo_add_rmsnorm_q8 for the same input.
//
// Work split: 256-thread blocks, LPR lanes per row (64 / LPR rows per wave, 4 waves), blockIdx.x ranges
// [o_m, o_{m+1}) select matrix m. Each wave issues all of its weight loads (cols <= 64 * LPR bytes per row)
// before the prologue runs, so the HBM stream overlaps the norm and quantization; x is then read from LDS.
#include "common.h"

using halo::kWave;

namespace {

constexpr std::uint32_t kProjMaxCols = 4096;

template <int LPR, int NB, int kMode>
__device__ __forceinline__ void ProjQ8(const float* __restrict__ x, const float* __restrict__ delta,
                                       const float* __restrict__ nw, float* __restrict__ res_out,
                                       const std::int8_t* __restrict__ xq_in, const float* __restrict__ xs_in,
                                       std::int8_t* __restrict__ xq_out, float* __restrict__ xs_out,
                                       const std::int8_t* qs, const std::uint16_t* d, float* y, std::uint32_t rows,
                                       std::uint32_t lb, std::uint32_t T, std::uint32_t cols, float eps) {
  __shared__ __attribute__((aligned(16))) std::int8_t lxq[NB][kProjMaxCols];
  __shared__ float lxs[NB][kProjMaxCols / 32];
  __shared__ float red[4];
  constexpr int P = kWave / LPR;          // rows per wave
  constexpr std::uint32_t kStep = LPR * 16;
  const std::uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, nblk = cols / 32;
  const std::uint32_t r = (lb * 4 + wave) * P + lane / LPR;
  const bool row_ok = r < rows;
  const std::uint32_t rr = row_ok ? r : rows - 1;
  const std::int8_t* rowp = qs + static_cast<std::size_t>(rr) * cols;
  const std::uint16_t* dp = d + static_cast<std::size_t>(rr) * nblk;
  // weights first: every load of the row is in flight before the prologue
  int4 q[4];
  float s[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const std::uint32_t c = (lane % LPR) * 16 + u * kStep;
    const bool ok = c < cols;
    const std::uint32_t cc = ok ? c : (lane % LPR) * 16;
    q[u] = __builtin_bit_cast(int4, __builtin_nontemporal_load(reinterpret_cast<const halo::V4i*>(rowp + cc)));
    s[u] = ok ? halo::F16(dp[cc / 32]) : 0.0f;
  }
  // prologue: the T activation rows into LDS as Q8
  for (std::uint32_t b = 0; b < T; ++b) {
    if constexpr (kMode == 0) {
      for (std::uint32_t i = threadIdx.x; i < cols / 16; i += blockDim.x)
        reinterpret_cast<int4*>(&lxq[b][0])[i] =
            reinterpret_cast<const int4*>(xq_in + static_cast<std::size_t>(b) * cols)[i];
      for (std::uint32_t i = threadIdx.x; i < nblk; i += blockDim.x) lxs[b][i] = xs_in[static_cast<std::size_t>(b) * nblk + i];
    } else {
      halo::Row8<kProjMaxCols / 2048> row;
      const std::size_t off = static_cast<std::size_t>(b) * cols;
      halo::LoadRow8(x + off, kMode == 2 && delta != nullptr ? delta + off : nullptr, cols, row);
      if constexpr (kMode == 2) {
        if (blockIdx.x == 0 && res_out != nullptr && delta != nullptr) halo::StoreRow8(res_out + off, cols, row);
        halo::RmsNormRow8(row, nw, cols, eps, red);
      }
      halo::QuantRow8(row, cols, &lxq[b][0], &lxs[b][0]);
      if (blockIdx.x == 0 && xq_out != nullptr) halo::QuantRow8(row, cols, xq_out + off, xs_out + b * nblk);
    }
  }
  __syncthreads();
  float acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const std::uint32_t c = (lane % LPR) * 16 + u * kStep;
    if (c < cols) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int4 xv = *reinterpret_cast<const int4*>(&lxq[b][c]);
        const float part = lxs[b][c / 32] * static_cast<float>(halo::Dot16(q[u], xv));
        acc[b] += s[u] * part;
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = halo::GroupSum<LPR>(acc[b]);
  if (row_ok && lane % LPR == 0)
#pragma unroll
    for (int b = 0; b < NB; ++b)
      if (b < static_cast<int>(T)) y[static_cast<std::size_t>(b) * rows + r] = acc[b];
}

}  // namespace

// grid (o1 + blocks of matrix 3 ...), block 256. Matrix m (m < 4, rows_m = 0 when absent) covers blocks
// [o_m, o_{m+1}) with o_0 = 0; y_m [T][rows_m]. Weight rows are unpadded (qstride = cols), cols % 32 == 0,
// cols <= 64 * LPR, T <= NB.
#define HALO_PROJ_Q8(MODE, LETTER, LPR, NB)                                                                       \
  extern "C" __global__ void __launch_bounds__(256) halo_proj_q8##LETTER##_l##LPR##_b##NB(                       \
      const float* x, const float* delta, const float* nw, float* res_out, const std::int8_t* xq_in,           \
      const float* xs_in, std::int8_t* xq_out, float* xs_out, const std::int8_t* qs0, const std::uint16_t* d0,   \
      float* y0, const std::int8_t* qs1, const std::uint16_t* d1, float* y1, const std::int8_t* qs2,            \
      const std::uint16_t* d2, float* y2, const std::int8_t* qs3, const std::uint16_t* d3, float* y3,           \
      std::uint32_t rows0, std::uint32_t rows1, std::uint32_t rows2, std::uint32_t rows3, std::uint32_t o1,     \
      std::uint32_t o2, std::uint32_t o3, std::uint32_t T, std::uint32_t cols, float eps) {                      \
    const std::uint32_t bx = blockIdx.x;                                                                          \
    const std::uint32_t m = bx < o1 ? 0 : bx < o2 ? 1 : bx < o3 ? 2 : 3;                                        \
    const std::uint32_t lb = bx - (m == 0 ? 0 : m == 1 ? o1 : m == 2 ? o2 : o3);                               \
    const std::int8_t* qs = m == 0 ? qs0 : m == 1 ? qs1 : m == 2 ? qs2 : qs3;                                   \
    const std::uint16_t* d = m == 0 ? d0 : m == 1 ? d1 : m == 2 ? d2 : d3;                                      \
    float* y = m == 0 ? y0 : m == 1 ? y1 : m == 2 ? y2 : y3;                                                    \
    const std::uint32_t rows = m == 0 ? rows0 : m == 1 ? rows1 : m == 2 ? rows2 : rows3;                        \
    ProjQ8<LPR, NB, MODE>(x, delta, nw, res_out, xq_in, xs_in, xq_out, xs_out, qs, d, y, rows, lb, T, cols, eps); \
  }
#define HALO_PROJ_Q8_NB(MODE, LETTER, LPR) \
  HALO_PROJ_Q8(MODE, LETTER, LPR, 1) HALO_PROJ_Q8(MODE, LETTER, LPR, 2) HALO_PROJ_Q8(MODE, LETTER, LPR, 4) \
  HALO_PROJ_Q8(MODE, LETTER, LPR, 8)
#define HALO_PROJ_Q8_L(MODE, LETTER) \
  HALO_PROJ_Q8_NB(MODE, LETTER, 64) HALO_PROJ_Q8_NB(MODE, LETTER, 32) HALO_PROJ_Q8_NB(MODE, LETTER, 16)
HALO_PROJ_Q8_L(0, q)
HALO_PROJ_Q8_L(1, f)
HALO_PROJ_Q8_L(2, n)
#undef HALO_PROJ_Q8_L
#undef HALO_PROJ_Q8_NB
#undef HALO_PROJ_Q8
