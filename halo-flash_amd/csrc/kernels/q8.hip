// Q8_0 repack, activation quantizer and the decode GEMV family (gfx950, wave64).
//
// Weight layout in HBM (reference src/kernels/core.hip:2116-2124): a Q8_0 matrix [rows][cols] is repacked once at
// load into int8 rows `qs` (row stride `qstride` bytes, a multiple of 16) and fp16 scales `d` [rows][cols / 32].
// Activations are quantized per 32 values to int8 `xq` with an fp32 scale `xs` (amax / 127, round half to even).
//
// The GEMV streams weights with one 16-byte load per lane per row: a row is covered by LPR lanes (LPR * 16 bytes
// per instruction), a wave covers 64 / LPR rows per pass and R passes, so a wave owns R * 64 / LPR rows and keeps
// R * U 16-byte loads per lane in flight (U column steps issued before any arithmetic). The integer part of every
// 16-value half block is an exact v_dot4_i32_i8 chain; the epilogue per half block is acc += s_w * (s_x * isum).
#include "common.h"

#include <type_traits>

using halo::Dot16;
using halo::F16;
using halo::kWave;

// ---- repack ------------------------------------------------------------------------------------------------
// reference src/kernels/core.hip:2126-2138. One thread per 16-byte output vector (half a Q8_0 block): the 16 codes
// are read as eight 2-byte words (a 34-byte block is only 2-byte aligned) and written as one int4; the thread of the
// first half also moves the block's fp16 scale. Grid-stride over rows * (cols / 16) vectors.
extern "C" __global__ void __launch_bounds__(256)
    halo_repack_q8_0(const std::uint8_t* raw, std::int8_t* qs, std::uint16_t* d, std::uint32_t rows,
                     std::uint32_t cols, std::uint32_t qstride) {
  const std::uint64_t halves_per_row = cols / 16, n = halves_per_row * rows;
  for (std::uint64_t v = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; v < n;
       v += static_cast<std::uint64_t>(gridDim.x) * blockDim.x) {
    const std::uint64_t row = v / halves_per_row, h = v % halves_per_row, blk = row * (cols / 32) + h / 2;
    const std::uint16_t* src = reinterpret_cast<const std::uint16_t*>(raw + blk * 34);  // [scale][16 code pairs]
    std::uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<std::uint32_t>(src[1 + 8 * (h & 1) + 2 * i]) |
             (static_cast<std::uint32_t>(src[2 + 8 * (h & 1) + 2 * i]) << 16);
    *reinterpret_cast<int4*>(qs + row * qstride + 16 * h) =
        make_int4(static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]), static_cast<int>(w[3]));
    if ((h & 1) == 0) d[blk] = src[0];
  }
}

// ---- activation quantizer -----------------------------------------------------------------------------------
// reference src/kernels/core.hip:3089-3101. grid (T), any multiple of 64 threads; x [T][cols] -> xq [T][cols],
// xd [T][cols / 32]. A lane quantizes 4 values from one 16-byte load, 8 lanes per Q8_0 block (halo::QuantQuad: IEEE
// divide, round half to even), and stores its 4 codes as one word.
extern "C" __global__ void __launch_bounds__(256)
    halo_quantize_q8_rows(const float* x, std::int8_t* xq, float* xd, std::uint32_t cols) {
  const std::size_t t = blockIdx.x;
  const float4* row = reinterpret_cast<const float4*>(x + t * cols);
  std::uint32_t* codes = reinterpret_cast<std::uint32_t*>(xq + t * cols);
  for (std::uint32_t g = threadIdx.x; g < cols / 4; g += blockDim.x) {  // 8-lane groups stay whole (cols % 32)
    float scale;
    codes[g] = halo::QuantQuad(row[g], scale);
    if (g % 8 == 0) xd[t * (cols / 32) + g / 8] = scale;
  }
}

// Two independent inputs in one launch, grid (2 T): block t < T quantizes row t of x0 (cols0 wide), block T + t row t
// of x1 (cols1 wide), each as halo_quantize_q8_rows (the same bytes).
extern "C" __global__ void __launch_bounds__(256)
    halo_quantize_q8_rows2(const float* x0, std::int8_t* xq0, float* xd0, std::uint32_t cols0, const float* x1,
                           std::int8_t* xq1, float* xd1, std::uint32_t cols1, std::uint32_t T) {
  const bool second = blockIdx.x >= T;
  const std::size_t t = second ? blockIdx.x - T : blockIdx.x;
  const std::uint32_t cols = second ? cols1 : cols0;
  const float4* row = reinterpret_cast<const float4*>((second ? x1 : x0) + t * cols);
  std::uint32_t* codes = reinterpret_cast<std::uint32_t*>((second ? xq1 : xq0) + t * cols);
  float* xd = second ? xd1 : xd0;
  for (std::uint32_t g = threadIdx.x; g < cols / 4; g += blockDim.x) {
    float scale;
    codes[g] = halo::QuantQuad(row[g], scale);
    if (g % 8 == 0) xd[t * (cols / 32) + g / 8] = scale;
  }
}

// halo_quantize_q8_rows over 8 rows per block (grid ceil(T / 8)): the block's rows are one flat run of 16-byte
// groups, so short rows (the MoE's 512-wide h) keep every lane busy and each lane has several loads in flight.
// Q8_0 blocks and 8-lane groups line up as in the one-row form (cols % 32 == 0), so the codes are bitwise equal.
extern "C" __global__ void __launch_bounds__(256)
    halo_quantize_q8_rows8(const float* x, std::int8_t* xq, float* xd, std::uint32_t cols, std::uint32_t T) {
  const std::size_t t0 = static_cast<std::size_t>(blockIdx.x) * 8;
  const std::size_t rows = min(static_cast<std::size_t>(8), T - t0), n4 = rows * (cols / 4);
  const float4* src = reinterpret_cast<const float4*>(x + t0 * cols);
  std::uint32_t* codes = reinterpret_cast<std::uint32_t*>(xq + t0 * cols);
  float* scales = xd + t0 * (cols / 32);
  for (std::size_t g = threadIdx.x; g < n4; g += blockDim.x) {
    float scale;
    codes[g] = halo::QuantQuad(src[g], scale);
    if (g % 8 == 0) scales[g / 8] = scale;
  }
}

// reference src/kernels/batch_decode.hip:201-222. Grid (ceil(cols / 256), B), 256 threads: x column b at
// x + b * xstride -> xq + b * cols, xs + b * cols / 32; with xq2 the residual x - q * s (product rounded before the
// subtraction) is quantized again into xq2 / xs2. The block's 256 values go to its first wave, 4 values per lane
// (16-byte loads when the column is aligned), 8 lanes per Q8_0 block (QuantQuad); codes are stored a word per lane.
extern "C" __global__ void __launch_bounds__(256)
    halo_q8x_cols(const float* x, std::uint32_t xstride, std::uint32_t cols, std::int8_t* xq, float* xs,
                  std::int8_t* xq2, float* xs2) {
  if (threadIdx.x >= kWave) return;
  const std::size_t b = blockIdx.y;
  const std::uint32_t nblk = cols / 32, c = blockIdx.x * 256 + threadIdx.x * 4;
  if (c >= cols) return;  // groups of 8 lanes leave together (cols % 32 == 0)
  const float* src = x + b * xstride + c;
  float4 v;
  if ((reinterpret_cast<std::uintptr_t>(src) & 15u) == 0) {
    v = *reinterpret_cast<const float4*>(src);
  } else {
    v = make_float4(src[0], src[1], src[2], src[3]);
  }
  float s1;
  const std::uint32_t w1 = halo::QuantQuad(v, s1);
  *reinterpret_cast<std::uint32_t*>(xq + b * cols + c) = w1;
  const bool lead = threadIdx.x % 8 == 0;
  if (lead) xs[b * nblk + c / 32] = s1;
  if (!xq2) return;
  float4 r;
  {
#pragma clang fp contract(off)
    r.x = v.x - static_cast<float>(static_cast<std::int8_t>(w1)) * s1;
    r.y = v.y - static_cast<float>(static_cast<std::int8_t>(w1 >> 8)) * s1;
    r.z = v.z - static_cast<float>(static_cast<std::int8_t>(w1 >> 16)) * s1;
    r.w = v.w - static_cast<float>(static_cast<std::int8_t>(w1 >> 24)) * s1;
  }
  float s2;
  *reinterpret_cast<std::uint32_t*>(xq2 + b * cols + c) = halo::QuantQuad(r, s2);
  if (lead) xs2[b * nblk + c / 32] = s2;
}

// ---- int8-activation GEMV ------------------------------------------------------------------------------------
namespace {

constexpr int kInFlight = 4;  // column steps whose loads are issued before their arithmetic

// Rows r(k) = base + k * P + lane / LPR (P = 64 / LPR), columns [k0, k1) of NB activation columns. Returns the
// per-row sums reduced over the LPR lanes (valid in every lane).
template <int LPR, int R, int NB, bool kResid, bool kNT = false>
__device__ __forceinline__ void Q8A8Rows(const std::int8_t* __restrict__ qs, const std::uint16_t* __restrict__ d,
                                         const std::int8_t* __restrict__ xq, const float* __restrict__ xs,
                                         const std::int8_t* __restrict__ xq2, const float* __restrict__ xs2,
                                         std::uint32_t base, std::uint32_t rows, std::uint32_t cols,
                                         std::uint32_t qstride, std::uint32_t k0, std::uint32_t k1,
                                         float (&out)[NB][R]) {
  constexpr int P = kWave / LPR;
  constexpr std::uint32_t kStep = LPR * 16;
  const std::uint32_t lane = threadIdx.x % kWave, nblk = cols / 32;
  const std::uint32_t sub = lane / LPR;
  const std::int8_t* rowp[R];
  const std::uint16_t* dp[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const std::uint32_t r = min(base + k * P + sub, rows - 1);
    rowp[k] = qs + static_cast<std::size_t>(r) * qstride;
    dp[k] = d + static_cast<std::size_t>(r) * nblk;
  }
  float acc[NB][R];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int k = 0; k < R; ++k) acc[b][k] = 0.0f;

  for (std::uint32_t c0 = k0 + (lane % LPR) * 16; c0 < k1; c0 += kInFlight * kStep) {
    int4 q[kInFlight][R];
    float s[kInFlight][R];
    int4 xv[kInFlight][NB];
    float sx[kInFlight][NB];
    int4 rv[kInFlight][kResid ? NB : 1];
    float sr[kInFlight][kResid ? NB : 1];
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) {
      const std::uint32_t c = c0 + u * kStep;
      const bool ok = c < k1;
      const std::uint32_t cc = ok ? c : k0 + (lane % LPR) * 16;
#pragma unroll
      for (int k = 0; k < R; ++k) {
        if constexpr (kNT)
          q[u][k] = __builtin_bit_cast(int4, __builtin_nontemporal_load(reinterpret_cast<const halo::V4i*>(rowp[k] + cc)));
        else
          q[u][k] = *reinterpret_cast<const int4*>(rowp[k] + cc);
        const float sv = F16(dp[k][cc / 32]);  // unconditional: a load under a branch costs a vmcnt(0) wait
        s[u][k] = ok ? sv : 0.0f;
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        xv[u][b] = *reinterpret_cast<const int4*>(xq + static_cast<std::size_t>(b) * cols + cc);
        sx[u][b] = xs[static_cast<std::size_t>(b) * nblk + cc / 32];
        if constexpr (kResid) {
          rv[u][b] = *reinterpret_cast<const int4*>(xq2 + static_cast<std::size_t>(b) * cols + cc);
          sr[u][b] = xs2[static_cast<std::size_t>(b) * nblk + cc / 32];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kInFlight; ++u)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int k = 0; k < R; ++k) {
          float part = sx[u][b] * static_cast<float>(Dot16(q[u][k], xv[u][b]));
          if constexpr (kResid) part += sr[u][b] * static_cast<float>(Dot16(q[u][k], rv[u][b]));
          acc[b][k] += s[u][k] * part;
        }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int k = 0; k < R; ++k) out[b][k] = halo::GroupSum<LPR>(acc[b][k]);
}

template <int LPR, int R, int NB, bool kResid>
__device__ __forceinline__ void StoreRows(float* y, std::uint32_t ystride, std::uint32_t base, std::uint32_t rows,
                                         const float (&out)[NB][R]) {
  constexpr int P = kWave / LPR;
  const std::uint32_t lane = threadIdx.x % kWave;
  if (lane % LPR != 0) return;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const std::uint32_t r = base + k * P + lane / LPR;
    if (r < rows)
#pragma unroll
      for (int b = 0; b < NB; ++b) y[static_cast<std::size_t>(b) * ystride + r] = out[b][k];
  }
}

// Reference-convention batched int8 GEMV (src/kernels/batch_decode.hip:273-298): a 256-thread block covers 8 * R
// rows (4 waves x 2 rows per pass x R), blockIdx.x = row block * groups + column group, blockIdx.y = split-K part
// over [part * chunk, (part + 1) * chunk) written to y plane part (offset part * rows).
template <int R, int NB, bool kResid>
__device__ __forceinline__ void GemvQ8rI8B(const std::int8_t* qs, const std::uint16_t* d, const std::int8_t* xq,
                                           const float* xs, const std::int8_t* xq2, const float* xs2, float* y,
                                           std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride,
                                           std::uint32_t ystride, std::uint32_t groups, std::uint32_t chunk) {
  const std::uint32_t k0 = blockIdx.y * chunk;
  const std::uint32_t k1 = min(cols, k0 + chunk);
  y += static_cast<std::size_t>(blockIdx.y) * rows;
  const std::uint32_t bx = blockIdx.x / groups, g = blockIdx.x % groups;
  xq += static_cast<std::size_t>(g) * NB * cols;
  xs += static_cast<std::size_t>(g) * NB * (cols / 32);
  if constexpr (kResid) {
    xq2 += static_cast<std::size_t>(g) * NB * cols;
    xs2 += static_cast<std::size_t>(g) * NB * (cols / 32);
  }
  y += static_cast<std::size_t>(g) * NB * ystride;
  const std::uint32_t base = (bx * (blockDim.x / kWave) + threadIdx.x / kWave) * (2 * R);
  if (base >= rows) return;
  float out[NB][R];
  Q8A8Rows<32, R, NB, kResid>(qs, d, xq, xs, xq2, xs2, base, rows, cols, qstride, k0, k1, out);
  StoreRows<32, R, NB, kResid>(y, ystride, base, rows, out);
}

// Two matrices with the same NB columns in one launch (reference batch_decode.hip:310-345): row blocks
// [0, blocks1) take matrix 1, the rest matrix 2; blockIdx.x = row block * groups + column group; no split-K.
template <int R, int NB, bool kResid>
__device__ __forceinline__ void GemvQ8rI8Dual(const std::int8_t* q1, const std::uint16_t* d1, float* y1,
                                              std::uint32_t rows1, std::uint32_t qstride1, const std::int8_t* q2,
                                              const std::uint16_t* d2, float* y2, std::uint32_t rows2,
                                              std::uint32_t qstride2, const std::int8_t* xq, const float* xs,
                                              const std::int8_t* xq2, const float* xs2, std::uint32_t cols,
                                              std::uint32_t blocks1, std::uint32_t ystride1, std::uint32_t ystride2,
                                              std::uint32_t groups) {
  const std::uint32_t bxg = blockIdx.x / groups, g = blockIdx.x % groups;
  xq += static_cast<std::size_t>(g) * NB * cols;
  xs += static_cast<std::size_t>(g) * NB * (cols / 32);
  if constexpr (kResid) {
    xq2 += static_cast<std::size_t>(g) * NB * cols;
    xs2 += static_cast<std::size_t>(g) * NB * (cols / 32);
  }
  const bool first = bxg < blocks1;
  const std::uint32_t bx = first ? bxg : bxg - blocks1, rows = first ? rows1 : rows2;
  const std::uint32_t ystride = first ? ystride1 : ystride2;
  float* y = (first ? y1 : y2) + static_cast<std::size_t>(g) * NB * ystride;
  const std::uint32_t base = (bx * (blockDim.x / kWave) + threadIdx.x / kWave) * (2 * R);
  if (base >= rows) return;
  float out[NB][R];
  Q8A8Rows<32, R, NB, kResid>(first ? q1 : q2, first ? d1 : d2, xq, xs, xq2, xs2, base, rows, cols,
                              first ? qstride1 : qstride2, 0, cols, out);
  StoreRows<32, R, NB, kResid>(y, ystride, base, rows, out);
}

}  // namespace

#define HALO_GEMV_I8_REF(NB, R, SUF, RES)                                                                        \
  extern "C" __global__ void __launch_bounds__(256) halo_gemv_q8r_i8##SUF##_r##R##_b##NB(                       \
      const std::int8_t* qs, const std::uint16_t* d, const std::int8_t* xq, const float* xs,                    \
      const std::int8_t* xq2, const float* xs2, float* y, std::uint32_t rows, std::uint32_t cols,               \
      std::uint32_t qstride, std::uint32_t ystride, std::uint32_t groups, std::uint32_t chunk) {                \
    GemvQ8rI8B<R, NB, RES>(qs, d, xq, xs, xq2, xs2, y, rows, cols, qstride, ystride, groups, chunk);            \
  }
#define HALO_GEMV_I8_DUAL_REF(NB, R, SUF, RES)                                                                   \
  extern "C" __global__ void __launch_bounds__(256) halo_gemv_q8r_i8##SUF##_dual_r##R##_b##NB(                  \
      const std::int8_t* q1, const std::uint16_t* d1, float* y1, std::uint32_t rows1, std::uint32_t qstride1,   \
      const std::int8_t* q2, const std::uint16_t* d2, float* y2, std::uint32_t rows2, std::uint32_t qstride2,   \
      const std::int8_t* xq, const float* xs, const std::int8_t* xq2, const float* xs2, std::uint32_t cols,     \
      std::uint32_t blocks1, std::uint32_t ystride1, std::uint32_t ystride2, std::uint32_t groups) {            \
    GemvQ8rI8Dual<R, NB, RES>(q1, d1, y1, rows1, qstride1, q2, d2, y2, rows2, qstride2, xq, xs, xq2, xs2, cols,  \
                              blocks1, ystride1, ystride2, groups);                                              \
  }
#define HALO_GEMV_I8_REF_NB(NB)                                                                                   \
  HALO_GEMV_I8_REF(NB, 1, , false) HALO_GEMV_I8_REF(NB, 2, , false) HALO_GEMV_I8_REF(NB, 4, , false)             \
  HALO_GEMV_I8_REF(NB, 1, x, true) HALO_GEMV_I8_REF(NB, 2, x, true) HALO_GEMV_I8_REF(NB, 4, x, true)             \
  HALO_GEMV_I8_DUAL_REF(NB, 1, , false) HALO_GEMV_I8_DUAL_REF(NB, 2, , false)                                    \
  HALO_GEMV_I8_DUAL_REF(NB, 4, , false) HALO_GEMV_I8_DUAL_REF(NB, 1, x, true)                                    \
  HALO_GEMV_I8_DUAL_REF(NB, 2, x, true) HALO_GEMV_I8_DUAL_REF(NB, 4, x, true)
HALO_GEMV_I8_REF_NB(1)
HALO_GEMV_I8_REF_NB(2)
HALO_GEMV_I8_REF_NB(3)
HALO_GEMV_I8_REF_NB(4)
HALO_GEMV_I8_REF_NB(5)
HALO_GEMV_I8_REF_NB(6)
HALO_GEMV_I8_REF_NB(7)
HALO_GEMV_I8_REF_NB(8)
#undef HALO_GEMV_I8_REF_NB
#undef HALO_GEMV_I8_DUAL_REF
#undef HALO_GEMV_I8_REF

// MI355X-native int8-activation GEMV (new name, no reference counterpart): blockDim.x / 64 waves per block, each
// wave owns R * 64 / LPR consecutive-pass rows; grid.x = ceil(rows / (waves * R * 64 / LPR)). No split-K: the
// dispatcher picks LPR and the block size so that the grid has >= 4 waves per CU.
//   y[b * ystride + r] = sum over 32-blocks of d[r] * xs[b] * isum, b < NB.
#define HALO_GEMV_Q8A8(LPR, R, NB)                                                                                \
  extern "C" __global__ void __launch_bounds__(256) halo_gemv_q8a8_l##LPR##_r##R##_b##NB(                       \
      const std::int8_t* qs, const std::uint16_t* d, const std::int8_t* xq, const float* xs, float* y,          \
      std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride, std::uint32_t ystride) {                   \
    constexpr std::uint32_t kRowsPerWave = R * (kWave / LPR);                                                   \
    const std::uint32_t base = (blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave) * kRowsPerWave;       \
    if (base >= rows) return;                                                                                    \
    float out[NB][R];                                                                                            \
    Q8A8Rows<LPR, R, NB, false, true>(qs, d, xq, xs, nullptr, nullptr, base, rows, cols, qstride, 0, cols, out); \
    StoreRows<LPR, R, NB, false>(y, ystride, base, rows, out);                                                  \
  }
#define HALO_GEMV_Q8A8_R(LPR, NB) HALO_GEMV_Q8A8(LPR, 1, NB) HALO_GEMV_Q8A8(LPR, 2, NB) HALO_GEMV_Q8A8(LPR, 4, NB)
#define HALO_GEMV_Q8A8_NB(LPR) \
  HALO_GEMV_Q8A8_R(LPR, 1) HALO_GEMV_Q8A8_R(LPR, 2) HALO_GEMV_Q8A8_R(LPR, 4) HALO_GEMV_Q8A8_R(LPR, 8)
HALO_GEMV_Q8A8_NB(64)
HALO_GEMV_Q8A8_NB(32)
HALO_GEMV_Q8A8_NB(16)
#undef HALO_GEMV_Q8A8_NB
#undef HALO_GEMV_Q8A8_R
#undef HALO_GEMV_Q8A8

// Variant with non-temporal weight loads (streamed once; kept out of the caches' reuse sets).
extern "C" __global__ void __launch_bounds__(256) halo_gemv_q8a8nt_l64_r1_b1(
    const std::int8_t* qs, const std::uint16_t* d, const std::int8_t* xq, const float* xs, float* y,
    std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride, std::uint32_t ystride) {
  const std::uint32_t base = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (base >= rows) return;
  float out[1][1];
  Q8A8Rows<64, 1, 1, false, true>(qs, d, xq, xs, nullptr, nullptr, base, rows, cols, qstride, 0, cols, out);
  StoreRows<64, 1, 1, false>(y, ystride, base, rows, out);
}

// Exact integer half-block dots for parity checks: isum[r][c / 16] = sum of 16 int8 products, computed by the
// same 16-byte loads and v_dot4 chain as the GEMV. Grid-stride over (row, 16-column piece).
extern "C" __global__ void __launch_bounds__(256)
    halo_q8_half_dots(const std::int8_t* qs, const std::int8_t* xq, std::int32_t* isum, std::uint32_t rows,
                      std::uint32_t cols, std::uint32_t qstride) {
  const std::uint32_t pieces = cols / 16;
  const std::uint64_t total = static_cast<std::uint64_t>(rows) * pieces;
  for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x) {
    const std::uint64_t r = i / pieces, p = i % pieces;
    const int4 q = *reinterpret_cast<const int4*>(qs + r * qstride + p * 16);
    const int4 x = *reinterpret_cast<const int4*>(xq + p * 16);
    isum[i] = Dot16(q, x);
  }
}

// ---- fp32-activation GEMV (reference names) -----------------------------------------------------------------
// reference src/kernels/core.hip:2147-2188, 2388-2443: y[r] = sum_b F16(d) * sum_i q * x with fp32 x. Wave64: a
// 256-thread block covers the reference's rows per block (8 * R); x is read through the vector cache.
namespace {
// Row block bx of 8 R rows (4 waves x 2 rows per pass x R).
// One lane's 16-value piece of an fp32-activation Q8_0 dot: sum over i of q[i] * x[i] as one fused chain in index
// order. The single-column and batched kernels both use it, so a column's bits do not depend on the batch.
__device__ __forceinline__ float Q8PieceF32(const int4& q, const float (&xr)[16]) {
  const std::int8_t* v = reinterpret_cast<const std::int8_t*>(&q);
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) part = __builtin_fmaf(static_cast<float>(v[i]), xr[i], part);
  return part;
}
__device__ __forceinline__ void LoadX16(const float* x, float (&xr)[16]) {
  const float4* xp = reinterpret_cast<const float4*>(x);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 v = xp[i];
    xr[4 * i] = v.x;
    xr[4 * i + 1] = v.y;
    xr[4 * i + 2] = v.z;
    xr[4 * i + 3] = v.w;
  }
}

// fp32-activation Q8_0 GEMV over NB columns (NB = 1: the single-column kernels): a 32-lane half wave per row, two
// rows per wave per pass, R passes (8 R rows per block of 256); each lane's 16-value pieces of a row at stride
// 32 * 16 columns, x read through the vector cache (no LDS copy, so no column limit). The weights of a piece are
// loaded once for all NB columns; each column's arithmetic (Q8PieceF32, acc = fma(scale, piece, acc) in column
// order, GroupSum<32>) is the single-column kernel's, so every column equals a single-column launch bit for bit.
// Column b reads x + b * xstride and writes y + b * ystride.
template <int R, int NB>
__device__ __forceinline__ void GemvQ8rF32At(const std::int8_t* __restrict__ qs, const std::uint16_t* __restrict__ d,
                                             const float* __restrict__ x, std::uint32_t xstride, float* __restrict__ y,
                                             std::uint32_t ystride, std::uint32_t rows, std::uint32_t cols,
                                             std::uint32_t qstride, std::uint32_t bx) {
  constexpr int LPR = 32, P = 2;
  const std::uint32_t base = (bx * (blockDim.x / kWave) + threadIdx.x / kWave) * (P * R);
  if (base >= rows) return;
  const std::uint32_t lane = threadIdx.x % kWave, nblk = cols / 32, sub = lane / LPR;
  float acc[NB][R];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int k = 0; k < R; ++k) acc[b][k] = 0.0f;
  for (std::uint32_t c = (lane % LPR) * 16; c < cols; c += LPR * 16) {
    int4 q[R];
    float s[R];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const std::uint32_t r = min(base + k * P + sub, rows - 1);
      q[k] = *reinterpret_cast<const int4*>(qs + static_cast<std::size_t>(r) * qstride + c);
      s[k] = F16(d[static_cast<std::size_t>(r) * nblk + c / 32]);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float xr[16];
      LoadX16(x + static_cast<std::size_t>(b) * xstride + c, xr);
#pragma unroll
      for (int k = 0; k < R; ++k) acc[b][k] = __builtin_fmaf(s[k], Q8PieceF32(q[k], xr), acc[b][k]);
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const float a = halo::GroupSum<LPR>(acc[b][k]);
      const std::uint32_t r = base + k * P + sub;
      if (lane % LPR == 0 && r < rows) y[static_cast<std::size_t>(b) * ystride + r] = a;
    }
}
template <int R>
__device__ __forceinline__ void GemvQ8rF32At(const std::int8_t* __restrict__ qs, const std::uint16_t* __restrict__ d,
                                             const float* __restrict__ x, float* __restrict__ y, std::uint32_t rows,
                                             std::uint32_t cols, std::uint32_t qstride, std::uint32_t bx) {
  GemvQ8rF32At<R, 1>(qs, d, x, 0, y, 0, rows, cols, qstride, bx);
}
template <int R>
__device__ __forceinline__ void GemvQ8rF32(const std::int8_t* __restrict__ qs, const std::uint16_t* __restrict__ d,
                                           const float* __restrict__ x, float* __restrict__ y, std::uint32_t rows,
                                           std::uint32_t cols, std::uint32_t qstride) {
  GemvQ8rF32At<R>(qs, d, x, y, rows, cols, qstride, blockIdx.x);
}
}  // namespace

extern "C" __global__ void __launch_bounds__(256)
    halo_gemv_q8r(const std::int8_t* qs, const std::uint16_t* d, const float* x, float* y, std::uint32_t rows,
                  std::uint32_t cols, std::uint32_t qstride) {
  GemvQ8rF32<1>(qs, d, x, y, rows, cols, qstride);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_gemv_q8r_r2(const std::int8_t* qs, const std::uint16_t* d, const float* x, float* y, std::uint32_t rows,
                     std::uint32_t cols, std::uint32_t qstride) {
  GemvQ8rF32<2>(qs, d, x, y, rows, cols, qstride);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_gemv_q8r_r4(const std::int8_t* qs, const std::uint16_t* d, const float* x, float* y, std::uint32_t rows,
                     std::uint32_t cols, std::uint32_t qstride) {
  GemvQ8rF32<4>(qs, d, x, y, rows, cols, qstride);
}

// ---- exact batched fp32-activation GEMVs (reference src/kernels/batch_decode.hip:133-190) ----------------------
// NB = 1..8 columns per launch, each byte-identical to halo_gemv_q8r_r4 / _r2 / halo_gemv_q8r_dual of that column
// alone. Grid as the reference launches them: blockIdx.x = row block * groups + column group (column group g covers
// columns g NB .. g NB + NB - 1), 8 R rows per block of 256 (dual: 32 rows, blocks [0, blocks1) matrix 1). The
// reference's _p (prefetch) / _s (small LDS) / _ps variants exist for its LDS staging of x; this body reads x
// through the vector cache, so the four names share it.
#define HALO_GEMV_Q8R_B(R, NB, SUF)                                                                                 \
  extern "C" __global__ void __launch_bounds__(256) halo_gemv_q8r_r##R##_b##NB##SUF(                               \
      const std::int8_t* qs, const std::uint16_t* d, const float* x, float* y, std::uint32_t rows,                 \
      std::uint32_t cols, std::uint32_t qstride, std::uint32_t xstride, std::uint32_t ystride,                     \
      std::uint32_t groups) {                                                                                       \
    const std::uint32_t g = blockIdx.x % groups;                                                                    \
    GemvQ8rF32At<R, NB>(qs, d, x + static_cast<std::size_t>(g) * NB * xstride, xstride,                            \
                        y + static_cast<std::size_t>(g) * NB * ystride, ystride, rows, cols, qstride,               \
                        blockIdx.x / groups);                                                                       \
  }
#define HALO_GEMV_Q8R_DUAL_B(NB, SUF)                                                                               \
  extern "C" __global__ void __launch_bounds__(256) halo_gemv_q8r_dual_b##NB##SUF(                                \
      const std::int8_t* q1, const std::uint16_t* d1, float* y1, std::uint32_t rows1, std::uint32_t qstride1,      \
      const std::int8_t* q2, const std::uint16_t* d2, float* y2, std::uint32_t rows2, std::uint32_t qstride2,      \
      const float* x, std::uint32_t cols, std::uint32_t blocks1, std::uint32_t xstride, std::uint32_t ystride1,    \
      std::uint32_t ystride2, std::uint32_t groups) {                                                               \
    const std::uint32_t bx = blockIdx.x / groups, g = blockIdx.x % groups;                                          \
    const bool first = bx < blocks1;                                                                                \
    const std::uint32_t ys = first ? ystride1 : ystride2;                                                           \
    GemvQ8rF32At<4, NB>(first ? q1 : q2, first ? d1 : d2, x + static_cast<std::size_t>(g) * NB * xstride, xstride,  \
                        (first ? y1 : y2) + static_cast<std::size_t>(g) * NB * ys, ys, first ? rows1 : rows2, cols, \
                        first ? qstride1 : qstride2, first ? bx : bx - blocks1);                                    \
  }
#define HALO_GEMV_Q8R_B_ALL(NB)                                                                                     \
  HALO_GEMV_Q8R_B(4, NB, ) HALO_GEMV_Q8R_B(4, NB, _p) HALO_GEMV_Q8R_B(4, NB, _s) HALO_GEMV_Q8R_B(4, NB, _ps)         \
  HALO_GEMV_Q8R_B(2, NB, ) HALO_GEMV_Q8R_B(2, NB, _p) HALO_GEMV_Q8R_B(2, NB, _s) HALO_GEMV_Q8R_B(2, NB, _ps)         \
  HALO_GEMV_Q8R_DUAL_B(NB, ) HALO_GEMV_Q8R_DUAL_B(NB, _p) HALO_GEMV_Q8R_DUAL_B(NB, _s) HALO_GEMV_Q8R_DUAL_B(NB, _ps)
HALO_GEMV_Q8R_B_ALL(1)
HALO_GEMV_Q8R_B_ALL(2)
HALO_GEMV_Q8R_B_ALL(3)
HALO_GEMV_Q8R_B_ALL(4)
HALO_GEMV_Q8R_B_ALL(5)
HALO_GEMV_Q8R_B_ALL(6)
HALO_GEMV_Q8R_B_ALL(7)
HALO_GEMV_Q8R_B_ALL(8)
#undef HALO_GEMV_Q8R_B_ALL
#undef HALO_GEMV_Q8R_DUAL_B
#undef HALO_GEMV_Q8R_B

// ---- synthetic tensors ------------------------------------------------------------------------------------------
// Seeded Q8_0 weights generated in place (no host copy of multi-GB models): q uniform in [-127, 127] from a
// counter hash of (seed, row, column), d = fp16(|N(0, sigma)| / 127) from a hash of (seed, row, block).
extern "C" __global__ void __launch_bounds__(256)
    halo_synth_q8(std::int8_t* qs, std::uint16_t* d, std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride,
                  std::uint64_t seed, float sigma) {
  const std::uint32_t pieces = cols / 16, nblk = cols / 32;
  const std::uint64_t total = static_cast<std::uint64_t>(rows) * pieces;
  for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x) {
    const std::uint64_t r = i / pieces, p = i % pieces;
    const std::uint64_t key = halo::Mix64(seed ^ (r * 0x100000001B3ull)) + p;
    int w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const std::uint64_t h = halo::Mix64(key * 4 + j);
      std::uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int v = static_cast<int>(((h >> (16 * b)) & 0xFFFF) % 255u) - 127;
        word |= (static_cast<std::uint32_t>(v) & 0xFFu) << (8 * b);
      }
      w[j] = static_cast<int>(word);
    }
    *reinterpret_cast<int4*>(qs + r * qstride + p * 16) = make_int4(w[0], w[1], w[2], w[3]);
    if (p % 2 == 0) {
      const float n = halo::Normal(halo::Mix64(seed + 0x5851F42D4C957F2Dull) ^ (r * nblk + p / 2));
      d[r * nblk + p / 2] = halo::ToF16Bits(fabsf(n) * sigma / 127.0f);
    }
  }
}

// fp32 N(0, sigma) or bf16 tensors from a counter hash.
extern "C" __global__ void __launch_bounds__(256)
    halo_synth_f32(float* x, std::uint64_t n, std::uint64_t seed, float sigma) {
  for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x)
    x[i] = sigma * halo::Normal(halo::Mix64(seed) ^ i);
}

// ---- bandwidth references ----------------------------------------------------------------------------------
// Plain streaming read and copy of n 16-byte vectors, the yardsticks the GEMV is compared against (and the
// calibration kernels for hardware byte counters). Each lane handles kPer vectors spaced a grid apart.
extern "C" __global__ void __launch_bounds__(256)
    halo_stream_read(const int4* __restrict__ src, std::uint64_t n, int* __restrict__ sink) {
  constexpr int kPer = 4;
  const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
  const std::uint64_t i0 = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x;
  int acc = 0;
  for (std::uint64_t base = i0; base < n; base += kPer * stride) {
    int4 v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const std::uint64_t i = base + u * stride;
      v[u] = i < n ? src[i] : make_int4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x7F3A5C11) sink[0] = acc;  // keeps the loads; practically never taken
}

// grid (1), block 64: out[slot] = the device's constant wall clock (wall_clock64, halo_wall_clock_khz ticks per ms).
// Graph nodes at the start and end of a timed region of back-to-back launches bracket it on the device itself.
extern "C" __global__ void __launch_bounds__(64) halo_clock_stamp(std::uint64_t* __restrict__ out, std::uint32_t slot) {
  if (threadIdx.x == 0) out[slot] = wall_clock64();
}

extern "C" __global__ void __launch_bounds__(256)
    halo_stream_copy(const int4* __restrict__ src, int4* __restrict__ dst, std::uint64_t n) {
  const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
  for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < n; i += stride)
    dst[i] = src[i];
}

// ---- int8 MFMA tiles for M >= 16 tokens (prefill, speculative verify) ----------------------------------------
// reference: halo_gemm_q8r_wmma / GemmQ8A8 (src/kernels/core.hip:3108-3153, 3344-3476): per 32-value block an
// integer product into int32, then the fp32 epilogue acc += d_w * (s_x * isum). Here one v_mfma_i32_16x16x32_i8 per
// (16 rows, 16 tokens, one Q8_0 block): A = 16 weight rows x 32 int8 (lane l: row l % 16, k 8 (l / 16) .. +8),
// B = 32 x 16 tokens (lane l: token l % 16, same k), D (lane l: token l % 16, rows 4 (l / 16) .. +4).
// A block of 4 waves owns 16 rows x 16 * NT tokens; the waves split the K blocks four ways and reduce through LDS
// (fixed order). grid (ceil(rows / 16), ceil(T / (16 NT))), block 256. y[t * ystride + r].
namespace {
typedef int V4I32 __attribute__((ext_vector_type(4)));

template <int NT>
__device__ __forceinline__ void GemmQ8A8Mfma(const std::int8_t* __restrict__ qs, const std::uint16_t* __restrict__ d,
                                             const std::int8_t* __restrict__ xq, const float* __restrict__ xs,
                                             float* __restrict__ y, std::uint32_t rows, std::uint32_t cols,
                                             std::uint32_t qstride, std::uint32_t T, std::uint32_t ystride) {
  __shared__ float red[4][NT][16][17];
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const std::uint32_t r0 = blockIdx.x * 16, t0 = blockIdx.y * 16 * NT;
  const std::uint32_t nblk = cols / 32;
  const std::uint32_t arow = min(r0 + lane % 16, rows - 1);
  const std::uint32_t kofs = (lane / 16) * 8;
  const std::int8_t* aptr = qs + static_cast<std::size_t>(arow) * qstride + kofs;
  const std::int8_t* bptr[NT];
  const float* sptr[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const std::uint32_t tok = min(t0 + n * 16 + lane % 16, T - 1);
    bptr[n] = xq + static_cast<std::size_t>(tok) * cols + kofs;
    sptr[n] = xs + static_cast<std::size_t>(tok) * nblk;
  }
  const std::uint16_t* dptr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    dptr[i] = d + static_cast<std::size_t>(min(r0 + (lane / 16) * 4 + i, rows - 1)) * nblk;
  float acc[NT][4];
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[n][i] = 0.0f;
  const std::uint32_t per = (nblk + 3) / 4, kb0 = wave * per, kb1 = min(nblk, kb0 + per);
  constexpr int U = 4;
  for (std::uint32_t kb = kb0; kb < kb1; kb += U) {
    long a[U];
    long b[U][NT];
    float dw[U][4], sx[U][NT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const std::uint32_t k = min(kb + u, kb1 - 1);
      a[u] = *reinterpret_cast<const long*>(aptr + k * 32);
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        b[u][n] = *reinterpret_cast<const long*>(bptr[n] + k * 32);
        sx[u][n] = sptr[n][k];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) dw[u][i] = F16(dptr[i][k]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (kb + u >= kb1) break;
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const V4I32 zero = {0, 0, 0, 0};
        const V4I32 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[u], b[u][n], zero, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[n][i] += dw[u][i] * (sx[u][n] * static_cast<float>(c[i]));
      }
    }
  }
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][n][(lane / 16) * 4 + i][lane % 16] = acc[n][i];
  __syncthreads();
  for (std::uint32_t e = threadIdx.x; e < NT * 256; e += blockDim.x) {
    const std::uint32_t n = e / 256, rr = (e % 256) / 16, tt = e % 16;
    const std::uint32_t r = r0 + rr, tok = t0 + n * 16 + tt;
    if (r < rows && tok < T)
      y[static_cast<std::size_t>(tok) * ystride + r] =
          ((red[0][n][rr][tt] + red[1][n][rr][tt]) + red[2][n][rr][tt]) + red[3][n][rr][tt];
  }
}
}  // namespace

extern "C" __global__ void __launch_bounds__(256) halo_gemm_q8a8_mfma_t1(
    const std::int8_t* qs, const std::uint16_t* d, const std::int8_t* xq, const float* xs, float* y, std::uint32_t rows,
    std::uint32_t cols, std::uint32_t qstride, std::uint32_t T, std::uint32_t ystride) {
  GemmQ8A8Mfma<1>(qs, d, xq, xs, y, rows, cols, qstride, T, ystride);
}
extern "C" __global__ void __launch_bounds__(256) halo_gemm_q8a8_mfma_t4(
    const std::int8_t* qs, const std::uint16_t* d, const std::int8_t* xq, const float* xs, float* y, std::uint32_t rows,
    std::uint32_t cols, std::uint32_t qstride, std::uint32_t T, std::uint32_t ystride) {
  GemmQ8A8Mfma<4>(qs, d, xq, xs, y, rows, cols, qstride, T, ystride);
}

// ---- tiled int8 MFMA GEMM for prefill-sized M (dense projections and the grouped MoE experts) --------------------
// The same arithmetic per Q8_0 block as above (an exact int32 block product scaled by d_w s_x and accumulated in fp32,
// blocks in ascending order), on v_mfma_i32_32x32x32_i8: one MFMA is one Q8_0 block of a 32-row x 32-token tile. The
// per-output scales d_w[r] s_x[t] of a tile come from a rank-1 fp32 MFMA in the same layout (k = 0 carries the
// factors, k = 1 zeros), so the VALU epilogue is acc = fma(float(isum), d_w s_x, acc).
// A block of 8 waves, WR x WT, owns ROWS = WR * MT * 32 weight rows x TOKS = WT * 32 tokens of one or two matrices
// (NMAT = 2: gate and up, combined as SiLU(gate) * up); wave (wr, wt) computes MT row tiles x one token tile. K
// advances 64 columns (two Q8_0 blocks) per stage. Each stage's weight and activation tiles (int8, rows padded to
// 80 bytes so the 16-byte fragment reads are conflict-free) and their scales are staged in LDS, double buffered;
// the loads of stage k + 2 are in flight in registers while stage k computes and stage k + 1 is stored.
// MFMA operands: lane l supplies 16 int8 of row (l % 32) at k 16 (l / 32) of the block, the same k split for both
// operands; the int32 result lane l holds token (l % 32) of the tile and rows 8 (j / 4) + 4 (l / 32) + j % 4.
// Tokens: tile token i reads activation row xrow[min(i, ntok - 1)] (or x0 + min(i, ntok - 1)) and, for i < ntok,
// writes y[(yrow0 + i) * ystride + r]. Matrices are [rows][qstride] int8 + [rows][cols / 32] fp16 scales; block row
// tile r0. Requires cols % 64 == 0.
namespace {
typedef int V16I32 __attribute__((ext_vector_type(16)));
typedef float V16F32 __attribute__((ext_vector_type(16)));
typedef float V32F32 __attribute__((ext_vector_type(32)));
constexpr int kTileLd = 64 + 16;
}  // namespace

namespace halo {
template <int WR, int MT, int WT, int NMAT, bool PAIR = false, bool KBLK = false>
__device__ __forceinline__ void GemmTileQ8(const std::int8_t* __restrict__ A0, const std::uint16_t* __restrict__ D0,
                                          const std::int8_t* __restrict__ A1, const std::uint16_t* __restrict__ D1,
                                          std::uint32_t rows, std::uint32_t qstride, std::uint32_t r0,
                                          const std::int8_t* __restrict__ xq, const float* __restrict__ xs,
                                          const std::uint32_t* __restrict__ xrow, std::uint32_t x0, std::uint32_t ntok,
                                          std::uint32_t cols, float* __restrict__ y, std::uint32_t yrow0,
                                          std::uint32_t ystride, std::uint32_t xtok = 0) {
  static_assert(WR * WT == 2 || WR * WT == 4 || WR * WT == 8, "2, 4 or 8 waves");
  constexpr std::uint32_t NTH = WR * WT * 64;  // the block size
  // activation layout: token rows [T][cols] int8 + [T][cols / 32] scales, or K-blocked (KBLK) [cols / 64][xtok][64]
  // int8 + [cols / 32][xtok] scales (halo_quantize_q8_kblocked)
  const std::size_t xstage = KBLK ? 64 * static_cast<std::size_t>(xtok) : 64;
  const std::size_t sstage = KBLK ? 2 * static_cast<std::size_t>(xtok) : 2;
  constexpr int ROWS = WR * MT * 32, TOKS = WT * 32;
  constexpr int NA = NMAT * ROWS * 4, NB = TOKS * 4;  // 16-byte chunks per stage
  constexpr int NDW = NMAT * ROWS * 2, NSX = TOKS * 2;  // scales per stage
  constexpr int LA = (NA + NTH - 1) / NTH, LB = (NB + NTH - 1) / NTH, LS = (NDW + NSX + NTH - 1) / NTH;
  __shared__ __attribute__((aligned(16))) std::int8_t la[2][NMAT][ROWS][kTileLd];
  __shared__ __attribute__((aligned(16))) std::int8_t lb[2][TOKS][kTileLd];
  __shared__ __attribute__((aligned(16))) float ldw[2][NMAT][2][ROWS];
  __shared__ __attribute__((aligned(16))) float lsx[2][2][TOKS];
  const std::uint32_t tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const std::uint32_t wr = wave / WT, wt = wave % WT;
  const std::uint32_t nblk = cols / 32, nk = cols / 64;
  const auto tokrow = [&](std::uint32_t i) {
    const std::uint32_t ii = min(i, ntok - 1);
    return xrow != nullptr ? xrow[ii] : x0 + ii;
  };
  // per-thread global sources (clamped, so every load is unconditional) and LDS destinations
  const std::int8_t* ga[LA];
  std::uint32_t amat[LA], arow[LA], apart[LA];
  bool aon[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const std::uint32_t c = tid + NTH * i, cc = min(c, static_cast<std::uint32_t>(NA - 1));
    aon[i] = c < static_cast<std::uint32_t>(NA);
    amat[i] = cc / (ROWS * 4);
    arow[i] = (cc / 4) % ROWS;
    apart[i] = cc % 4;
    ga[i] = (amat[i] ? A1 : A0) + static_cast<std::size_t>(min(r0 + arow[i], rows - 1)) * qstride + apart[i] * 16;
  }
  const std::int8_t* gb[LB];
  std::uint32_t brow[LB], bpart[LB];
  bool bon[LB];
#pragma unroll
  for (int i = 0; i < LB; ++i) {
    const std::uint32_t c = tid + NTH * i, cc = min(c, static_cast<std::uint32_t>(NB - 1));
    bon[i] = c < static_cast<std::uint32_t>(NB);
    brow[i] = cc / 4;
    bpart[i] = cc % 4;
    gb[i] = xq + static_cast<std::size_t>(tokrow(brow[i])) * (KBLK ? 64 : cols) + bpart[i] * 16;
  }
  // scales: index c < NDW is (mat, row, blk) of a weight scale, the rest (token, blk) of an activation scale
  const std::uint16_t* gd[LS];
  const float* gs[LS];
  std::uint32_t sidx[LS];
#pragma unroll
  for (int i = 0; i < LS; ++i) {
    const std::uint32_t c = min(tid + NTH * i, static_cast<std::uint32_t>(NDW + NSX - 1));
    sidx[i] = c;
    const std::uint32_t cw = min(c, static_cast<std::uint32_t>(NDW - 1)), cs = c < NDW ? 0u : c - NDW;
    const std::uint32_t m = cw / (ROWS * 2), rr = (cw / 2) % ROWS;
    gd[i] = (m ? D1 : D0) + static_cast<std::size_t>(min(r0 + rr, rows - 1)) * nblk + cw % 2;
    gs[i] = KBLK ? xs + static_cast<std::size_t>(cs % 2) * xtok + tokrow(cs / 2)
                 : xs + static_cast<std::size_t>(tokrow(cs / 2)) * nblk + cs % 2;
  }
  const bool son_last = tid + NTH * (LS - 1) < static_cast<std::uint32_t>(NDW + NSX);
  struct Staged {
    int4 a[LA], b[LB];
    float sc[LS];
  };
  auto load = [&](std::uint32_t kc, Staged& r) {
#pragma unroll
    for (int i = 0; i < LA; ++i)
      r.a[i] = __builtin_bit_cast(int4, __builtin_nontemporal_load(reinterpret_cast<const V4i*>(ga[i] + kc * 64)));
#pragma unroll
    for (int i = 0; i < LB; ++i) r.b[i] = *reinterpret_cast<const int4*>(gb[i] + kc * xstage);
#pragma unroll
    for (int i = 0; i < LS; ++i) {
      const float dv = F16(gd[i][kc * 2]), sv = gs[i][kc * sstage];  // both loaded (clamped addresses), one kept
      r.sc[i] = sidx[i] < static_cast<std::uint32_t>(NDW) ? dv : sv;
    }
  };
  auto store = [&](std::uint32_t st, const Staged& r) {
#pragma unroll
    for (int i = 0; i < LA; ++i)
      if (aon[i]) *reinterpret_cast<int4*>(&la[st][amat[i]][arow[i]][apart[i] * 16]) = r.a[i];
#pragma unroll
    for (int i = 0; i < LB; ++i)
      if (bon[i]) *reinterpret_cast<int4*>(&lb[st][brow[i]][bpart[i] * 16]) = r.b[i];
#pragma unroll
    for (int i = 0; i < LS; ++i) {
      if (i == LS - 1 && !son_last) continue;
      const std::uint32_t c = sidx[i];
      if (c < static_cast<std::uint32_t>(NDW))
        ldw[st][c / (ROWS * 2)][c % 2][(c / 2) % ROWS] = r.sc[i];
      else
        lsx[st][(c - NDW) % 2][(c - NDW) / 2] = r.sc[i];
    }
  };
  float acc[NMAT][MT][16];
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[m][mt][j] = 0.0f;
  const std::uint32_t fr = lane % 32, fk = 16 * (lane / 32);
  // PAIR (one matrix): both Q8_0 blocks of the stage take one two-block rank-1 fp32 MFMA for their scales (block b
  // from lanes 32 b .. 32 b + 31, result registers 16 b .. 16 b + 15), then the int8 MFMAs, then the epilogue in
  // block order. It needs about 200 VGPRs (one block per CU), so it serves grids of at most one block per CU.
  // Otherwise one Q8_0 block at a time, each with its own rank-1 MFMA.
  auto compute = [&](std::uint32_t st) {
    if constexpr (PAIR) {
      static_assert(NMAT == 1, "one matrix");
      const V4i bf0 = *reinterpret_cast<const V4i*>(&lb[st][wt * 32 + fr][fk]);
      const V4i bf1 = *reinterpret_cast<const V4i*>(&lb[st][wt * 32 + fr][32 + fk]);
      const float sx = lsx[st][lane / 32][wt * 32 + fr];
      const V16I32 zero = {};
      const V32F32 fzero = {};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const std::uint32_t rr = wr * MT * 32 + mt * 32 + fr;
        const V4i af0 = *reinterpret_cast<const V4i*>(&la[st][0][rr][fk]);
        const V4i af1 = *reinterpret_cast<const V4i*>(&la[st][0][rr][32 + fk]);
        const float dw = ldw[st][0][lane / 32][rr];
        const V32F32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(dw, sx, fzero, 0, 0, 0);
        const V16I32 c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af0, bf0, zero, 0, 0, 0);
        const V16I32 c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af1, bf1, zero, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[0][mt][j] = __builtin_fmaf(static_cast<float>(c0[j]), sc[j], acc[0][mt][j]);
#pragma unroll
        for (int j = 0; j < 16; ++j)
          acc[0][mt][j] = __builtin_fmaf(static_cast<float>(c1[j]), sc[16 + j], acc[0][mt][j]);
      }
    } else {
#pragma unroll 1
      for (int blk = 0; blk < 2; ++blk) {
        const V4i bf = *reinterpret_cast<const V4i*>(&lb[st][wt * 32 + fr][blk * 32 + fk]);
        const float sx = lsx[st][blk][wt * 32 + fr];
        const float bsx = lane < 32 ? sx : 0.0f;
        const V16I32 zero = {};
        const V16F32 fzero = {};
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const std::uint32_t rr = wr * MT * 32 + mt * 32 + fr;
            const V4i af = *reinterpret_cast<const V4i*>(&la[st][m][rr][blk * 32 + fk]);
            const float dw = ldw[st][m][blk][rr];
            const V16F32 sc = __builtin_amdgcn_mfma_f32_32x32x2f32(lane < 32 ? dw : 0.0f, bsx, fzero, 0, 0, 0);
            const V16I32 c = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, zero, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 16; ++j)
              acc[m][mt][j] = __builtin_fmaf(static_cast<float>(c[j]), sc[j], acc[m][mt][j]);
          }
      }
    }
  };
  // one stage: prefetch kc + 2 into `fill`, compute kc, store kc + 1 (from `next`) into the other buffer, barrier.
  // The other buffer was last read in stage kc - 1, before the barrier that ended it.
  auto stage = [&](std::uint32_t kc, Staged& next, Staged& fill) {
    if (kc + 2 < nk) load(kc + 2, fill);
    compute(kc & 1u);
    if (kc + 1 < nk) store((kc + 1) & 1u, next);
    LdsSync();  // LDS only: the loads of stage kc + 2 stay in flight
  };
  Staged s0, s1;
  load(0, s0);
  if (nk > 1) load(1, s1);
  store(0, s0);
  __syncthreads();
  for (std::uint32_t kc = 0; kc < nk; kc += 2) {
    stage(kc, s1, s0);
    if (kc + 1 < nk) stage(kc + 1, s0, s1);
  }
  const std::uint32_t i = wt * 32 + fr;
  if (i >= ntok) return;
  float* yt = y + static_cast<std::size_t>(yrow0 + i) * ystride;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const std::uint32_t r = r0 + wr * MT * 32 + mt * 32 + g * 8 + (lane / 32) * 4;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = NMAT == 2 ? Silu(acc[0][mt][4 * g + e]) * acc[NMAT - 1][mt][4 * g + e] : acc[0][mt][4 * g + e];
      if (r + 3 < rows && ystride % 4 == 0) {
        *reinterpret_cast<float4*>(yt + r) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (r + e < rows) yt[r + e] = v[e];
      }
    }
}
}  // namespace halo

// ---- the same tiled GEMM with its stages filled by LDS DMA ------------------------------------------------------
// Same arithmetic, operands and block order as GemmTileQ8 (results are bit-identical); the staging differs. Each stage
// (64 columns: two Q8_0 blocks) lands in LDS through global_load_lds (16-byte rows of the weight and activation tiles,
// 4-byte fp16 scale pairs and fp32 scale pairs), issued by the waves in turn with no register staging; three stage
// buffers, the loads of stage k + 2 in flight while stage k computes, so one wait and one barrier per stage.
// Tile rows are 64 bytes with the 16-byte chunk index xor-swizzled by (row >> 2) & 3, which keeps the fragment reads
// (32 consecutive rows, one chunk each) free of bank conflicts. The stage loop is unrolled by three so every LDS
// address is a per-lane constant plus an immediate. The scale MFMA is the two-block rank-1 v_mfma_f32_32x32x1_2b,
// covering two tiles (NMAT * MT even) or both blocks of the stage (a single tile).
// Limits: cols % 64 == 0; every weight offset (rows * qstride) and activation offset fits in 32 bits.
using halo::DmaDword;
using halo::DmaRow16;
using halo::WaitVmem;
namespace {
__device__ __forceinline__ std::uint32_t ChunkSwz(std::uint32_t r) { return (r >> 2) & 3u; }
// An empty asm that reads and writes the 16 values: everything computing them is done before this point.
__device__ __forceinline__ void PinVgprs(float (&a)[16]) {
#pragma unroll
  for (int j = 0; j < 16; ++j) asm volatile("" : "+v"(a[j]));
}
}  // namespace

namespace halo {
template <int WR, int MT, int WT, int NMAT, bool KBLK = false, int PRIO = 0>
__device__ __forceinline__ void GemmTileQ8Dma(const std::int8_t* __restrict__ A0, const std::uint16_t* __restrict__ D0,
                                             const std::int8_t* __restrict__ A1, const std::uint16_t* __restrict__ D1,
                                             std::uint32_t rows, std::uint32_t qstride, std::uint32_t r0,
                                             const std::int8_t* __restrict__ xq, const float* __restrict__ xs,
                                             const std::uint32_t* __restrict__ xrow, std::uint32_t x0,
                                             std::uint32_t ntok, std::uint32_t cols, float* __restrict__ y,
                                             std::uint32_t yrow0, std::uint32_t ystride, std::uint32_t xtok = 0) {
  constexpr int NW = WR * WT, ROWS = WR * MT * 32, TOKS = WT * 32, NT = NMAT * MT;
  static_assert(NT == 1 || MT % 2 == 0 || MT == 1, "scale pairs with a uniform row step");
  constexpr int ABYTES = NMAT * ROWS * 64, BBYTES = TOKS * 64, SD = NMAT * ROWS, SX = 2 * TOKS;
  constexpr int WA = ABYTES / 1024, WB = BBYTES / 1024, WSD = (SD + 63) / 64, WSX = (SX + 63) / 64;
  constexpr int SPR = (WA + WB + NW - 1) / NW, SPS = (WSD + WSX + NW - 1) / NW;  // loads per wave per stage
  constexpr int RB = ABYTES, RS = ABYTES + BBYTES, RX = RS + WSD * 256;  // regions (scale regions whole loads)
  constexpr int STAGE = (RX + WSX * 256 + 1023) / 1024 * 1024;
  static_assert(3 * STAGE <= 65536, "LDS immediates");
  __shared__ __attribute__((aligned(1024))) std::int8_t lds[3 * STAGE];
  const std::uint32_t tid = threadIdx.x, lane = tid % 64;
  const std::uint32_t wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const std::uint32_t wr = wave / WT, wt = wave % WT;
  const std::uint32_t nblk = cols / 32, nk = cols / 64;
  const std::uint32_t lbase = static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>(lds));
  const auto tokrow = [&](std::uint32_t i) {
    const std::uint32_t ii = min(i, ntok - 1);
    return xrow != nullptr ? xrow[ii] : x0 + ii;
  };
  // The wave's loads of a stage, in turn over the waves (the last load repeated where the count is uneven): 16-byte
  // rows of the weight tiles then the activation tile (a wave-uniform base + a per-lane 32-bit offset), and 4-byte
  // scale pairs (per-lane addresses; lanes past a region's end load a clamped address into the region's padding).
  const std::int8_t* rbase[SPR];
  std::uint32_t roff[SPR], rstep[SPR], rlds[SPR];
#pragma unroll
  for (int i = 0; i < SPR; ++i) {
    const std::uint32_t j = min(wave + NW * i, static_cast<std::uint32_t>(WA + WB - 1));
    if (j < WA) {
      const std::uint32_t p = j * 64 + lane, m = j * 64 / (ROWS * 4), pp = p % (ROWS * 4);
      const std::uint32_t r = pp / 4, c = (pp % 4) ^ ChunkSwz(r);
      rbase[i] = m ? A1 : A0;
      roff[i] = min(r0 + r, rows - 1) * qstride + c * 16;
      rstep[i] = 64;
      rlds[i] = j * 1024;
    } else {
      const std::uint32_t jb = j - WA, p = jb * 64 + lane, t = p / 4, c = (p % 4) ^ ChunkSwz(t);
      rbase[i] = xq;
      roff[i] = tokrow(t) * (KBLK ? 64u : cols) + c * 16;
      rstep[i] = KBLK ? 64 * xtok : 64;
      rlds[i] = RB + jb * 1024;
    }
  }
  const char* saddr[SPS];
  std::uint32_t sstep[SPS], slds[SPS];
#pragma unroll
  for (int i = 0; i < SPS; ++i) {
    const std::uint32_t j = min(wave + NW * i, static_cast<std::uint32_t>(WSD + WSX - 1));
    if (j < WSD) {
      const std::uint32_t q = min(j * 64 + lane, static_cast<std::uint32_t>(SD - 1)), m = q / ROWS, r = q % ROWS;
      saddr[i] = reinterpret_cast<const char*>((m ? D1 : D0) + static_cast<std::size_t>(min(r0 + r, rows - 1)) * nblk);
      sstep[i] = 4;
      slds[i] = RS + j * 256;
    } else {
      const std::uint32_t jx = j - WSD, q = min(jx * 64 + lane, static_cast<std::uint32_t>(SX - 1));
      const std::uint32_t t = q / 2, part = q % 2;
      saddr[i] = reinterpret_cast<const char*>(KBLK ? xs + static_cast<std::size_t>(part) * xtok + tokrow(t)
                                                    : xs + static_cast<std::size_t>(tokrow(t)) * nblk + part);
      sstep[i] = KBLK ? 8 * xtok : 8;
      slds[i] = RX + jx * 256;
    }
  }
  const auto issue = [&](std::uint32_t kc, std::uint32_t buf) {
#pragma unroll
    for (int i = 0; i < SPR; ++i) DmaRow16(rbase[i] + static_cast<std::size_t>(kc) * rstep[i], roff[i], lbase + buf * STAGE + rlds[i]);
#pragma unroll
    for (int i = 0; i < SPS; ++i) DmaDword(saddr[i] + static_cast<std::size_t>(kc) * sstep[i], lbase + buf * STAGE + slds[i]);
  };
  float acc[NT][16];
#pragma unroll
  for (int p = 0; p < NT; ++p)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[p][j] = 0.0f;
  const std::uint32_t fr = lane % 32, fh = lane / 32;
  const std::uint32_t tok = wt * 32 + fr, ra = wr * MT * 32 + fr;
  const std::uint32_t a0 = ra * 64 + ((fh ^ ChunkSwz(ra)) * 16), b0 = tok * 64 + ((fh ^ ChunkSwz(tok)) * 16);
  constexpr std::uint32_t kPairStep = NT == 1 ? 2u : (MT % 2 == 0 ? 128u : ROWS * 4u);
  const std::uint32_t dwo = RS + ra * 4 + fh * kPairStep, sxo = RX + tok * 8 + (NT == 1 ? fh * 4 : 0u);
  const auto tile_row_off = [](int p) { return ((p / MT) * ROWS + (p % MT) * 32) * 4; };
  const auto compute = [&](auto bufc) {
    constexpr int BO = decltype(bufc)::value * STAGE;
    const std::int8_t* sb = lds + BO;
    const V16I32 z = {};
    const V32F32 fz = {};
    if constexpr (NT == 1) {
      const float dw = F16(*reinterpret_cast<const std::uint16_t*>(sb + dwo));
      const float sx = *reinterpret_cast<const float*>(sb + sxo);
      const V32F32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(dw, sx, fz, 0, 0, 0);
      const V4i af0 = *reinterpret_cast<const V4i*>(sb + a0), af1 = *reinterpret_cast<const V4i*>(sb + (a0 ^ 32u));
      const V4i bf0 = *reinterpret_cast<const V4i*>(sb + RB + b0);
      const V4i bf1 = *reinterpret_cast<const V4i*>(sb + RB + (b0 ^ 32u));
      const V16I32 c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af0, bf0, z, 0, 0, 0);
      const V16I32 c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af1, bf1, z, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[0][j] = __builtin_fmaf(static_cast<float>(c0[j]), sc[j], acc[0][j]);
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[0][j] = __builtin_fmaf(static_cast<float>(c1[j]), sc[16 + j], acc[0][j]);
    } else {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        __builtin_amdgcn_sched_barrier(0);  // one block's MFMA results live at a time
        const std::uint32_t ao = blk ? a0 ^ 32u : a0, bo = blk ? b0 ^ 32u : b0;
        const V4i bf = *reinterpret_cast<const V4i*>(sb + RB + bo);
        const float sx = *reinterpret_cast<const float*>(sb + sxo + blk * 4);
#pragma unroll
        for (int q = 0; q < NT / 2; ++q) {
          const int p0 = 2 * q, p1 = 2 * q + 1;
          if constexpr (PRIO) {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(PRIO);  // issue this wave's MFMAs ahead of other waves' epilogues
          }
          const float dw = F16(*reinterpret_cast<const std::uint16_t*>(sb + dwo + tile_row_off(p0) + blk * 2));
          const V32F32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(dw, sx, fz, 0, 0, 0);
          const V4i af0 = *reinterpret_cast<const V4i*>(sb + ao + (p0 / MT) * ROWS * 64 + (p0 % MT) * 2048);
          const V4i af1 = *reinterpret_cast<const V4i*>(sb + ao + (p1 / MT) * ROWS * 64 + (p1 % MT) * 2048);
          const V16I32 c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af0, bf, z, 0, 0, 0);
          const V16I32 c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af1, bf, z, 0, 0, 0);
          if constexpr (PRIO) {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
          }
#pragma unroll
          for (int j = 0; j < 16; ++j) acc[p0][j] = __builtin_fmaf(static_cast<float>(c0[j]), sc[j], acc[p0][j]);
#pragma unroll
          for (int j = 0; j < 16; ++j) acc[p1][j] = __builtin_fmaf(static_cast<float>(c1[j]), sc[16 + j], acc[p1][j]);
        }
      }
    }
  };
  // stage kc from buffer B: wait for this wave's loads of stage kc (stage kc + 1's stay in flight), barrier (every
  // wave's loads of kc landed, every wave done with buffer (B + 2) % 3), load stage kc + 2 (clamped: the count per
  // stage stays fixed), compute
  const auto stage = [&](std::uint32_t kc, auto bufc) {
    constexpr std::uint32_t B = decltype(bufc)::value;
    __builtin_amdgcn_sched_barrier(0);  // stages do not interleave: one stage's MFMA results live at a time
    WaitVmem<SPR + SPS>();
    __builtin_amdgcn_s_barrier();
    issue(min(kc + 2, nk - 1), (B + 2) % 3);
    compute(bufc);
#pragma unroll
    for (int p = 0; p < NT; ++p) PinVgprs(acc[p]);  // the stage's epilogue stays in the stage
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  using B2 = std::integral_constant<int, 2>;
  issue(0, 0);
  issue(min(1u, nk - 1), 1);
  std::uint32_t kc = 0;
  for (; kc + 3 <= nk; kc += 3) {
    stage(kc, B0{});
    stage(kc + 1, B1{});
    stage(kc + 2, B2{});
  }
  if (kc < nk) stage(kc++, B0{});
  if (kc < nk) stage(kc++, B1{});
  WaitVmem<0>();  // no DMA may land after the block's LDS is released
  if (tok >= ntok) return;
  float* yt = y + static_cast<std::size_t>(yrow0 + tok) * ystride;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const std::uint32_t r = r0 + wr * MT * 32 + mt * 32 + g * 8 + fh * 4;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = NMAT == 2 ? Silu(acc[mt][4 * g + e]) * acc[MT + mt][4 * g + e] : acc[mt][4 * g + e];
      if (r + 3 < rows && ystride % 4 == 0) {
        *reinterpret_cast<float4*>(yt + r) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (r + e < rows) yt[r + e] = v[e];
      }
    }
}
}  // namespace halo

// Dense: 128 rows x 128 tokens per block (8 waves of 64 rows x 32 tokens), LDS-DMA staged.
// grid (ceil(rows / 128), ceil(T / 128)), block 512. y[t * ystride + r]. rows * qstride < 2^32.
extern "C" __global__ void __launch_bounds__(512) halo_gemm_q8a8_mfma32(
    const std::int8_t* __restrict__ qs, const std::uint16_t* __restrict__ d, const std::int8_t* __restrict__ xq,
    const float* __restrict__ xs, float* __restrict__ y, std::uint32_t rows, std::uint32_t cols,
    std::uint32_t qstride, std::uint32_t T, std::uint32_t ystride) {
  const std::uint32_t t0 = blockIdx.y * 128;
  halo::GemmTileQ8Dma<2, 2, 4, 1, false, 1>(qs, d, nullptr, nullptr, rows, qstride, blockIdx.x * 128, xq, xs, nullptr,
                                            t0, min(128u, T - t0), cols, y, t0, ystride);
}

// The same GEMM on the register-staged tile with paired block scales (the earlier design, kept as a second entry for
// grids of at most one block per CU and as a cross-check: both are bit-identical to the oracle's block order).
extern "C" __global__ void __launch_bounds__(512) halo_gemm_q8a8_mfma32_p(
    const std::int8_t* __restrict__ qs, const std::uint16_t* __restrict__ d, const std::int8_t* __restrict__ xq,
    const float* __restrict__ xs, float* __restrict__ y, std::uint32_t rows, std::uint32_t cols,
    std::uint32_t qstride, std::uint32_t T, std::uint32_t ystride) {
  const std::uint32_t t0 = blockIdx.y * 128;
  halo::GemmTileQ8<2, 2, 4, 1, true>(qs, d, nullptr, nullptr, rows, qstride, blockIdx.x * 128, xq, xs, nullptr, t0,
                                     min(128u, T - t0), cols, y, t0, ystride);
}

// x = a * x + b over n floats (shapes seeded tensors such as norm weights around 1).
extern "C" __global__ void __launch_bounds__(256)
    halo_affine_f32(float* x, std::uint64_t n, float a, float b) {
  for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x)
    x[i] = a * x[i] + b;
}

// dst = src over n bytes (16-byte vectors; n % 16 == 0): session state forks.
extern "C" __global__ void __launch_bounds__(256)
    halo_copy16(const int4* __restrict__ src, int4* __restrict__ dst, std::uint64_t n16) {
  for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < n16;
       i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x)
    dst[i] = src[i];
}

// Zero fill (used instead of memset nodes so that fills can sit in captured graphs).
extern "C" __global__ void __launch_bounds__(256) halo_zero16(int4* __restrict__ dst, std::uint64_t n16) {
  for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < n16;
       i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x)
    dst[i] = make_int4(0, 0, 0, 0);
}

// The batch-1 int8 GEMV with the activation row staged in LDS once per block (one row per wave, 4 waves): the
// block's threads copy xq (16 bytes each) and xs into LDS by DMA before issuing their weight loads, then wait for
// those two loads only (the weights stay in flight) and read the row from LDS: a wave issues 8 vector-memory loads
// instead of 16, and the 4 KB row is read from L2 once per block instead of once per wave. Arithmetic and order are
// those of halo_gemv_q8a8_l64_r1_b1 (bitwise the same y). cols 2048 or 4096, block 256, grid ceil(rows / 4).
// (Copying each wave's row of weight scales by DMA as well, and 8- or 16-wave blocks, measured slower.)
extern "C" __global__ void __launch_bounds__(256) halo_gemv_q8a8s_l64_r1_b1(
    const std::int8_t* __restrict__ qs, const std::uint16_t* __restrict__ d, const std::int8_t* __restrict__ xq,
    const float* __restrict__ xs, float* __restrict__ y, std::uint32_t rows, std::uint32_t cols,
    std::uint32_t qstride, std::uint32_t ystride) {
  __shared__ __attribute__((aligned(16))) std::int8_t xl[4096];
  __shared__ __attribute__((aligned(16))) float sl[128];
  const std::uint32_t tid = threadIdx.x, lane = tid % kWave, nblk = cols / 32;
  const std::uint32_t wv = tid / kWave;
  const std::uint32_t row = blockIdx.x * (blockDim.x / kWave) + wv;
  const std::uint32_t lx = static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>(xl));
  const std::uint32_t ls = static_cast<std::uint32_t>(reinterpret_cast<std::uintptr_t>(sl));
  // staging (a DMA load writes lane l's element at the wave-uniform LDS base + 4 l or 16 l): wave w copies the 64
  // row pieces and the 64 scales from min(64 w, count - 64); a wave past the end repeats the last 64 (same bytes)
  const std::uint32_t bx = min(64 * wv, cols / 16 - 64), bs = min(64 * wv, nblk - 64);
  DmaRow16(xq, (bx + lane) * 16, lx + bx * 16);
  DmaDword(xs + bs + lane, ls + bs * 4);
  const std::uint32_t r = min(row, rows - 1);
  const std::int8_t* rowp = qs + static_cast<std::size_t>(r) * qstride;
  const std::uint16_t* dp = d + static_cast<std::size_t>(r) * nblk;
  int4 q[4];
  float s[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const std::uint32_t c = lane * 16 + u * 1024;
    const std::uint32_t cc = c < cols ? c : lane * 16;
    q[u] = __builtin_bit_cast(int4, __builtin_nontemporal_load(reinterpret_cast<const halo::V4i*>(rowp + cc)));
    s[u] = F16(dp[cc / 32]);
  }
  // the two staging loads (issued first) have landed; the 8 weight and scale loads stay in flight (loads complete in
  // issue order; the count of loads the compiler emits between the DMAs and this wait is checked on the built code)
  WaitVmem<8>();
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const bool ok = lane * 16 + u * 1024 < cols;
    const std::uint32_t cc = ok ? lane * 16 + u * 1024 : lane * 16;
    const int4 xv = *reinterpret_cast<const int4*>(xl + cc);
    const float sx = sl[cc / 32];
    const float part = sx * static_cast<float>(Dot16(q[u], xv));
    acc += (ok ? s[u] : 0.0f) * part;
  }
  acc = halo::GroupSum(acc);
  if (lane == 0 && row < rows) y[row] = acc;
  (void)ystride;
}
