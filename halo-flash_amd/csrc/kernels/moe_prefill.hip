// MoE layer for a batch of T tokens (prefill; gfx950, wave64): fp32 router GEMM, block-per-token top-k, grouping
// of the (token, slot) pairs by expert, grouped int8 MFMA gate/up with the SwiGLU epilogue and grouped down over each
// expert's pairs, and the slot-order combine.
//
// Reference semantics: ReferenceModel::Moe (src/model/reference.cpp:530-578), cpu::RouteTopK
// (src/model/cpu_ops.cpp:187-207); the reference's prefill groups pairs by expert with halo_moe_bucket* and runs
// MoeGateUp / MoeDown per expert group (src/kernels/core.hip:4730-4860, 5155, 5270; GroupedMoe,
// src/engine/prefill_chunk.cpp:1156-1222). Here the shared expert is one more group (index E) holding every token,
// so one grouped launch covers routed and shared experts.
//
// Pair order: pairs are sorted by expert, and within an expert by token (deterministic, no atomics). pos[t k + s] is
// the sorted position of token t's slot s; the shared expert's pairs follow at P + t (P = T k).
#include "common.h"

using halo::F16;
using halo::kWave;

// ---- fp32 GEMM for the router: C[t][n] = sum_k X[t][k] W[n][k] -----------------------------------------------------
// On v_mfma_f32_32x32x2f32. grid (ceil((N + 1) / 64), ceil(T / 64)), block 256: a 64-token x 64-row tile, wave
// (wt, wn) a 32 x 32 sub-tile; K in stages of 32 through LDS (rows padded to 36 floats: the 16-byte reads are
// conflict-free); K % 4 == 0, a trailing partial stage reads zeros. Within a stage, MFMA step s takes k = s from
// lanes 0-31 and k = 16 + s from lanes 32-63 (any k split shared by both operands sums the same products). The
// result lane l holds row n = l % 32 of its sub-tile and tokens 8 (j / 4) + 4 (l / 32) + j % 4. C [T][ldc] for rows n < N of W; when wlast is non-null it is one more row,
// whose products go to clast [T] (the shared-gate logit next to the router logits).
namespace {
typedef float V16F32R __attribute__((ext_vector_type(16)));
}
namespace halo {
// One 64 x 64 tile at rows n0 and tokens t0; K % 4 == 0 (k past K reads as zero: a trailing partial stage adds
// nothing). Every thread of the 256 must call it.
__device__ __forceinline__ void GemmF32NtTile(const float* __restrict__ X, const float* __restrict__ W,
                                              const float* __restrict__ wlast, float* __restrict__ Cm,
                                              float* __restrict__ clast, std::uint32_t T, std::uint32_t N,
                                              std::uint32_t K, std::uint32_t ldc, std::uint32_t n0,
                                              std::uint32_t t0) {
  constexpr int kLd = 36;
  __shared__ __attribute__((aligned(16))) float xl[64][kLd];
  __shared__ __attribute__((aligned(16))) float wl[64][kLd];
  const std::uint32_t tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const std::uint32_t wt = wave / 2, wn = wave % 2;
  const std::uint32_t NN = N + (wlast != nullptr ? 1u : 0u);
  // stage loads: 64 rows x 32 k per operand = 512 float4, two per thread (row c / 8, k 4 (c % 8))
  const float* gx[2];
  const float* gw[2];
  std::uint32_t lr[2], lk[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const std::uint32_t c = tid + 256u * i;
    lr[i] = c / 8;
    lk[i] = 4 * (c % 8);
    gx[i] = X + static_cast<std::size_t>(min(t0 + lr[i], T - 1)) * K;
    const std::uint32_t nr = min(n0 + lr[i], NN - 1);
    gw[i] = nr < N ? W + static_cast<std::size_t>(nr) * K : wlast;
  }
  // 4 values at k = k0 + lk of a row; past K they read as zero (from a clamped, in-bounds address)
  const auto ld = [K](const float* row, std::uint32_t k) {
    const float4 v = *reinterpret_cast<const float4*>(row + min(k, K - 4));
    return k < K ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  };
  V16F32R acc = {};
  // next stage's operands (the last stage reloads its own rows: in bounds, unused)
  float4 rx0 = ld(gx[0], lk[0]), rx1 = ld(gx[1], lk[1]);
  float4 rw0 = ld(gw[0], lk[0]), rw1 = ld(gw[1], lk[1]);
  const std::uint32_t fr = lane % 32, fh = 16 * (lane / 32);
  for (std::uint32_t k0 = 0; k0 < K; k0 += 32) {
    *reinterpret_cast<float4*>(&xl[lr[0]][lk[0]]) = rx0;
    *reinterpret_cast<float4*>(&xl[lr[1]][lk[1]]) = rx1;
    *reinterpret_cast<float4*>(&wl[lr[0]][lk[0]]) = rw0;
    *reinterpret_cast<float4*>(&wl[lr[1]][lk[1]]) = rw1;
    __syncthreads();
    const std::uint32_t kn = k0 + 32 < K ? k0 + 32 : k0;
    rx0 = ld(gx[0], kn + lk[0]);
    rx1 = ld(gx[1], kn + lk[1]);
    rw0 = ld(gw[0], kn + lk[0]);
    rw1 = ld(gw[1], kn + lk[1]);
    float a[16], b[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 av = *reinterpret_cast<const float4*>(&xl[wt * 32 + fr][fh + 4 * q]);
      const float4 bv = *reinterpret_cast<const float4*>(&wl[wn * 32 + fr][fh + 4 * q]);
      a[4 * q] = av.x, a[4 * q + 1] = av.y, a[4 * q + 2] = av.z, a[4 * q + 3] = av.w;
      b[4 * q] = bv.x, b[4 * q + 1] = bv.y, b[4 * q + 2] = bv.z, b[4 * q + 3] = bv.w;
    }
#pragma unroll
    for (int s = 0; s < 16; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], acc, 0, 0, 0);
    __syncthreads();
  }
  const std::uint32_t n = n0 + wn * 32 + fr;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const std::uint32_t t = t0 + wt * 32 + 8 * (j / 4) + 4 * (lane / 32) + j % 4;
    if (t < T && n < N) Cm[static_cast<std::size_t>(t) * ldc + n] = acc[j];
    if (t < T && n == N && wlast != nullptr) clast[t] = acc[j];
  }
}
}  // namespace halo

extern "C" __global__ void __launch_bounds__(256) halo_gemm_f32_nt(
    const float* __restrict__ X, const float* __restrict__ W, const float* __restrict__ wlast, float* __restrict__ Cm,
    float* __restrict__ clast, std::uint32_t T, std::uint32_t N, std::uint32_t K, std::uint32_t ldc) {
  halo::GemmF32NtTile(X, W, wlast, Cm, clast, T, N, K, ldc, blockIdx.x * 64, blockIdx.y * 64);
}

// ---- grouping of (token, slot) pairs by expert --------------------------------------------------------------------
// grid (ceil(T k / 4096)), block 256: count[b][e] = how many of the pairs [4096 b, 4096 b + 4096) of ids [T][k]
// select expert e (an LDS histogram per block: integer sums, so the result does not depend on the order of the
// atomics). E <= 1024.
extern "C" __global__ void __launch_bounds__(256)
    halo_moe_group_count(const std::uint32_t* __restrict__ ids, std::uint32_t* __restrict__ count, std::uint32_t T,
                         std::uint32_t k, std::uint32_t E) {
  __shared__ std::uint32_t hist[1024];
  for (std::uint32_t e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
  __syncthreads();
  const std::uint32_t p0 = blockIdx.x * 4096, p1 = min(p0 + 4096, T * k);
  for (std::uint32_t i = p0 + threadIdx.x; i < p1; i += blockDim.x) atomicAdd(&hist[ids[i]], 1u);
  __syncthreads();
  for (std::uint32_t e = threadIdx.x; e < E; e += blockDim.x) count[static_cast<std::size_t>(blockIdx.x) * E + e] = hist[e];
}

// grid 1, block 1024: start[e] = exclusive prefix of the group sizes (group e < E: the sum of count[b][e] over the nb
// partial histograms; group E: T for the shared expert when shared, else 0), and the tile table: groups cut into tiles of `tile` pairs, tiles[i] = {group, first pair, pairs},
// ntiles[0] = the tile count. E + 1 <= 1024.
extern "C" __global__ void __launch_bounds__(1024)
    halo_moe_group_scan(const std::uint32_t* __restrict__ count, std::uint32_t* __restrict__ start,
                        std::uint32_t* __restrict__ tiles, std::uint32_t* __restrict__ ntiles, std::uint32_t E,
                        std::uint32_t T, std::uint32_t shared, std::uint32_t tile, std::uint32_t nb) {
  __shared__ std::uint32_t c[1024], tcount[1024];
  const std::uint32_t g = threadIdx.x;
  std::uint32_t n = g == E && shared ? T : 0u;
  if (g < E)
    for (std::uint32_t b = 0; b < nb; ++b) n += count[static_cast<std::size_t>(b) * E + g];
  c[g] = n;
  tcount[g] = (n + tile - 1) / tile;
  __syncthreads();
  // serial prefix by one thread (E <= 1023): a few microseconds against a prefill layer
  if (g == 0) {
    std::uint32_t p = 0, q = 0;
    for (std::uint32_t i = 0; i <= E; ++i) {
      const std::uint32_t ci = c[i], ti = tcount[i];
      c[i] = p;
      tcount[i] = q;
      p += ci;
      q += ti;
    }
    start[E + 1] = p;
    ntiles[0] = q;
  }
  __syncthreads();
  if (g <= E) {
    start[g] = c[g];
    const std::uint32_t first = tcount[g];
    for (std::uint32_t i = 0; i * tile < n; ++i) {
      std::uint32_t* tt = tiles + 3 * static_cast<std::size_t>(first + i);
      tt[0] = g;
      tt[1] = c[g] + i * tile;
      tt[2] = min(tile, n - i * tile);
    }
  }
}

// grid (E + shared), block 1024: group e's pairs in token order: token[start[e] + j] = the j-th token selecting e
// (the shared group: every token), pos[t k + s] = that position for routed pairs. Compaction by ballot per chunk of
// 1024 tokens, chunks in order (16 waves per block: a quarter of the serial chunk steps of 256-token chunks).
extern "C" __global__ void __launch_bounds__(1024)
    halo_moe_group_fill(const std::uint32_t* __restrict__ ids, const std::uint32_t* __restrict__ start,
                        std::uint32_t* __restrict__ token, std::uint32_t* __restrict__ pos, std::uint32_t T,
                        std::uint32_t k, std::uint32_t E) {
  __shared__ std::uint32_t wcount[16];
  __shared__ std::uint32_t base_s;
  const std::uint32_t e = blockIdx.x, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (threadIdx.x == 0) base_s = start[e];
  __syncthreads();
  for (std::uint32_t t0 = 0; t0 < T; t0 += blockDim.x) {
    const std::uint32_t t = t0 + threadIdx.x;
    std::uint32_t slot = 0xFFFFFFFFu;
    if (t < T) {
      if (e == E) {
        slot = 0;
      } else {
#pragma unroll 4
        for (std::uint32_t s = 0; s < k; ++s)
          if (ids[static_cast<std::size_t>(t) * k + s] == e) slot = s;
      }
    }
    const bool hit = slot != 0xFFFFFFFFu;
    const std::uint64_t m = __ballot(hit);
    const std::uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<std::uint32_t>(m >> 32),
                                                          __builtin_amdgcn_mbcnt_lo(static_cast<std::uint32_t>(m), 0u));
    if (lane == 0) wcount[wave] = static_cast<std::uint32_t>(__builtin_popcountll(m));
    __syncthreads();
    std::uint32_t off = base_s;
    for (std::uint32_t w = 0; w < wave; ++w) off += wcount[w];
    if (hit) {
      const std::uint32_t p = off + below;
      token[p] = t;
      if (e < E) pos[static_cast<std::size_t>(t) * k + slot] = p;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      std::uint32_t sum = 0;
      for (std::uint32_t w = 0; w < blockDim.x / kWave; ++w) sum += wcount[w];
      base_s += sum;
    }
    __syncthreads();
  }
}

// ---- grouped int8 MFMA over the pairs of each group ---------------------------------------------------------------
// halo::GemmTileQ8Dma per (rows of group g's matrix, one tile of up to 64 (_t128: 128) pairs): group g < E reads rows g * rows + r
// of the stacked expert tensors, group E the shared expert's. Pair p's activation row is xq[gather ? gather[p] : p].
// The gate/up launch computes both matrices (64 rows of each per block, 4 waves) and writes h = SiLU(gate) * up; the
// down launch (128 rows per block, 8 waves) writes the projection. grid (ceil(rows / 64) or ceil(rows / 128), max
// tiles), block 256 / 512 (_t128: 512 / 512); blocks past ntiles[0] exit. y [pairs][ystride].
namespace {
// TOKS = 32 WT pairs per tile: WT = 2 (4 waves gate/up, 8 waves down with 128 rows) for groups of a few dozen pairs,
// WT = 4 (8 waves each, 128-pair tiles, twice the weight reuse per stage) for groups of a hundred pairs and more.
template <int WT>
__device__ __forceinline__ void GroupedGateUp(const std::int8_t* gq, const std::uint16_t* gd, const std::int8_t* uq,
                                              const std::uint16_t* ud, const std::int8_t* sgq, const std::uint16_t* sgd,
                                              const std::int8_t* suq, const std::uint16_t* sud, const std::int8_t* xq,
                                              const float* xs, const std::uint32_t* gather, const std::uint32_t* tiles,
                                              const std::uint32_t* ntiles, float* h, std::uint32_t ff, std::uint32_t H,
                                              std::uint32_t E, std::uint32_t hstride) {
  if (blockIdx.y >= ntiles[0]) return;
  const std::uint32_t* tt = tiles + 3 * static_cast<std::size_t>(blockIdx.y);
  const std::uint32_t g = tt[0], p0 = tt[1], np = tt[2];
  const bool sh = g == E;
  const std::size_t row0 = sh ? 0 : static_cast<std::size_t>(g) * ff;
  const std::uint32_t nblk = H / 32;
  halo::GemmTileQ8Dma<2, 1, WT, 2, false, 1>((sh ? sgq : gq) + row0 * H, (sh ? sgd : gd) + row0 * nblk,
                                             (sh ? suq : uq) + row0 * H, (sh ? sud : ud) + row0 * nblk, ff, H,
                                             blockIdx.x * 64, xq, xs, gather + p0, 0, np, H, h, p0, hstride);
}
template <int WR, int MT, int WT>
__device__ __forceinline__ void GroupedDown(const std::int8_t* dq, const std::uint16_t* dd, const std::int8_t* sdq,
                                            const std::uint16_t* sdd, const std::int8_t* hq, const float* hs,
                                            const std::uint32_t* tiles, const std::uint32_t* ntiles, float* y,
                                            std::uint32_t H, std::uint32_t ff, std::uint32_t E) {
  if (blockIdx.y >= ntiles[0]) return;
  const std::uint32_t* tt = tiles + 3 * static_cast<std::size_t>(blockIdx.y);
  const std::uint32_t g = tt[0], p0 = tt[1], np = tt[2];
  const bool sh = g == E;
  const std::size_t row0 = sh ? 0 : static_cast<std::size_t>(g) * H;
  const std::uint32_t nblk = ff / 32;
  halo::GemmTileQ8Dma<WR, MT, WT, 1>((sh ? sdq : dq) + row0 * ff, (sh ? sdd : dd) + row0 * nblk, nullptr, nullptr, H,
                                     ff, blockIdx.x * 128, hq, hs, nullptr, p0, np, ff, y, p0, H);
}
}  // namespace

#define HALO_GROUPED_GATE_UP(NAME, WT, THREADS)                                                                    \
  extern "C" __global__ void __launch_bounds__(THREADS) NAME(                                                      \
      const std::int8_t* gq, const std::uint16_t* gd, const std::int8_t* uq, const std::uint16_t* ud,              \
      const std::int8_t* sgq, const std::uint16_t* sgd, const std::int8_t* suq, const std::uint16_t* sud,          \
      const std::int8_t* xq, const float* xs, const std::uint32_t* gather, const std::uint32_t* tiles,             \
      const std::uint32_t* ntiles, float* h, std::uint32_t ff, std::uint32_t H, std::uint32_t E,                   \
      std::uint32_t hstride) {                                                                                     \
    GroupedGateUp<WT>(gq, gd, uq, ud, sgq, sgd, suq, sud, xq, xs, gather, tiles, ntiles, h, ff, H, E, hstride);    \
  }
HALO_GROUPED_GATE_UP(halo_moe_grouped_gate_up_q8, 2, 256)
HALO_GROUPED_GATE_UP(halo_moe_grouped_gate_up_q8_t128, 4, 512)
#undef HALO_GROUPED_GATE_UP

#define HALO_GROUPED_DOWN(NAME, WR, MT, WT)                                                                        \
  extern "C" __global__ void __launch_bounds__(512) NAME(                                                          \
      const std::int8_t* dq, const std::uint16_t* dd, const std::int8_t* sdq, const std::uint16_t* sdd,            \
      const std::int8_t* hq, const float* hs, const std::uint32_t* tiles, const std::uint32_t* ntiles, float* y,   \
      std::uint32_t H, std::uint32_t ff, std::uint32_t E) {                                                        \
    GroupedDown<WR, MT, WT>(dq, dd, sdq, sdd, hq, hs, tiles, ntiles, y, H, ff, E);                                \
  }
HALO_GROUPED_DOWN(halo_moe_grouped_down_q8, 4, 1, 2)
HALO_GROUPED_DOWN(halo_moe_grouped_down_q8_t128, 2, 2, 4)
#undef HALO_GROUPED_DOWN

// grid (ceil(H / 1024), T), block 256 (H % 4 == 0): out[t][r] = sum over s < k, in order, of weights[t][s] * y[pos[t k + s]][r],
// then + sigmoid(sgl[t]) * y[P + t][r] when the shared expert is present (sgl: its gate logit).
extern "C" __global__ void __launch_bounds__(256) halo_moe_prefill_combine(
    const float* __restrict__ y, const std::uint32_t* __restrict__ pos, const float* __restrict__ weights,
    const float* __restrict__ sgl, float* __restrict__ out, std::uint32_t T, std::uint32_t H, std::uint32_t k,
    std::uint32_t shared) {
  // four consecutive outputs per thread (16-byte loads of each selected row), each summed in slot order
  const std::uint32_t t = blockIdx.y, r = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (r >= H) return;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (std::uint32_t s = 0; s < k; ++s) {
    const float w = weights[static_cast<std::size_t>(t) * k + s];
    const float4 v = *reinterpret_cast<const float4*>(y + static_cast<std::size_t>(pos[static_cast<std::size_t>(t) * k + s]) * H + r);
    acc.x += w * v.x;
    acc.y += w * v.y;
    acc.z += w * v.z;
    acc.w += w * v.w;
  }
  if (shared) {
    const float g = halo::Sigmoid(sgl[t]);
    const float4 v = *reinterpret_cast<const float4*>(y + (static_cast<std::size_t>(T) * k + t) * H + r);
    acc.x += g * v.x;
    acc.y += g * v.y;
    acc.z += g * v.z;
    acc.w += g * v.w;
  }
  *reinterpret_cast<float4*>(out + static_cast<std::size_t>(t) * H + r) = acc;
}
