// Reference-named fp32 DeltaNet prefill kernels (src/kernels/core.hip:5925, 6053, 6111; launched by name from
// src/engine/prefill_chunk.cpp:604-645): the same names, parameter lists and grids, over one sequence of `tokens`
// tokens per launch, on this build's chunked (WY) form with fp32 matrix cores.
//
// Per value head h (key head h % num_k_heads), with log decay lg_t = a[h] softplus(alpha[t][h] + dt[h]),
// b_t = sigmoid(beta[t][h]) and the state S[i][j] (i key, j value; fp32 [heads][128][128] key-major, in place), a
// token does (reference ReferenceModel::LinearAttention, src/model/reference.cpp:329-364)
//   delta = b (v - e^lg S^T k),  S <- e^lg S + k delta^T,  o = S^T q / sqrt(128)   (o ungated).
// Over a chunk of 16 tokens with inclusive cumulative log decay G_t and starting state S0 this is exactly
//   Delta = T diag(b) (V - diag(e^G) K S0),  T = (I + A)^-1,  A[t][s] = b_t e^(G_t - G_s) (k_t . k_s)  (s < t)
//   O = (diag(e^G) Q S0 + P Delta) / sqrt(128),  P[t][s] = e^(G_t - G_s) (q_t . k_s)  (s <= t)
//   S_C = e^(G_last) S0 + K^T diag(e^(G_last - G_t)) Delta.
// halo_gdn_chunk_prep forms what does not depend on the state for every chunk in parallel (G, b, T and P);
// halo_gdn_chunk_scan walks the chunks of a head in order; halo_gdn_prefill_split does both in one launch (each block
// forms its chunks' G, b, T and P itself). Tokens past a partial chunk's end are zero rows (k = q = v = 0, b = 0,
// lg = 0), so their rows of every product vanish.
//   q, k rows at t * qk_stride (key head kh at kh * 128), v at t * v_stride (head h at h * 128), out at t * o_stride;
//   alpha, beta [tokens][heads] (heads = gridDim.y); a, dt [heads].
#include "common.h"

namespace {
constexpr std::uint32_t kRc = 16;                           // tokens per chunk (the reference's grid convention)
constexpr std::uint32_t kRd = 128;                          // head dim
constexpr std::uint32_t kRPrep = 2 * kRc + 2 * kRc * kRc;   // per (head, chunk): G, b, T, P = 544 floats
constexpr std::uint32_t kRow = kRd + 4;                     // LDS row stride of token-major q / k tiles
typedef float V4R __attribute__((ext_vector_type(4)));

// Loads chunk rows [t0, t0 + n) of q and k (key head kh) into ks / qs (rows >= n zeroed); all 256 threads. With kt,
// also K transposed (kt[key][token], row stride 20).
__device__ __forceinline__ void LoadQK(const float* __restrict__ q, const float* __restrict__ k, std::uint32_t t0,
                                       std::uint32_t n, std::uint32_t kh, std::uint32_t qk_stride,
                                       float (*ks)[kRow], float (*qs)[kRow], float (*kt)[20]) {
  const std::uint32_t tid = threadIdx.x;
#pragma unroll
  for (std::uint32_t p = 0; p < 2; ++p) {
    const std::uint32_t x = tid + 256 * p, tt = x / 32, i = (x % 32) * 4;
    float4 kv = make_float4(0.0f, 0.0f, 0.0f, 0.0f), qv = kv;
    if (tt < n) {
      const std::size_t row = static_cast<std::size_t>(t0 + tt) * qk_stride + kh * kRd + i;
      kv = *reinterpret_cast<const float4*>(k + row);
      qv = *reinterpret_cast<const float4*>(q + row);
    }
    *reinterpret_cast<float4*>(&ks[tt][i]) = kv;
    *reinterpret_cast<float4*>(&qs[tt][i]) = qv;
    if (kt != nullptr) {
      kt[i][tt] = kv.x;
      kt[i + 1][tt] = kv.y;
      kt[i + 2][tt] = kv.z;
      kt[i + 3][tt] = kv.w;
    }
  }
}

// One chunk's G, b, T and P into pp (layout: G [16], b [16], T [16][16], P [16][16]) from ks / qs in LDS and the
// chunk's gate inputs; all 256 threads, barriers inside; pp complete when it returns.
__device__ __forceinline__ void ChunkGates(const float (*ks)[kRow], const float (*qs)[kRow],
                                           const float* __restrict__ alpha, const float* __restrict__ beta, float ah,
                                           float dth, std::uint32_t h, std::uint32_t heads, std::uint32_t t0,
                                           std::uint32_t n, float* pp, float (*A)[kRc + 1]) {
  const std::uint32_t tid = threadIdx.x;
  float* G = pp;
  float* bs = pp + kRc;
  float* T = pp + 2 * kRc;
  float* P = T + kRc * kRc;
  if (tid < kRc) {  // lanes 0-15 of wave 0: gates and the inclusive prefix sum of the log decays
    const bool on = tid < n;
    const std::size_t at = static_cast<std::size_t>(t0 + (on ? tid : 0)) * heads + h;
    float g = on ? ah * halo::Softplus(alpha[at] + dth) : 0.0f;
#pragma unroll
    for (std::uint32_t o = 1; o < kRc; o <<= 1) {
      const float up = __shfl_up(g, o, kRc);
      if (tid >= o) g += up;
    }
    G[tid] = g;
    bs[tid] = on ? halo::Sigmoid(beta[at]) : 0.0f;
  }
  __syncthreads();
  {  // thread (t, s): k_t . k_s and q_t . k_s over the 128 dims
    const std::uint32_t t = tid / kRc, s = tid % kRc;
    float kk = 0.0f, qk = 0.0f;
#pragma unroll 8
    for (std::uint32_t i = 0; i < kRd; i += 4) {
      const float4 a4 = *reinterpret_cast<const float4*>(&ks[t][i]);
      const float4 q4 = *reinterpret_cast<const float4*>(&qs[t][i]);
      const float4 b4 = *reinterpret_cast<const float4*>(&ks[s][i]);
      kk += a4.x * b4.x + a4.y * b4.y + a4.z * b4.z + a4.w * b4.w;
      qk += q4.x * b4.x + q4.y * b4.y + q4.z * b4.z + q4.w * b4.w;
    }
    const float e = s <= t ? expf(G[t] - G[s]) : 0.0f;
    A[t][s] = s < t ? bs[t] * e * kk : 0.0f;
    P[t * kRc + s] = e * qk;
  }
  __syncthreads();
  if (tid < kRc) {  // T = (I + A)^-1, unit lower triangular: lane c forms column c by forward substitution
    const std::uint32_t c = tid;
    float col[kRc];
#pragma unroll
    for (std::uint32_t t = 0; t < kRc; ++t) {
      float r = t == c ? 1.0f : 0.0f;
      if (t > c) {
#pragma unroll
        for (std::uint32_t u = 0; u < t; ++u)
          if (u >= c) r -= A[t][u] * col[u];
      }
      col[t] = r;
      T[t * kRc + c] = r;
    }
  }
  __syncthreads();
}

// The chunk-serial part for 64 value columns [64 cb, 64 cb + 64) of head h (block of 4 waves, wave w the 16
// columns 16 w ..; every product on v_mfma_f32_16x16x4f32: A lane l = A[l % 16][k], B lane l = B[k][l % 16], D lane l
// holds column l % 16 and rows 4 (l / 16) + r, each lane quarter taking a contiguous quarter of the k range so
// operand reads are 16 bytes). The state slice stays in LDS transposed (st[column][key]) for the whole sequence.
// chunk_prep(c, t0, n) fills pp for chunk c (after the chunk's q / k are in ks / qs, kt).
template <typename PrepFn>
__device__ __forceinline__ void ChunkScan(const float* __restrict__ q, const float* __restrict__ k,
                                          const float* __restrict__ v, float* __restrict__ state,
                                          float* __restrict__ out, std::uint32_t num_k_heads, std::uint32_t tokens,
                                          std::uint32_t qk_stride, std::uint32_t v_stride, std::uint32_t o_stride,
                                          float* pp, PrepFn chunk_prep, float (*ks)[kRow], float (*qs)[kRow]) {
  __shared__ __attribute__((aligned(16))) float kt[kRd][20];
  __shared__ __attribute__((aligned(16))) float st[64][kRow];
  __shared__ __attribute__((aligned(16))) float vs[kRc][64];
  __shared__ __attribute__((aligned(16))) float rt[64][20], dlt[64][20], wt[64][20];
  const std::uint32_t h = blockIdx.y, cb = blockIdx.x, tid = threadIdx.x;
  const std::uint32_t wave = tid / 64, lane = tid % 64, lr = lane % 16, q4 = lane / 16;
  const std::uint32_t col = 16 * wave + lr;  // this lane's column within the block's 64
  const std::uint32_t kh = h % num_k_heads;
  float* Sg = state + static_cast<std::size_t>(h) * kRd * kRd + 64 * cb;
  for (std::uint32_t x = tid; x < kRd * 16; x += 256) {  // 128 keys x 16 float4 columns
    const std::uint32_t key = x / 16, c4 = (x % 16) * 4;
    const float4 s4 = *reinterpret_cast<const float4*>(Sg + static_cast<std::size_t>(key) * kRd + c4);
    st[c4][key] = s4.x;
    st[c4 + 1][key] = s4.y;
    st[c4 + 2][key] = s4.z;
    st[c4 + 3][key] = s4.w;
  }
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(kRd));
  const std::uint32_t nchunks = (tokens + kRc - 1) / kRc;
  for (std::uint32_t c = 0; c < nchunks; ++c) {
    const std::uint32_t t0 = c * kRc, n = min(kRc, tokens - t0);
    __syncthreads();  // the previous chunk's LDS reads are done
    LoadQK(q, k, t0, n, kh, qk_stride, ks, qs, kt);
    for (std::uint32_t x = tid; x < kRc * 16; x += 256) {
      const std::uint32_t tt = x / 16, c4 = (x % 16) * 4;
      float4 v4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (tt < n)
        v4 = *reinterpret_cast<const float4*>(v + static_cast<std::size_t>(t0 + tt) * v_stride + h * kRd + 64 * cb + c4);
      *reinterpret_cast<float4*>(&vs[tt][c4]) = v4;
    }
    __syncthreads();
    chunk_prep(c, t0, n);  // pp ready after this (its own barriers)
    const float* G = pp;
    const float* bs = pp + kRc;
    const float* T = pp + 2 * kRc;
    const float* P = T + kRc * kRc;
    // U = K S0 and Qd = Q S0 (16 tokens x this wave's 16 columns), k over the 128 keys
    V4R u = {0.0f, 0.0f, 0.0f, 0.0f}, qd = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (std::uint32_t kb = 0; kb < 8; ++kb) {
      const std::uint32_t key = 32 * q4 + 4 * kb;
      const float4 a4 = *reinterpret_cast<const float4*>(&ks[lr][key]);
      const float4 c4 = *reinterpret_cast<const float4*>(&qs[lr][key]);
      const float4 b4 = *reinterpret_cast<const float4*>(&st[col][key]);
      u = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, b4.x, u, 0, 0, 0);
      qd = __builtin_amdgcn_mfma_f32_16x16x4f32(c4.x, b4.x, qd, 0, 0, 0);
      u = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, b4.y, u, 0, 0, 0);
      qd = __builtin_amdgcn_mfma_f32_16x16x4f32(c4.y, b4.y, qd, 0, 0, 0);
      u = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, b4.z, u, 0, 0, 0);
      qd = __builtin_amdgcn_mfma_f32_16x16x4f32(c4.z, b4.z, qd, 0, 0, 0);
      u = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, b4.w, u, 0, 0, 0);
      qd = __builtin_amdgcn_mfma_f32_16x16x4f32(c4.w, b4.w, qd, 0, 0, 0);
    }
    // R = diag(b) (V - diag(e^G) U), stored transposed for the next product's B operand
    float4 r4;
    {
      float rr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const std::uint32_t t = 4 * q4 + r;
        rr[r] = bs[t] * (vs[t][col] - expf(G[t]) * u[r]);
      }
      r4 = make_float4(rr[0], rr[1], rr[2], rr[3]);
      *reinterpret_cast<float4*>(&rt[col][4 * q4]) = r4;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Delta = T R
    V4R dl = {0.0f, 0.0f, 0.0f, 0.0f};
    {
      const float4 a4 = *reinterpret_cast<const float4*>(&T[lr * kRc + 4 * q4]);
      const float4 b4 = *reinterpret_cast<const float4*>(&rt[col][4 * q4]);
      dl = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, b4.x, dl, 0, 0, 0);
      dl = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, b4.y, dl, 0, 0, 0);
      dl = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, b4.z, dl, 0, 0, 0);
      dl = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, b4.w, dl, 0, 0, 0);
    }
    const float glast = G[n - 1];
    {
      float w4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) w4[r] = expf(glast - G[4 * q4 + r]) * dl[r];
      *reinterpret_cast<float4*>(&dlt[col][4 * q4]) = make_float4(dl[0], dl[1], dl[2], dl[3]);
      *reinterpret_cast<float4*>(&wt[col][4 * q4]) = make_float4(w4[0], w4[1], w4[2], w4[3]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // O = (diag(e^G) Qd + P Delta) / sqrt(d)
    {
      V4R o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = expf(G[4 * q4 + r]) * qd[r];
      const float4 a4 = *reinterpret_cast<const float4*>(&P[lr * kRc + 4 * q4]);
      const float4 b4 = *reinterpret_cast<const float4*>(&dlt[col][4 * q4]);
      o = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, b4.x, o, 0, 0, 0);
      o = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, b4.y, o, 0, 0, 0);
      o = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, b4.z, o, 0, 0, 0);
      o = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, b4.w, o, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const std::uint32_t t = 4 * q4 + r;
        if (t < n) out[static_cast<std::size_t>(t0 + t) * o_stride + h * kRd + 64 * cb + col] = o[r] * inv_sqrt_d;
      }
    }
    // S = e^G_last S0 + K^T W, W = diag(e^(G_last - G)) Delta; key tiles of 16, this wave's 16 columns
    const float en = expf(glast);
    const float4 wb = *reinterpret_cast<const float4*>(&wt[col][4 * q4]);
#pragma unroll
    for (std::uint32_t m = 0; m < kRd / 16; ++m) {
      const std::uint32_t key0 = 16 * m + 4 * q4;
      const float4 s4 = *reinterpret_cast<const float4*>(&st[col][key0]);
      V4R acc = {en * s4.x, en * s4.y, en * s4.z, en * s4.w};
      const float4 a4 = *reinterpret_cast<const float4*>(&kt[16 * m + lr][4 * q4]);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, wb.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, wb.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, wb.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, wb.w, acc, 0, 0, 0);
      *reinterpret_cast<float4*>(&st[col][key0]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
  }
  __syncthreads();
  for (std::uint32_t x = tid; x < kRd * 16; x += 256) {
    const std::uint32_t key = x / 16, c4 = (x % 16) * 4;
    *reinterpret_cast<float4*>(Sg + static_cast<std::size_t>(key) * kRd + c4) =
        make_float4(st[c4][key], st[c4 + 1][key], st[c4 + 2][key], st[c4 + 3][key]);
  }
}
}  // namespace

// grid (ceil(tokens / 16), heads), block 256: per (chunk, value head) G, b, T and P into
// prep [head][chunk][544] (the reference engine's gdnprep buffer holds 576 floats per (head, 16-token chunk)).
extern "C" __global__ void __launch_bounds__(256)
    halo_gdn_chunk_prep(const float* q, const float* k, const float* alpha, const float* beta, const float* a,
                        const float* dt, float* prep, std::uint32_t num_k_heads, std::uint32_t tokens,
                        std::uint32_t qk_stride) {
  __shared__ __attribute__((aligned(16))) float ks[kRc][kRow], qs[kRc][kRow];
  __shared__ __attribute__((aligned(16))) float pp[kRPrep];
  __shared__ float A[kRc][kRc + 1];
  const std::uint32_t c = blockIdx.x, h = blockIdx.y, heads = gridDim.y;
  const std::uint32_t t0 = c * kRc, n = min(kRc, tokens - t0);
  LoadQK(q, k, t0, n, h % num_k_heads, qk_stride, ks, qs, nullptr);
  __syncthreads();
  ChunkGates(ks, qs, alpha, beta, a[h], dt[h], h, heads, t0, n, pp, A);
  float* dst = prep + (static_cast<std::size_t>(h) * gridDim.x + c) * kRPrep;
  for (std::uint32_t x = threadIdx.x; x < kRPrep; x += blockDim.x) dst[x] = pp[x];
}

// grid (2, heads), block 256: the chunk scan over halo_gdn_chunk_prep's output (block x: value columns 64 x ..).
extern "C" __global__ void __launch_bounds__(256)
    halo_gdn_chunk_scan(const float* q, const float* k, const float* v, const float* prep, float* state, float* out,
                        std::uint32_t num_k_heads, std::uint32_t tokens, std::uint32_t qk_stride,
                        std::uint32_t v_stride, std::uint32_t o_stride) {
  __shared__ __attribute__((aligned(16))) float ks[kRc][kRow], qs[kRc][kRow];
  __shared__ __attribute__((aligned(16))) float pp[kRPrep];
  const std::uint32_t h = blockIdx.y, nchunks = (tokens + kRc - 1) / kRc;
  auto prep_of = [&](std::uint32_t c, std::uint32_t, std::uint32_t) {
    const float* src = prep + (static_cast<std::size_t>(h) * nchunks + c) * kRPrep;
    for (std::uint32_t x = threadIdx.x; x < kRPrep; x += blockDim.x) pp[x] = src[x];
    __syncthreads();
  };
  ChunkScan(q, k, v, state, out, num_k_heads, tokens, qk_stride, v_stride, o_stride, pp, prep_of, ks, qs);
}

// grid (2, heads), block 256: the whole recurrence in one launch (each block forms its chunks' G, b, T and P).
extern "C" __global__ void __launch_bounds__(256)
    halo_gdn_prefill_split(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                           const float* a, const float* dt, float* state, float* out, std::uint32_t num_k_heads,
                           std::uint32_t tokens, std::uint32_t qk_stride, std::uint32_t v_stride,
                           std::uint32_t o_stride) {
  __shared__ __attribute__((aligned(16))) float ks[kRc][kRow], qs[kRc][kRow];
  __shared__ __attribute__((aligned(16))) float pp[kRPrep];
  __shared__ float A[kRc][kRc + 1];
  const std::uint32_t h = blockIdx.y, heads = gridDim.y;
  const float ah = a[h], dth = dt[h];
  auto prep_here = [&](std::uint32_t, std::uint32_t t0, std::uint32_t n) {
    ChunkGates(ks, qs, alpha, beta, ah, dth, h, heads, t0, n, pp, A);
  };
  ChunkScan(q, k, v, state, out, num_k_heads, tokens, qk_stride, v_stride, o_stride, pp, prep_here, ks, qs);
}
