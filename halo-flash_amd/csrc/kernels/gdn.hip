// Gated DeltaNet recurrence (gfx950, wave64): the decode step for S sessions and the chunked prefill.
//
// Per value head h (key head h % Hk), with decay = exp(g) and the state S[i][j] (i key, j value), a token does
// (reference ReferenceModel::LinearAttention, src/model/reference.cpp:329-364):
//   u = (decay S)^T k,  delta = (v - u) * beta,  S <- decay S + k delta^T,  o = S^T q / sqrt(d).
// State layout in HBM: fp32 [session][head][i][j], key-major (row i holds the 128 value columns contiguously),
// so that a lane's 16-byte load covers 4 value columns and a wave covers whole rows.
#include "common.h"

using halo::kWave;

namespace {
constexpr int kD = 128;       // head dim (d_k = d_v)
constexpr int kJBlock = 32;   // value columns per block
}  // namespace

// grid (S * Hv * 4), block 256. Block -> (session s, head h, value columns [32 jb, 32 jb + 32)); thread: 4 value
// columns (one float4) x 4 key rows. Columns are independent in the recurrence, so the four column blocks of a
// head run in parallel.
//   state [S][Hv][128][128] fp32 (in place), q, k [S][Hk][128], v [S][Hv][128], g, beta [S][Hv], o [S][Hv][128].
extern "C" __global__ void __launch_bounds__(256)
    halo_gdn_decode_d128(float* __restrict__ state, const float* __restrict__ q, const float* __restrict__ k,
                         const float* __restrict__ v, const float* __restrict__ g, const float* __restrict__ beta,
                         float* __restrict__ o, std::uint32_t S, std::uint32_t Hv, std::uint32_t Hk) {
  __shared__ float red[32][kJBlock + 1];
  __shared__ float dl[kJBlock];
  const std::uint32_t b = blockIdx.x, jb = b % 4, h = (b / 4) % Hv, s = b / (4 * Hv);
  if (s >= S) return;
  const std::uint32_t t = threadIdx.x, r8 = t % 8, ig = t / 8;
  const std::uint32_t j0 = jb * kJBlock + r8 * 4, i0 = ig * 4;
  const std::uint32_t kh = h % Hk;
  float* St = state + ((static_cast<std::size_t>(s) * Hv + h) * kD) * kD;
  const float* kk = k + (static_cast<std::size_t>(s) * Hk + kh) * kD;
  const float* qq = q + (static_cast<std::size_t>(s) * Hk + kh) * kD;
  const float decay = expf(g[s * Hv + h]);
  const float bt = beta[s * Hv + h];
  float4 row[4];
  float ki[4], qi[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    row[r] = *reinterpret_cast<const float4*>(St + static_cast<std::size_t>(i0 + r) * kD + j0);
    ki[r] = kk[i0 + r];
    qi[r] = qq[i0 + r];
  }
  float u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    row[r].x *= decay;
    row[r].y *= decay;
    row[r].z *= decay;
    row[r].w *= decay;
    u[0] += row[r].x * ki[r];
    u[1] += row[r].y * ki[r];
    u[2] += row[r].z * ki[r];
    u[3] += row[r].w * ki[r];
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) red[ig][r8 * 4 + c] = u[c];
  __syncthreads();
  if (t < kJBlock) {
    float acc = 0.0f;
    for (int i = 0; i < 32; ++i) acc += red[i][t];
    const float vj = v[(static_cast<std::size_t>(s) * Hv + h) * kD + jb * kJBlock + t];
    dl[t] = (vj - acc) * bt;
  }
  __syncthreads();
  const float d0 = dl[r8 * 4], d1 = dl[r8 * 4 + 1], d2 = dl[r8 * 4 + 2], d3 = dl[r8 * 4 + 3];
  float oo[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    row[r].x += ki[r] * d0;
    row[r].y += ki[r] * d1;
    row[r].z += ki[r] * d2;
    row[r].w += ki[r] * d3;
    oo[0] += row[r].x * qi[r];
    oo[1] += row[r].y * qi[r];
    oo[2] += row[r].z * qi[r];
    oo[3] += row[r].w * qi[r];
    *reinterpret_cast<float4*>(St + static_cast<std::size_t>(i0 + r) * kD + j0) = row[r];
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) red[ig][r8 * 4 + c] = oo[c];
  __syncthreads();
  if (t < kJBlock) {
    float acc = 0.0f;
    for (int i = 0; i < 32; ++i) acc += red[i][t];
    o[(static_cast<std::size_t>(s) * Hv + h) * kD + jb * kJBlock + t] = acc * (1.0f / sqrtf(static_cast<float>(kD)));
  }
}

// ---- chunked prefill (C = 64) over a ragged batch of sequences -----------------------------------------------
// Within a chunk of C tokens with cumulative log-decay G_t (gamma_t = exp(G_t)) and initial state S0, the token
// recurrence above is exactly (reference math comment src/kernels/core.hip:6035-6048, there with C = 16):
//   (I + A) Delta = diag(beta) V - diag(beta gamma) K S0,   A[t][s] = beta_t exp(G_t - G_s) (k_t . k_s), s < t
//   O = (diag(gamma) Q S0 + P Delta) / sqrt(d),             P[t][s] = exp(G_t - G_s) (q_t . k_s),         s <= t
//   S_C = gamma_C S0 + K^T diag(exp(G_C - G_s)) Delta.
// halo_gdn_chunk_prep computes, for every (chunk, head) in parallel, T = (I + A)^-1 (forward substitution), P and
// G; halo_gdn_chunk_scan walks each sequence's chunks in order carrying S, with Delta = T Z and
// Z = diag(beta) V - diag(beta gamma) (K S0). Tokens past a partial chunk's end are zero-padded (beta = 0, g = 0),
// which makes them contribute nothing. Inputs q, k [tokens][Hk][128] and v [tokens][Hv][128] are bf16 (the C3 operator) or fp32 (the model's
// prefill, which matches its decode step); g, beta
// [tokens][Hv] fp32 (g = log decay, beta after its sigmoid); state fp32 [seq][Hv][128][128] key-major.
// chunks [n][3] = {first token, length, sequence}; seqs [n_seq][2] = {first chunk, chunk count}.
namespace {
constexpr int kC = 64;

__device__ __forceinline__ float Bf(std::uint16_t h) { return __uint_as_float(static_cast<std::uint32_t>(h) << 16); }
__device__ __forceinline__ float Cv(std::uint16_t h) { return Bf(h); }
__device__ __forceinline__ float Cv(float x) { return x; }
// eight consecutive inputs (16 bytes of bf16, 32 of fp32)
template <typename In>
struct alignas(16) Pack8 {
  In v[8];
};
template <typename In>
__device__ __forceinline__ Pack8<In> Ld8(const In* p) {
  return *reinterpret_cast<const Pack8<In>*>(p);
}
template <typename In>
__device__ __forceinline__ Pack8<In> Zero8() {
  Pack8<In> z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z.v[e] = In{};
  return z;
}
}  // namespace

// grid (n_chunks, Hv), block 256. Tm, Pm [n_chunks][Hv][64][64] fp32, Gc [n_chunks][Hv][64]. In: std::uint16_t
// (bf16) or float.
template <typename In>
__device__ __forceinline__ void ChunkPrep(const In* __restrict__ q, const In* __restrict__ k,
                                          const float* __restrict__ g, const float* __restrict__ beta,
                                          const std::uint32_t* __restrict__ chunks, float* __restrict__ Tm,
                                          float* __restrict__ Pm, float* __restrict__ Gc, std::uint32_t Hv,
                                          std::uint32_t Hk) {
  __shared__ union {
    struct {
      In kb[kC][kD];
      In qb[kC][kD];
    } in;
    float tm[kC][kC + 1];
  } u;
  __shared__ float am[kC][kC + 1];
  __shared__ float G[kC], B[kC];
  const std::uint32_t c = blockIdx.x, h = blockIdx.y, kh = h % Hk, tid = threadIdx.x;
  const std::uint32_t start = chunks[c * 3], L = chunks[c * 3 + 1];
  for (std::uint32_t idx = tid; idx < kC * (kD / 8); idx += blockDim.x) {
    const std::uint32_t t = idx / (kD / 8), p = idx % (kD / 8);
    Pack8<In> kv = Zero8<In>(), qv = Zero8<In>();
    if (t < L) {
      const std::size_t off = (static_cast<std::size_t>(start + t) * Hk + kh) * kD + p * 8;
      kv = Ld8(k + off);
      qv = Ld8(q + off);
    }
    *reinterpret_cast<Pack8<In>*>(&u.in.kb[t][p * 8]) = kv;
    *reinterpret_cast<Pack8<In>*>(&u.in.qb[t][p * 8]) = qv;
  }
  if (tid < kC) {
    const bool in = tid < L;
    G[tid] = in ? g[static_cast<std::size_t>(start + tid) * Hv + h] : 0.0f;
    B[tid] = in ? beta[static_cast<std::size_t>(start + tid) * Hv + h] : 0.0f;
  }
  __syncthreads();
  if (tid == 0)
    for (int t = 1; t < kC; ++t) G[t] += G[t - 1];
  __syncthreads();
  // A (strictly lower) and P (lower incl. diagonal); thread: row t, 16 columns
  const std::size_t mat = (static_cast<std::size_t>(c) * Hv + h) * kC * kC;
  {
    const std::uint32_t t = tid / 4, s0 = (tid % 4) * 16;
    float kk[16], qk[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) kk[j] = qk[j] = 0.0f;
    for (int i = 0; i < kD; i += 8) {
      const Pack8<In> kt = Ld8(&u.in.kb[t][i]);
      const Pack8<In> qt = Ld8(&u.in.qb[t][i]);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const Pack8<In> ks = Ld8(&u.in.kb[s0 + j][i]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float kse = Cv(ks.v[e]);
          kk[j] += Cv(kt.v[e]) * kse;
          qk[j] += Cv(qt.v[e]) * kse;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const std::uint32_t s = s0 + j;
      const float dec = expf(G[t] - G[s]);
      am[t][s] = s < t ? B[t] * dec * kk[j] : 0.0f;
      Pm[mat + t * kC + s] = s <= t ? dec * qk[j] : 0.0f;
    }
  }
  __syncthreads();
  // T = (I + A)^-1 by rows: T[t][c] = -sum_{s=c}^{t-1} A[t][s] T[s][c] (c < t), 1 on the diagonal. One wave; LDS
  // accesses of a wave complete in order, so rows need no block barrier.
  if (tid < kC) {
    const std::uint32_t col = tid;
    for (std::uint32_t t = 0; t < kC; ++t) {
      float v = col == t ? 1.0f : 0.0f;
      if (col < t)
        for (std::uint32_t s = col; s < t; ++s) v -= am[t][s] * u.tm[s][col];
      u.tm[t][col] = v;
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();
  for (std::uint32_t e = tid; e < kC * kC; e += blockDim.x) Tm[mat + e] = u.tm[e / kC][e % kC];
  if (tid < kC) Gc[(static_cast<std::size_t>(c) * Hv + h) * kC + tid] = G[tid];
}

// grid (n_seq * Hv * 4), block 256: block -> (sequence, head, 32 value columns); walks the sequence's chunks.
// o [tokens][Hv][128] fp32; state [seq][Hv][128][128] read as the initial state and overwritten with the final one.
template <typename In>
__device__ __forceinline__ void ChunkScan(
    const In* __restrict__ q, const In* __restrict__ k, const In* __restrict__ v, const float* __restrict__ beta, const std::uint32_t* __restrict__ chunks, const std::uint32_t* __restrict__ seqs,
    const float* __restrict__ Tm, const float* __restrict__ Pm, const float* __restrict__ Gc,
    float* __restrict__ state, float* __restrict__ o, std::uint32_t Hv, std::uint32_t Hk) {
  __shared__ float S0[kD][kJBlock];
  __shared__ float Zd[kC][kJBlock + 1];
  __shared__ float tm[kC][kC];
  __shared__ float pm[kC][kC];
  __shared__ float G[kC], Bt[kC], Wd[kC];
  const std::uint32_t b = blockIdx.x, jb = b % 4, h = (b / 4) % Hv, sq = b / (4 * Hv), kh = h % Hk;
  const std::uint32_t tid = threadIdx.x;
  const std::uint32_t c0 = seqs[sq * 2], nc = seqs[sq * 2 + 1];
  float* St = state + (static_cast<std::size_t>(sq) * Hv + h) * kD * kD;
  for (std::uint32_t e = tid; e < kD * kJBlock; e += blockDim.x)
    S0[e / kJBlock][e % kJBlock] = St[static_cast<std::size_t>(e / kJBlock) * kD + jb * kJBlock + e % kJBlock];
  const std::uint32_t t = tid / 4, jg = tid % 4;             // rows of the chunk x 8 columns
  const std::uint32_t si = tid % kD, sh = tid / kD;          // state row x 16 columns
  const float qscale = 1.0f / sqrtf(static_cast<float>(kD));
  for (std::uint32_t ci = 0; ci < nc; ++ci) {
    const std::uint32_t c = c0 + ci, start = chunks[c * 3], L = chunks[c * 3 + 1];
    const std::size_t mat = (static_cast<std::size_t>(c) * Hv + h) * kC * kC;
    __syncthreads();
    for (std::uint32_t e = tid * 4; e < kC * kC; e += blockDim.x * 4) {
      *reinterpret_cast<float4*>(&tm[0][0] + e) = *reinterpret_cast<const float4*>(Tm + mat + e);
      *reinterpret_cast<float4*>(&pm[0][0] + e) = *reinterpret_cast<const float4*>(Pm + mat + e);
    }
    if (tid < kC) {
      G[tid] = Gc[(static_cast<std::size_t>(c) * Hv + h) * kC + tid];
      Bt[tid] = tid < L ? beta[static_cast<std::size_t>(start + tid) * Hv + h] : 0.0f;
    }
    __syncthreads();
    if (tid < kC) Wd[tid] = expf(G[kC - 1] - G[tid]);
    // X = K S0, Y = Q S0 (row t, 8 columns)
    float X[8], Y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) X[j] = Y[j] = 0.0f;
    const bool live = t < L;
    const std::size_t krow = (static_cast<std::size_t>(start + t) * Hk + kh) * kD;
    for (int i = 0; i < kD; i += 8) {
      Pack8<In> kv = Zero8<In>(), qv = Zero8<In>();
      if (live) {
        kv = Ld8(k + krow + i);
        qv = Ld8(q + krow + i);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float ke = Cv(kv.v[e]), qe = Cv(qv.v[e]);
        const float4 s_lo = *reinterpret_cast<const float4*>(&S0[i + e][jg * 8]);
        const float4 s_hi = *reinterpret_cast<const float4*>(&S0[i + e][jg * 8 + 4]);
        X[0] += ke * s_lo.x; X[1] += ke * s_lo.y; X[2] += ke * s_lo.z; X[3] += ke * s_lo.w;
        X[4] += ke * s_hi.x; X[5] += ke * s_hi.y; X[6] += ke * s_hi.z; X[7] += ke * s_hi.w;
        Y[0] += qe * s_lo.x; Y[1] += qe * s_lo.y; Y[2] += qe * s_lo.z; Y[3] += qe * s_lo.w;
        Y[4] += qe * s_hi.x; Y[5] += qe * s_hi.y; Y[6] += qe * s_hi.z; Y[7] += qe * s_hi.w;
      }
    }
    const float gam = expf(G[t]);
    {
      Pack8<In> vv = Zero8<In>();
      if (live) vv = Ld8(v + (static_cast<std::size_t>(start + t) * Hv + h) * kD + jb * kJBlock + jg * 8);
#pragma unroll
      for (int j = 0; j < 8; ++j) Zd[t][jg * 8 + j] = Bt[t] * (Cv(vv.v[j]) - gam * X[j]);
    }
    __syncthreads();
    float D[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) D[j] = 0.0f;
    for (std::uint32_t s = 0; s <= t; ++s) {
      const float w = tm[t][s];
#pragma unroll
      for (int j = 0; j < 8; ++j) D[j] += w * Zd[s][jg * 8 + j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) Zd[t][jg * 8 + j] = D[j];
    __syncthreads();
    if (live) {
      float O[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) O[j] = gam * Y[j];
      for (std::uint32_t s = 0; s <= t; ++s) {
        const float w = pm[t][s];
#pragma unroll
        for (int j = 0; j < 8; ++j) O[j] += w * Zd[s][jg * 8 + j];
      }
      float* orow = o + (static_cast<std::size_t>(start + t) * Hv + h) * kD + jb * kJBlock + jg * 8;
      *reinterpret_cast<float4*>(orow) = make_float4(O[0] * qscale, O[1] * qscale, O[2] * qscale, O[3] * qscale);
      *reinterpret_cast<float4*>(orow + 4) = make_float4(O[4] * qscale, O[5] * qscale, O[6] * qscale, O[7] * qscale);
    }
    // S <- gamma_C S + K^T diag(exp(G_C - G_t)) Delta   (row si, 16 columns)
    const float gc = expf(G[kC - 1]);
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = gc * S0[si][sh * 16 + j];
    for (std::uint32_t tt = 0; tt < L; ++tt) {
      const float w = Cv(k[(static_cast<std::size_t>(start + tt) * Hk + kh) * kD + si]) * Wd[tt];
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[j] += w * Zd[tt][sh * 16 + j];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) S0[si][sh * 16 + j] = acc[j];
  }
  __syncthreads();
  for (std::uint32_t e = tid; e < kD * kJBlock; e += blockDim.x)
    St[static_cast<std::size_t>(e / kJBlock) * kD + jb * kJBlock + e % kJBlock] = S0[e / kJBlock][e % kJBlock];
}

extern "C" __global__ void __launch_bounds__(256)
    halo_gdn_chunk_prep(const std::uint16_t* __restrict__ q, const std::uint16_t* __restrict__ k,
                        const float* __restrict__ g, const float* __restrict__ beta,
                        const std::uint32_t* __restrict__ chunks, float* __restrict__ Tm, float* __restrict__ Pm,
                        float* __restrict__ Gc, std::uint32_t Hv, std::uint32_t Hk) {
  ChunkPrep(q, k, g, beta, chunks, Tm, Pm, Gc, Hv, Hk);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_gdn_chunk_prep_f32(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ g,
                            const float* __restrict__ beta, const std::uint32_t* __restrict__ chunks,
                            float* __restrict__ Tm, float* __restrict__ Pm, float* __restrict__ Gc, std::uint32_t Hv,
                            std::uint32_t Hk) {
  ChunkPrep(q, k, g, beta, chunks, Tm, Pm, Gc, Hv, Hk);
}
extern "C" __global__ void __launch_bounds__(256) halo_gdn_chunk_scan(
    const std::uint16_t* __restrict__ q, const std::uint16_t* __restrict__ k, const std::uint16_t* __restrict__ v,
    const float* __restrict__ beta, const std::uint32_t* __restrict__ chunks, const std::uint32_t* __restrict__ seqs,
    const float* __restrict__ Tm, const float* __restrict__ Pm, const float* __restrict__ Gc,
    float* __restrict__ state, float* __restrict__ o, std::uint32_t Hv, std::uint32_t Hk) {
  ChunkScan(q, k, v, beta, chunks, seqs, Tm, Pm, Gc, state, o, Hv, Hk);
}
extern "C" __global__ void __launch_bounds__(256) halo_gdn_chunk_scan_f32(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ beta, const std::uint32_t* __restrict__ chunks, const std::uint32_t* __restrict__ seqs,
    const float* __restrict__ Tm, const float* __restrict__ Pm, const float* __restrict__ Gc,
    float* __restrict__ state, float* __restrict__ o, std::uint32_t Hv, std::uint32_t Hk) {
  ChunkScan(q, k, v, beta, chunks, seqs, Tm, Pm, Gc, state, o, Hv, Hk);
}

// ---- the whole DeltaNet token step of the decode graph, one block per (session, value head) -----------------
// Fuses the prologue (causal conv + SiLU, q / k L2 norms, decay and beta gates), the delta-rule recurrence and the
// output RMSNorm * w * sigmoid(z) with its Q8 quantization for the output projection (reference
// ReferenceModel::LinearAttention, src/model/reference.cpp:278-366). The conv history is a ring of K slots per
// channel: position p's projection lives in slot p % K, so step p reads slots (p + 1 + j) % K (j < K - 1) and writes
// slot p % K, which no block of the same step reads; q / k channels of key head kh are read by every value head with
// h % Hk == kh but written only by value head h = kh (h < Hk), v channels by their own head. Positions: nkv[s] - 1.
//   qkv [S][C] (C = 2 Hk d + Hv d), z [S][Hv d], ab [S][2 Hv] (alpha | beta logits), ring [S][K][C], conv_w [C][K],
//   a, dt [Hv], norm_w [d], state [S][Hv][d][d] key-major fp32 (in place) -> oq [S][Hv d] int8, os [S][Hv d / 32].
// grid (S * Hv), block 512: thread t owns state rows 8 (t / 32) .. + 8 and columns 4 (t % 32) .. + 4. d = 128.
extern "C" __global__ void __launch_bounds__(512) halo_gdn_step_q8(
    const float* __restrict__ qkv, const float* __restrict__ z, const float* __restrict__ ab, float* __restrict__ ring,
    const float* __restrict__ conv_w, const float* __restrict__ a, const float* __restrict__ dt,
    const float* __restrict__ norm_w, float* __restrict__ state, const std::uint32_t* __restrict__ nkv,
    std::int8_t* __restrict__ oq, float* __restrict__ os, std::uint32_t Hk, std::uint32_t Hv, std::uint32_t K,
    float eps) {
  __shared__ float sq[kD], sk[kD], sv[kD], dl[kD];
  __shared__ float red[16][kD + 4];
  __shared__ float part[8];
  __shared__ float gates[2];
  const std::uint32_t s = blockIdx.x / Hv, h = blockIdx.x % Hv, kh = h % Hk;
  const std::uint32_t t = threadIdx.x, wave = t / kWave, lane = t % kWave;
  const std::uint32_t cg = t % 32, rg = t / 32, j0 = 4 * cg, i0 = 8 * rg;
  const std::uint32_t Dk = Hk * kD, Dv = Hv * kD, C = 2 * Dk + Dv;
  float* St = state + (static_cast<std::size_t>(s) * Hv + h) * kD * kD;
  // the head's state first (64 KB per block, eight 16-byte loads per thread)
  float4 row[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) row[r] = *reinterpret_cast<const float4*>(St + static_cast<std::size_t>(i0 + r) * kD + j0);
  // prologue: threads 0..383 take the q, k and v channels of this head (128 each: waves 0-1, 2-3, 4-5)
  const std::uint32_t pos = nkv[s] - 1;
  const std::uint32_t seg = t / kD, i = t % kD;
  float y = 0.0f;
  if (seg < 3) {
    const std::uint32_t ch = seg == 0 ? kh * kD + i : seg == 1 ? Dk + kh * kD + i : 2 * Dk + h * kD + i;
    const float x = qkv[static_cast<std::size_t>(s) * C + ch];
    float* rs = ring + static_cast<std::size_t>(s) * K * C;
    float acc = conv_w[static_cast<std::size_t>(ch) * K + K - 1] * x;
    for (std::uint32_t j = 0; j + 1 < K; ++j)
      acc += conv_w[static_cast<std::size_t>(ch) * K + j] * rs[static_cast<std::size_t>((pos + 1 + j) % K) * C + ch];
    if (seg == 2 || h < Hk) rs[static_cast<std::size_t>(pos % K) * C + ch] = x;
    y = halo::Silu(acc);
  }
  const float ss = halo::GroupSum(y * y);
  if (lane == 0) part[wave] = ss;
  if (t == 0) {
    gates[0] = a[h] * halo::Softplus(ab[static_cast<std::size_t>(s) * 2 * Hv + h] + dt[h]);
    gates[1] = halo::Sigmoid(ab[static_cast<std::size_t>(s) * 2 * Hv + Hv + h]);
  }
  __syncthreads();
  if (seg < 2) {
    const float sc = 1.0f / sqrtf(part[2 * seg] + part[2 * seg + 1] + eps);
    (seg == 0 ? sq : sk)[i] = y * sc;
  } else if (seg == 2) {
    sv[i] = y;
  }
  __syncthreads();
  // recurrence: u = (decay S)^T k, delta = (v - u) beta, S <- decay S + k delta^T, o = S^T q / sqrt(d)
  const float decay = expf(gates[0]), bt = gates[1];
  float u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const float ki = sk[i0 + r];
    row[r].x *= decay;
    row[r].y *= decay;
    row[r].z *= decay;
    row[r].w *= decay;
    u[0] += row[r].x * ki;
    u[1] += row[r].y * ki;
    u[2] += row[r].z * ki;
    u[3] += row[r].w * ki;
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) red[rg][j0 + c] = u[c];
  __syncthreads();
  if (t < kD) {
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc += red[r][t];
    dl[t] = (sv[t] - acc) * bt;
  }
  __syncthreads();
  const float d0 = dl[j0], d1 = dl[j0 + 1], d2 = dl[j0 + 2], d3 = dl[j0 + 3];
  float oo[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const float ki = sk[i0 + r], qi = sq[i0 + r];
    row[r].x += ki * d0;
    row[r].y += ki * d1;
    row[r].z += ki * d2;
    row[r].w += ki * d3;
    oo[0] += row[r].x * qi;
    oo[1] += row[r].y * qi;
    oo[2] += row[r].z * qi;
    oo[3] += row[r].w * qi;
    *reinterpret_cast<float4*>(St + static_cast<std::size_t>(i0 + r) * kD + j0) = row[r];
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) red[rg][j0 + c] = oo[c];
  __syncthreads();
  // output: RMSNorm over the head's 128 values * w * sigmoid(z), quantized per 32 (waves 0 and 1)
  float o = 0.0f;
  if (t < kD) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o += red[r][t];
    o *= 1.0f / sqrtf(static_cast<float>(kD));
  }
  const float so = halo::GroupSum(o * o);
  if (lane == 0 && wave < 2) part[wave] = so;
  __syncthreads();
  if (t < kD) {
    const float sc = 1.0f / sqrtf((part[0] + part[1]) / static_cast<float>(kD) + eps);
    const std::size_t off = static_cast<std::size_t>(s) * Dv + h * kD + t;
    const float v = o * sc * norm_w[t] * halo::Sigmoid(z[off]);
    const float amax = halo::GroupMax<32>(fabsf(v));
    const float scale = amax / 127.0f;
    oq[off] = static_cast<std::int8_t>(scale > 0.0f ? static_cast<int>(rintf(v / scale)) : 0);
    if (t % 32 == 0) os[off / 32] = scale;
  }
}
