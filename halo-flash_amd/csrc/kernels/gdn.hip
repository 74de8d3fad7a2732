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

// ---- chunked prefill (C = 64) over a ragged batch of sequences, on fp32 MFMA -----------------------------------
// Within a chunk of C tokens with cumulative log-decay G_t (gamma_t = exp(G_t)) and initial state S0, the token
// recurrence above is exactly (reference math comment src/kernels/core.hip:6035-6048, there with C = 16):
//   (I + A) Delta = diag(beta) V - diag(beta gamma) K S0,   A[t][s] = beta_t exp(G_t - G_s) (k_t . k_s), s < t
//   O = (diag(gamma) Q S0 + P Delta) / sqrt(d),             P[t][s] = exp(G_t - G_s) (q_t . k_s),         s <= t
//   S_C = gamma_C S0 + K^T diag(exp(G_C - G_s)) Delta.
// With T = (I + A)^-1 this splits into what does not depend on the state (WY form, computed for every chunk in
// parallel by halo_gdn_wy_prep):
//   Uk = T diag(beta gamma) K,  Wv = T diag(beta) V,  Qe = diag(gamma) Q - P Uk,  Ov = P Wv      (64 x 128 each)
// and the chunk-serial part (halo_gdn_wy_scan), three products per chunk:
//   Delta = Wv - Uk S0,  O = (Qe S0 + Ov) / sqrt(d),  S_C = gamma_C S0 + K^T diag(exp(G_C - G_s)) Delta.
// Tokens past a partial chunk's end are zero-padded (k = q = v = 0, beta = 0, g = 0): their rows of every product are
// zero. Inputs q, k [tokens][Hk][128] and v [tokens][Hv][128] are bf16 (the C3 operator) or fp32 (the model's
// prefill, which matches its decode step); g, beta [tokens][Hv] fp32 (g = log decay, beta after its sigmoid); state
// fp32 [seq][Hv][128][128] key-major. chunks [n][3] = {first token, length, sequence}; seqs [n_seq][2] = {first
// chunk, chunk count}. Workspace per (chunk, head): Uk, Qe, Wv, Ov fp32 [64][128] and G [64].
namespace {
constexpr int kC = 64;
constexpr int kCL = 132;  // LDS row stride (floats) of a 64 x 128 tile
constexpr int kPL = 68;   // of a 64 x 64 tile
typedef float V16F __attribute__((ext_vector_type(16)));
typedef float V4F __attribute__((ext_vector_type(4)));

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
// row r of a 64 x 128 LDS tile from 8 inputs: two float4 stores, zeros when !on
template <typename In>
__device__ __forceinline__ void Put8(float* dst, const Pack8<In>& x, bool on) {
  float f[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = on ? Cv(x.v[e]) : 0.0f;
  reinterpret_cast<float4*>(dst)[0] = make_float4(f[0], f[1], f[2], f[3]);
  reinterpret_cast<float4*>(dst)[1] = make_float4(f[4], f[5], f[6], f[7]);
}
}  // namespace

// grid (n_chunks, Hv), block 256 (4 waves). MFMA v_mfma_f32_32x32x2f32: A lane l = A[l % 32][k], B lane l =
// B[k][l % 32] with k split in halves (lanes 0-31 the first half of the K range, 32-63 the second), D lane l holds
// column l % 32 and rows 8 (r / 4) + 4 (l / 32) + r % 4. Wave w owns the 32 x 32 tile (w / 2, w % 2) of K K^T and
// of Q K^T, then two 32-column tiles of each 64 x 128 product. T = (I + A)^-1 by forward substitution in wave 0,
// one column per lane, in registers.
template <typename In>
__device__ __forceinline__ void WyPrep(const In* __restrict__ q, const In* __restrict__ k, const In* __restrict__ v,
                                       const float* __restrict__ g, const float* __restrict__ beta,
                                       const std::uint32_t* __restrict__ chunks, float* __restrict__ wy,
                                       float* __restrict__ Gc, std::uint32_t Hv, std::uint32_t Hk) {
  __shared__ __attribute__((aligned(16))) float kl[kC][kCL];
  __shared__ __attribute__((aligned(16))) float ql[kC][kCL];
  __shared__ __attribute__((aligned(16))) float vl[kC][kCL];
  __shared__ __attribute__((aligned(16))) float am[kC][kPL];  // A, then T
  __shared__ __attribute__((aligned(16))) float pm[kC][kPL];
  __shared__ float G[kC], Bt[kC], Bg[kC], Gm[kC];
  const std::uint32_t c = blockIdx.x, h = blockIdx.y, kh = h % Hk, tid = threadIdx.x;
  const std::uint32_t wave = tid / kWave, lane = tid % kWave, fr = lane % 32, hh = lane / 32;
  const std::uint32_t start = chunks[c * 3], L = chunks[c * 3 + 1];
  for (std::uint32_t idx = tid; idx < kC * (kD / 8); idx += blockDim.x) {
    const std::uint32_t t = idx / (kD / 8), p = idx % (kD / 8), tt = min(t, L - 1);
    const bool on = t < L;
    const std::size_t kq = (static_cast<std::size_t>(start + tt) * Hk + kh) * kD + p * 8;
    const std::size_t vv = (static_cast<std::size_t>(start + tt) * Hv + h) * kD + p * 8;
    Put8(&kl[t][p * 8], Ld8(k + kq), on);
    Put8(&ql[t][p * 8], Ld8(q + kq), on);
    Put8(&vl[t][p * 8], Ld8(v + vv), on);
  }
  if (tid < kC) {
    const std::uint32_t tt = min(tid, L - 1);
    const bool on = tid < L;
    const float gv = g[static_cast<std::size_t>(start + tt) * Hv + h], bv = beta[static_cast<std::size_t>(start + tt) * Hv + h];
    G[tid] = on ? gv : 0.0f;
    Bt[tid] = on ? bv : 0.0f;
  }
  __syncthreads();
  if (tid == 0)
    for (int t = 1; t < kC; ++t) G[t] += G[t - 1];
  __syncthreads();
  if (tid < kC) {
    Gm[tid] = expf(G[tid]);
    Bg[tid] = Bt[tid] * expf(G[tid]);
  }
  // K K^T and Q K^T, tile (ti, tj) = (wave / 2, wave % 2), K range = 128 keys (step s: key s + 64 hh)
  const std::uint32_t ti = wave / 2, tj = wave % 2;
  V16F kk = {}, qk = {};
#pragma unroll 4
  for (int sb = 0; sb < 16; ++sb) {
    const float4 ka = *reinterpret_cast<const float4*>(&kl[32 * ti + fr][4 * sb + 64 * hh]);
    const float4 qa = *reinterpret_cast<const float4*>(&ql[32 * ti + fr][4 * sb + 64 * hh]);
    const float4 kb = *reinterpret_cast<const float4*>(&kl[32 * tj + fr][4 * sb + 64 * hh]);
    kk = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.x, kb.x, kk, 0, 0, 0);
    qk = __builtin_amdgcn_mfma_f32_32x32x2f32(qa.x, kb.x, qk, 0, 0, 0);
    kk = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.y, kb.y, kk, 0, 0, 0);
    qk = __builtin_amdgcn_mfma_f32_32x32x2f32(qa.y, kb.y, qk, 0, 0, 0);
    kk = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.z, kb.z, kk, 0, 0, 0);
    qk = __builtin_amdgcn_mfma_f32_32x32x2f32(qa.z, kb.z, qk, 0, 0, 0);
    kk = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.w, kb.w, kk, 0, 0, 0);
    qk = __builtin_amdgcn_mfma_f32_32x32x2f32(qa.w, kb.w, qk, 0, 0, 0);
  }
  __syncthreads();  // Gm / Bg visible
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const std::uint32_t t = 32 * ti + 8 * (r / 4) + 4 * hh + r % 4, s = 32 * tj + fr;
    const bool low = s < t, leq = s <= t;
    const float dec = expf(leq ? G[t] - G[s] : 0.0f);
    am[t][s] = low ? Bt[t] * dec * kk[r] : 0.0f;
    pm[t][s] = leq ? dec * qk[r] : 0.0f;
  }
  __syncthreads();
  // T = (I + A)^-1: lane = column, rows in order; A rows are read as broadcasts, four partial sums per row
  if (wave == 0) {
    float T[kC];
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s4 = 0; s4 < t; s4 += 4) {
        const float4 ar = *reinterpret_cast<const float4*>(&am[t][s4]);
        const float av[4] = {ar.x, ar.y, ar.z, ar.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (s4 + e < t) acc[e] = __builtin_fmaf(av[e], T[s4 + e], acc[e]);
      }
      const float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
      T[t] = lane == static_cast<std::uint32_t>(t) ? 1.0f : -sum;
    }
    // every lane has read all of A above (program order within the wave); T replaces it
#pragma unroll
    for (int t = 0; t < kC; ++t) am[t][lane] = T[t];
  }
  __syncthreads();
  // Uk = T diag(beta gamma) K and Wv = T diag(beta) V: wave w owns rows 32 ti, columns 32 (2 (w % 2) + u), u < 2;
  // K range = 64 tokens (step s: token s + 32 hh)
  float* out = wy + (static_cast<std::size_t>(c) * Hv + h) * 4 * kC * kD;  // Uk, Qe, Wv, Ov
  V16F uk[2] = {{}, {}}, wv[2] = {{}, {}};
#pragma unroll 2
  for (int sb = 0; sb < 8; ++sb) {
    const float4 ta = *reinterpret_cast<const float4*>(&am[32 * ti + fr][4 * sb + 32 * hh]);
    const float tv[4] = {ta.x, ta.y, ta.z, ta.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const std::uint32_t tok = 4 * sb + e + 32 * hh;
      const float bg = Bg[tok], bt = Bt[tok];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const std::uint32_t col = 32 * (2 * tj + u) + fr;
        uk[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(tv[e], bg * kl[tok][col], uk[u], 0, 0, 0);
        wv[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(tv[e], bt * vl[tok][col], wv[u], 0, 0, 0);
      }
    }
  }
  __syncthreads();  // K and V are no longer read: Uk and Wv take their places
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const std::uint32_t t = 32 * ti + 8 * (r / 4) + 4 * hh + r % 4, col = 32 * (2 * tj + u) + fr;
      kl[t][col] = uk[u][r];
      vl[t][col] = wv[u][r];
      out[0 * kC * kD + t * kD + col] = uk[u][r];
      out[2 * kC * kD + t * kD + col] = wv[u][r];
    }
  __syncthreads();
  // Qe = diag(gamma) Q - P Uk and Ov = P Wv
  V16F qe[2], ov[2] = {{}, {}};
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const std::uint32_t t = 32 * ti + 8 * (r / 4) + 4 * hh + r % 4, col = 32 * (2 * tj + u) + fr;
      qe[u][r] = Gm[t] * ql[t][col];
    }
#pragma unroll 2
  for (int sb = 0; sb < 8; ++sb) {
    const float4 pa = *reinterpret_cast<const float4*>(&pm[32 * ti + fr][4 * sb + 32 * hh]);
    const float pv[4] = {pa.x, pa.y, pa.z, pa.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const std::uint32_t tok = 4 * sb + e + 32 * hh;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const std::uint32_t col = 32 * (2 * tj + u) + fr;
        qe[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(-pv[e], kl[tok][col], qe[u], 0, 0, 0);
        ov[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(pv[e], vl[tok][col], ov[u], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const std::uint32_t t = 32 * ti + 8 * (r / 4) + 4 * hh + r % 4, col = 32 * (2 * tj + u) + fr;
      out[1 * kC * kD + t * kD + col] = qe[u][r];
      out[3 * kC * kD + t * kD + col] = ov[u][r];
    }
  if (tid < kC) Gc[(static_cast<std::size_t>(c) * Hv + h) * kC + tid] = G[tid];
}

// grid (n_seq * Hv * 8), block 512 (8 waves): block -> (sequence, head, 16 value columns [16 cb, 16 cb + 16)); walks
// the sequence's chunks carrying its 128 x 16 slice of S in LDS. MFMA v_mfma_f32_16x16x4f32: A lane l = A[l % 16][k],
// B lane l = B[k][l % 16] with k = 4 s + l / 16 at step s, D lane l holds column l % 16 and rows 4 (l / 16) + r.
// Per chunk: waves 0-3 form Delta rows 16 w .. + 16 (= Wv - Uk S0), waves 4-7 the output rows (Qe S0 + Ov); then
// wave w updates S rows 16 w .. + 16. The next chunk's operands are loaded into registers during the current one.
template <typename In>
__device__ __forceinline__ void WyScan(const In* __restrict__ k, const float* __restrict__ wy,
                                       const float* __restrict__ Gc, const std::uint32_t* __restrict__ chunks,
                                       const std::uint32_t* __restrict__ seqs, float* __restrict__ state,
                                       float* __restrict__ o, std::uint32_t Hv, std::uint32_t Hk) {
  constexpr int kNC = 16, kSL = 20;
  __shared__ __attribute__((aligned(16))) float ukl[kC][kCL];
  __shared__ __attribute__((aligned(16))) float qel[kC][kCL];
  __shared__ __attribute__((aligned(16))) float kxl[kC][kCL];
  __shared__ __attribute__((aligned(16))) float wvl[kC][kSL];
  __shared__ __attribute__((aligned(16))) float ovl[kC][kSL];
  __shared__ __attribute__((aligned(16))) float Sl[kD][kSL];
  __shared__ __attribute__((aligned(16))) float Dl[kC][kSL];
  __shared__ float Gl[kC];
  const std::uint32_t b = blockIdx.x, cb = b % 8, h = (b / 8) % Hv, sq = b / (8 * Hv), kh = h % Hk;
  const std::uint32_t tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, fc = lane % 16, fq = lane / 16;
  const std::uint32_t j0 = cb * kNC;
  const std::uint32_t c0 = seqs[sq * 2], nc = seqs[sq * 2 + 1];
  float* St = state + (static_cast<std::size_t>(sq) * Hv + h) * kD * kD;
  // S slice: 128 rows x 16 columns = 512 float4, one per thread
  {
    const std::uint32_t r = tid / 4, p = tid % 4;
    *reinterpret_cast<float4*>(&Sl[r][4 * p]) = *reinterpret_cast<const float4*>(St + static_cast<std::size_t>(r) * kD + j0 + 4 * p);
  }
  // staged operands of one chunk, in registers: Uk, Qe (8192 floats each: 4 float4 per thread), K (8192 inputs: two
  // packs of 8), the Wv or Ov slice (64 x 16: threads < 256 Wv, the rest Ov, one float4 each) and G (threads < 64)
  float4 ru0, ru1, ru2, ru3, rq0, rq1, rq2, rq3, rwo;
  Pack8<In> rk0, rk1;
  float rg;
  auto load = [&](std::uint32_t c) {
    const float4* bu = reinterpret_cast<const float4*>(wy + (static_cast<std::size_t>(c) * Hv + h) * 4 * kC * kD);
    const float4* bq = bu + kC * kD / 4;
    ru0 = bu[tid], ru1 = bu[tid + 512], ru2 = bu[tid + 1024], ru3 = bu[tid + 1536];
    rq0 = bq[tid], rq1 = bq[tid + 512], rq2 = bq[tid + 1024], rq3 = bq[tid + 1536];
    const std::uint32_t start = chunks[c * 3], L = chunks[c * 3 + 1];
    const std::uint32_t t0 = tid / 16, p8 = 8 * (tid % 16);  // packs tid and tid + 512: rows t0 and t0 + 32
    rk0 = Ld8(k + (static_cast<std::size_t>(start + min(t0, L - 1)) * Hk + kh) * kD + p8);
    rk1 = Ld8(k + (static_cast<std::size_t>(start + min(t0 + 32, L - 1)) * Hk + kh) * kD + p8);
    const std::uint32_t e = tid % 256;
    const float* src = reinterpret_cast<const float*>(bu) + (tid < 256 ? 2 : 3) * kC * kD;
    rwo = *reinterpret_cast<const float4*>(src + (e / 4) * kD + j0 + 4 * (e % 4));
    rg = Gc[(static_cast<std::size_t>(c) * Hv + h) * kC + tid % kC];
  };
  auto store = [&](std::uint32_t c) {
    const std::uint32_t L = chunks[c * 3 + 1];
    // float4 e = tid + 512 i of a 64 x 128 tile is row e / 32 = tid / 32 + 16 i, column 4 (tid % 32)
    const std::uint32_t t0 = tid / 32, p4 = 4 * (tid % 32);
    *reinterpret_cast<float4*>(&ukl[t0][p4]) = ru0;
    *reinterpret_cast<float4*>(&ukl[t0 + 16][p4]) = ru1;
    *reinterpret_cast<float4*>(&ukl[t0 + 32][p4]) = ru2;
    *reinterpret_cast<float4*>(&ukl[t0 + 48][p4]) = ru3;
    *reinterpret_cast<float4*>(&qel[t0][p4]) = rq0;
    *reinterpret_cast<float4*>(&qel[t0 + 16][p4]) = rq1;
    *reinterpret_cast<float4*>(&qel[t0 + 32][p4]) = rq2;
    *reinterpret_cast<float4*>(&qel[t0 + 48][p4]) = rq3;
    const std::uint32_t tk = tid / 16, pk = 8 * (tid % 16);
    Put8(&kxl[tk][pk], rk0, tk < L);
    Put8(&kxl[tk + 32][pk], rk1, tk + 32 < L);
    const std::uint32_t e = tid % 256;
    float(*dst)[kSL] = tid < 256 ? wvl : ovl;
    *reinterpret_cast<float4*>(&dst[e / 4][4 * (e % 4)]) = rwo;
    if (tid < kC) Gl[tid] = rg;
  };
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(kD));
  // one register set: chunk ci's operands go to LDS, then chunk ci + 1's loads are in flight during ci's products
  if (nc > 0) load(c0);
  for (std::uint32_t ci = 0; ci < nc; ++ci) {
    const std::uint32_t c = c0 + ci, start = chunks[c * 3], L = chunks[c * 3 + 1];
    store(c);
    __syncthreads();
    load(ci + 1 < nc ? c + 1 : c);  // unconditional (the last chunk reloads itself): no loads under a branch
    // Delta (waves 0-3) or the output (waves 4-7): rows 16 (w % 4) .. + 16, K range = 128 keys
    {
      const std::uint32_t r0 = 16 * (wave % 4);
      float(*A)[kCL] = wave < 4 ? ukl : qel;
      V4F acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
      for (int s = 0; s < kD / 4; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[r0 + fc][4 * s + fq], Sl[4 * s + fq][fc], acc, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const std::uint32_t t = r0 + 4 * fq + i;
        if (wave < 4) {
          Dl[t][fc] = wvl[t][fc] - acc[i];
        } else if (t < L) {
          o[(static_cast<std::size_t>(start + t) * Hv + h) * kD + j0 + fc] = (acc[i] + ovl[t][fc]) * inv_sqrt_d;
        }
      }
    }
    __syncthreads();
    // S rows 16 w .. + 16: gamma_C S + (K diag(exp(G_C - G_t)))^T Delta, K range = 64 tokens
    {
      const std::uint32_t r0 = 16 * wave;
      const float GC = Gl[kC - 1], gc = expf(GC);
      V4F acc;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = gc * Sl[r0 + 4 * fq + i][fc];
#pragma unroll 4
      for (int s = 0; s < kC / 4; ++s) {
        const std::uint32_t tok = 4 * s + fq;
        const float a = kxl[tok][r0 + fc] * expf(GC - Gl[tok]);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, Dl[tok][fc], acc, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) Sl[r0 + 4 * fq + i][fc] = acc[i];
    }
    __syncthreads();
  }
  {
    const std::uint32_t r = tid / 4, p = tid % 4;
    *reinterpret_cast<float4*>(St + static_cast<std::size_t>(r) * kD + j0 + 4 * p) = *reinterpret_cast<const float4*>(&Sl[r][4 * p]);
  }
}

extern "C" __global__ void __launch_bounds__(256)
    halo_gdn_wy_prep(const std::uint16_t* __restrict__ q, const std::uint16_t* __restrict__ k,
                     const std::uint16_t* __restrict__ v, const float* __restrict__ g, const float* __restrict__ beta,
                     const std::uint32_t* __restrict__ chunks, float* __restrict__ wy, float* __restrict__ Gc,
                     std::uint32_t Hv, std::uint32_t Hk) {
  WyPrep(q, k, v, g, beta, chunks, wy, Gc, Hv, Hk);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_gdn_wy_prep_f32(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                         const float* __restrict__ g, const float* __restrict__ beta,
                         const std::uint32_t* __restrict__ chunks, float* __restrict__ wy, float* __restrict__ Gc,
                         std::uint32_t Hv, std::uint32_t Hk) {
  WyPrep(q, k, v, g, beta, chunks, wy, Gc, Hv, Hk);
}
extern "C" __global__ void __launch_bounds__(512)
    halo_gdn_wy_scan(const std::uint16_t* __restrict__ k, const float* __restrict__ wy, const float* __restrict__ Gc,
                     const std::uint32_t* __restrict__ chunks, const std::uint32_t* __restrict__ seqs,
                     float* __restrict__ state, float* __restrict__ o, std::uint32_t Hv, std::uint32_t Hk) {
  WyScan(k, wy, Gc, chunks, seqs, state, o, Hv, Hk);
}
extern "C" __global__ void __launch_bounds__(512)
    halo_gdn_wy_scan_f32(const float* __restrict__ k, const float* __restrict__ wy, const float* __restrict__ Gc,
                         const std::uint32_t* __restrict__ chunks, const std::uint32_t* __restrict__ seqs,
                         float* __restrict__ state, float* __restrict__ o, std::uint32_t Hv, std::uint32_t Hk) {
  WyScan(k, wy, Gc, chunks, seqs, state, o, Hv, Hk);
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
