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

// grid (n_chunks, Hv), block 512 (8 waves). MFMA v_mfma_f32_32x32x2f32: A lane l = A[l % 32][k], B lane l =
// B[k][l % 32] with k split in halves (lanes 0-31 the first half of the K range, 32-63 the second), D lane l holds
// column l % 32 and rows 8 (r / 4) + 4 (l / 32) + r % 4. Wave w owns the 32 x 32 tile ((w % 4) / 2, w % 2) of K K^T
// (w < 4) or Q K^T (w >= 4), then the 32-column tile 2 (w % 2) + w / 4 of each 64 x 128 product. T = (I + A)^-1 by
// forward substitution in wave 0, one column per lane, in registers.
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
  if (tid == 0) {  // running sum in a register: the loads are independent, only the adds form a chain
    float run = G[0];
#pragma unroll
    for (int t = 1; t < kC; ++t) {
      run += G[t];
      G[t] = run;
    }
  }
  __syncthreads();
  if (tid < kC) {
    Gm[tid] = expf(G[tid]);
    Bg[tid] = Bt[tid] * expf(G[tid]);
  }
  // K K^T (waves 0-3) and Q K^T (waves 4-7), tile (ti, tj) = ((wave % 4) / 2, wave % 2), K range = 128 keys
  // (step s: key s + 64 hh); eight waves, two per SIMD, so one wave's MFMA chain overlaps another's loads and stores
  const std::uint32_t w4 = wave % 4, ti = w4 / 2, tj = w4 % 2, half = wave / 4;
  float(*xa)[kCL] = half ? ql : kl;
  V16F kq = {};
#pragma unroll 4
  for (int sb = 0; sb < 16; ++sb) {
    const float4 xa4 = *reinterpret_cast<const float4*>(&xa[32 * ti + fr][4 * sb + 64 * hh]);
    const float4 kb = *reinterpret_cast<const float4*>(&kl[32 * tj + fr][4 * sb + 64 * hh]);
    kq = __builtin_amdgcn_mfma_f32_32x32x2f32(xa4.x, kb.x, kq, 0, 0, 0);
    kq = __builtin_amdgcn_mfma_f32_32x32x2f32(xa4.y, kb.y, kq, 0, 0, 0);
    kq = __builtin_amdgcn_mfma_f32_32x32x2f32(xa4.z, kb.z, kq, 0, 0, 0);
    kq = __builtin_amdgcn_mfma_f32_32x32x2f32(xa4.w, kb.w, kq, 0, 0, 0);
  }
  __syncthreads();  // Gm / Bg visible
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const std::uint32_t t = 32 * ti + 8 * (r / 4) + 4 * hh + r % 4, s = 32 * tj + fr;
    const bool low = s < t, leq = s <= t;
    const float dec = expf(leq ? G[t] - G[s] : 0.0f);
    if (half)
      pm[t][s] = leq ? dec * kq[r] : 0.0f;
    else
      am[t][s] = low ? Bt[t] * dec * kq[r] : 0.0f;
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
  // Uk = T diag(beta gamma) K and Wv = T diag(beta) V: wave w owns rows 32 ti, columns 32 (2 (w % 2) + w / 4);
  // K range = 64 tokens (step s: token s + 32 hh)
  float* out = wy + (static_cast<std::size_t>(c) * Hv + h) * 4 * kC * kD;  // Uk, Qe, Wv, Ov
  const std::uint32_t col = 32 * (2 * tj + half) + fr;
  V16F uk = {}, wv = {};
#pragma unroll 2
  for (int sb = 0; sb < 8; ++sb) {
    const float4 ta = *reinterpret_cast<const float4*>(&am[32 * ti + fr][4 * sb + 32 * hh]);
    const float tv[4] = {ta.x, ta.y, ta.z, ta.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const std::uint32_t tok = 4 * sb + e + 32 * hh;
      uk = __builtin_amdgcn_mfma_f32_32x32x2f32(tv[e], Bg[tok] * kl[tok][col], uk, 0, 0, 0);
      wv = __builtin_amdgcn_mfma_f32_32x32x2f32(tv[e], Bt[tok] * vl[tok][col], wv, 0, 0, 0);
    }
  }
  __syncthreads();  // K and V are no longer read: Uk and Wv take their places
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const std::uint32_t t = 32 * ti + 8 * (r / 4) + 4 * hh + r % 4;
    kl[t][col] = uk[r];
    vl[t][col] = wv[r];
    out[0 * kC * kD + t * kD + col] = uk[r];
    out[2 * kC * kD + t * kD + col] = wv[r];
  }
  __syncthreads();
  // Qe = diag(gamma) Q - P Uk and Ov = P Wv
  V16F qe, ov = {};
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const std::uint32_t t = 32 * ti + 8 * (r / 4) + 4 * hh + r % 4;
    qe[r] = Gm[t] * ql[t][col];
  }
#pragma unroll 2
  for (int sb = 0; sb < 8; ++sb) {
    const float4 pa = *reinterpret_cast<const float4*>(&pm[32 * ti + fr][4 * sb + 32 * hh]);
    const float pv[4] = {pa.x, pa.y, pa.z, pa.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const std::uint32_t tok = 4 * sb + e + 32 * hh;
      qe = __builtin_amdgcn_mfma_f32_32x32x2f32(-pv[e], kl[tok][col], qe, 0, 0, 0);
      ov = __builtin_amdgcn_mfma_f32_32x32x2f32(pv[e], vl[tok][col], ov, 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const std::uint32_t t = 32 * ti + 8 * (r / 4) + 4 * hh + r % 4;
    out[1 * kC * kD + t * kD + col] = qe[r];
    out[3 * kC * kD + t * kD + col] = ov[r];
  }
  if (tid < kC) Gc[(static_cast<std::size_t>(c) * Hv + h) * kC + tid] = G[tid];
}

// grid (n_seq * Hv * 128 / kNC), block 512 (8 waves): block -> (sequence, head, kNC value columns); walks
// the sequence's chunks carrying its 128 x kNC slice of S in LDS. kNC = 32 (four blocks per head): each chunk's Uk,
// Qe and K are read by four blocks (measured on C3: 16 columns per block 910 us, 32 878 us, 64 1339 us; narrower
// slices re-read more, wider ones leave fewer waves per head for the chunk-serial MFMA work).
// MFMA v_mfma_f32_16x16x4f32 (A lane l = A[l % 16][k], B lane l = B[k][l % 16], D lane l holds column l % 16 and
// rows 4 (l / 16) + r) with each lane's k contiguous: lane quarter fq takes k in [K/4 fq, K/4 (fq + 1)), so every
// operand read is 16 bytes (4 steps); a wave's four column tiles are four independent accumulator chains. The LDS
// tiles that serve as B or as a transposed A are stored transposed: S as st[column][key], Delta as dt[column][token],
// K as kt[key][token] (kt reuses Uk's space once Uk has been read).
// Per chunk: waves 0-3 form Delta rows 16 w .. + 16 (= Wv - Uk S0), waves 4-7 the output rows (Qe S0 + Ov), four
// 16-column tiles each; then wave w updates S rows 16 w .. + 16. The next chunk's operands are loaded into registers
// during the current one; the block barriers inside the chunk loop synchronize LDS only, so those loads stay in
// flight across them.
// Column of token `tok` in row `key` of the K^T tile: 4-token groups xor-swizzled by (key / 8) & 15. With the 72-float
// row stride, both the transposed 4-byte stores (64 lanes: 16 key rows x 4 tokens) and the 16-byte operand reads (16
// key rows, one 4-token group) land on distinct banks of the 64-bank LDS.
__device__ __forceinline__ std::uint32_t KtCol(std::uint32_t key, std::uint32_t tok) {
  return 4 * ((tok / 4) ^ ((key / 8) & 15)) + tok % 4;
}

template <typename In, int kNC>
__device__ __forceinline__ void WyScan(const In* __restrict__ k, const float* __restrict__ wy,
                                       const float* __restrict__ Gc, const std::uint32_t* __restrict__ chunks,
                                       const std::uint32_t* __restrict__ seqs, float* __restrict__ state,
                                       float* __restrict__ o, std::uint32_t Hv, std::uint32_t Hk) {
  constexpr int kNB = kD / kNC, kNT = kNC / 16, kTL = kC + 8, kDL = kC + 4, kStL = kD + 4, kWL = kNC + 4;
  constexpr int kUkF = kC * kCL, kKtF = kD * kTL, kAF = kUkF > kKtF ? kUkF : kKtF;
  __shared__ __attribute__((aligned(16))) float ua[kAF];       // Uk [64][kCL], then K^T [128][kTL]
  __shared__ __attribute__((aligned(16))) float qel[kC][kCL];
  __shared__ __attribute__((aligned(16))) float st[kNC][kStL];  // S^T slice: [column][key]
  __shared__ __attribute__((aligned(16))) float dt[kNC][kDL];   // Delta^T slice: [column][token]
  __shared__ __attribute__((aligned(16))) float wvl[kC][kWL];
  __shared__ __attribute__((aligned(16))) float ovl[kC][kWL];
  __shared__ __attribute__((aligned(16))) float Gl[kC], Wl[kC];
  float(*ukl)[kCL] = reinterpret_cast<float(*)[kCL]>(ua);
  float(*kt)[kTL] = reinterpret_cast<float(*)[kTL]>(ua);
  // Blocks are dispatched in id order and a block's LDS leaves room for one per CU, so the longest sequences take
  // the lowest ids (rank by descending chunk count, ties by index; up to 64 sequences, else in order): the chunk-
  // serial critical path starts first.
  __shared__ std::uint32_t sq_s;
  const std::uint32_t b = blockIdx.x, cb = b % kNB, h = (b / kNB) % Hv, rank = b / (kNB * Hv);
  const std::uint32_t n_seq = gridDim.x / (kNB * Hv);
  if (threadIdx.x == 0) {
    std::uint32_t pick = rank;
    if (n_seq <= 64) {
      for (std::uint32_t j = 0; j < n_seq; ++j) {
        const std::uint32_t cj = seqs[j * 2 + 1];
        std::uint32_t r = 0;
        for (std::uint32_t i = 0; i < n_seq; ++i) {
          const std::uint32_t ci = seqs[i * 2 + 1];
          r += (ci > cj) || (ci == cj && i < j);
        }
        if (r == rank) pick = j;
      }
    }
    sq_s = pick;
  }
  __syncthreads();
  const std::uint32_t sq = sq_s, kh = h % Hk;
  const std::uint32_t tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave, fc = lane % 16, fq = lane / 16;
  const std::uint32_t j0 = cb * kNC;
  const std::uint32_t c0 = seqs[sq * 2], nc = seqs[sq * 2 + 1];
  // a sequence's chunks are consecutive 64-token runs: chunk ci starts at first + 64 ci and holds
  // min(64, len - 64 ci) tokens (no chunk-table read per chunk: those scalar loads sat on the serial path)
  const std::uint32_t first = nc ? chunks[c0 * 3] : 0u;
  const std::uint32_t len = nc ? chunks[(c0 + nc - 1) * 3] + chunks[(c0 + nc - 1) * 3 + 1] - first : 0u;
  float* Sg = state + (static_cast<std::size_t>(sq) * Hv + h) * kD * kD;
  // S slice into st: 128 keys x kNC columns, kNC / 16 float4 per thread (key (tid / (kNC / 4)) + (2048 / kNC) i,
  // columns 4 (tid % (kNC / 4)))
#pragma unroll
  for (int i = 0; i < kNT; ++i) {
    const std::uint32_t r = tid / (kNC / 4) + (2048 / kNC) * i, p = tid % (kNC / 4);
    const float4 v4 = *reinterpret_cast<const float4*>(Sg + static_cast<std::size_t>(r) * kD + j0 + 4 * p);
    st[4 * p][r] = v4.x, st[4 * p + 1][r] = v4.y, st[4 * p + 2][r] = v4.z, st[4 * p + 3][r] = v4.w;
  }
  // staged operands of one chunk, in registers: Uk, Qe (8192 floats each: 4 float4 per thread), the Wv and Ov slices
  // (64 x 64 each: rows tid / 16 and tid / 16 + 32, columns 4 (tid % 16)), G (threads < 64); K (8192 inputs: two
  // packs of 8) on its own, since it is stored later in the chunk
  // Wv / Ov slices: 64 x kNC floats = 16 kNC float4, float4 e = tid + 512 i at row e / (kNC / 4), column 4 (e % (kNC / 4));
  // with kNC = 16 the first 256 threads hold one each
  constexpr int kWN = (kC * kNC / 4 + 511) / 512;
  constexpr bool kWAll = kC * kNC / 4 >= 512;
  float4 ru0, ru1, ru2, ru3, rq0, rq1, rq2, rq3, rw[kWN], ro[kWN];
  Pack8<In> rk0, rk1;
  float rg;
  auto load = [&](std::uint32_t ci) {
    const std::uint32_t c = c0 + ci;
    const float* base = wy + (static_cast<std::size_t>(c) * Hv + h) * 4 * kC * kD;
    const float4* bu = reinterpret_cast<const float4*>(base);
    const float4* bq = reinterpret_cast<const float4*>(base + kC * kD);
    ru0 = bu[tid], ru1 = bu[tid + 512], ru2 = bu[tid + 1024], ru3 = bu[tid + 1536];
    rq0 = bq[tid], rq1 = bq[tid + 512], rq2 = bq[tid + 1024], rq3 = bq[tid + 1536];
    const std::uint32_t t = tid / (kNC / 4), p = 4 * (tid % (kNC / 4));
    const float* bw = base + 2 * kC * kD + j0 + p;
    const float* bo = base + 3 * kC * kD + j0 + p;
#pragma unroll
    for (int i = 0; i < kWN; ++i)
      if (kWAll || tid < kC * kNC / 4) {
        rw[i] = *reinterpret_cast<const float4*>(bw + (t + (2048 / kNC) * i) * kD);
        ro[i] = *reinterpret_cast<const float4*>(bo + (t + (2048 / kNC) * i) * kD);
      }
    rg = Gc[(static_cast<std::size_t>(c) * Hv + h) * kC + tid % kC];
  };
  auto load_k = [&](std::uint32_t ci) {
    const std::uint32_t start = first + 64 * ci, L = min(64u, len - 64 * ci);
    const std::uint32_t t0 = tid / 16, p8 = 8 * (tid % 16);  // packs tid and tid + 512: rows t0 and t0 + 32
    rk0 = Ld8(k + (static_cast<std::size_t>(start + min(t0, L - 1)) * Hk + kh) * kD + p8);
    rk1 = Ld8(k + (static_cast<std::size_t>(start + min(t0 + 32, L - 1)) * Hk + kh) * kD + p8);
  };
  auto store = [&]() {
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
    const std::uint32_t t = tid / (kNC / 4), p = 4 * (tid % (kNC / 4));
#pragma unroll
    for (int i = 0; i < kWN; ++i)
      if (kWAll || tid < kC * kNC / 4) {
        *reinterpret_cast<float4*>(&wvl[t + (2048 / kNC) * i][p]) = rw[i];
        *reinterpret_cast<float4*>(&ovl[t + (2048 / kNC) * i][p]) = ro[i];
      }
    if (tid < kC) Gl[tid] = rg;
  };
  auto store_k = [&](std::uint32_t L) {
    const std::uint32_t tk = tid / 16, pk = 8 * (tid % 16);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      kt[pk + e][KtCol(pk + e, tk)] = tk < L ? Cv(rk0.v[e]) : 0.0f;
      kt[pk + e][KtCol(pk + e, tk + 32)] = tk + 32 < L ? Cv(rk1.v[e]) : 0.0f;
    }
  };
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(kD));
  if (nc > 0) {
    load(0);
    load_k(0);
  }
  for (std::uint32_t ci = 0; ci < nc; ++ci) {
    const std::uint32_t start = first + 64 * ci, L = min(64u, len - 64 * ci), cn = ci + 1 < nc ? ci + 1 : ci;
    store();
    halo::LdsSync();
    load(cn);  // unconditional (the last chunk reloads itself): no loads under a branch
    if (tid < kC) Wl[tid] = expf(Gl[kC - 1] - Gl[tid]);  // the S-update weights exp(G_C - G_t)
    // Delta (waves 0-3) or the output (waves 4-7): token rows 16 (w % 4) .. + 16, four 16-column tiles, K range =
    // 128 keys, lane keys 32 fq .. + 32
    {
      const std::uint32_t r0 = 16 * (wave % 4);
      float(*A)[kCL] = wave < 4 ? ukl : qel;
      V4F acc[kNT];
#pragma unroll
      for (int ct = 0; ct < kNT; ++ct) acc[ct] = V4F{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 2
      for (int sb = 0; sb < 8; ++sb) {
        const float4 av = *reinterpret_cast<const float4*>(&A[r0 + fc][32 * fq + 4 * sb]);
#pragma unroll
        for (int ct = 0; ct < kNT; ++ct) {
          const float4 bv = *reinterpret_cast<const float4*>(&st[16 * ct + fc][32 * fq + 4 * sb]);
          acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, acc[ct], 0, 0, 0);
          acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc[ct], 0, 0, 0);
          acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc[ct], 0, 0, 0);
          acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc[ct], 0, 0, 0);
        }
      }
#pragma unroll
      for (int ct = 0; ct < kNT; ++ct) {
        const std::uint32_t col = 16 * ct + fc;
        if (wave < 4) {
          float d4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) d4[i] = wvl[r0 + 4 * fq + i][col] - acc[ct][i];
          *reinterpret_cast<float4*>(&dt[col][r0 + 4 * fq]) = make_float4(d4[0], d4[1], d4[2], d4[3]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const std::uint32_t t = r0 + 4 * fq + i;
            if (t < L)
              o[(static_cast<std::size_t>(start + t) * Hv + h) * kD + j0 + col] = (acc[ct][i] + ovl[t][col]) * inv_sqrt_d;
          }
        }
      }
    }
    halo::LdsSync();
    store_k(L);  // Uk has been read: K^T takes its place
    load_k(cn);
    halo::LdsSync();
    // S rows 16 w .. + 16, four 16-column tiles: gamma_C S + (K diag(exp(G_C - G_t)))^T Delta, K range = 64 tokens,
    // lane tokens 16 fq .. + 16
    {
      const std::uint32_t r0 = 16 * wave;
      const float gc = expf(Gl[kC - 1]);
      V4F acc[kNT];
#pragma unroll
      for (int ct = 0; ct < kNT; ++ct) {
        const float4 s4 = *reinterpret_cast<const float4*>(&st[16 * ct + fc][r0 + 4 * fq]);
        acc[ct][0] = gc * s4.x, acc[ct][1] = gc * s4.y, acc[ct][2] = gc * s4.z, acc[ct][3] = gc * s4.w;
      }
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) {
        const std::uint32_t tk = 16 * fq + 4 * sb;
        const float4 kv = *reinterpret_cast<const float4*>(&kt[r0 + fc][KtCol(r0 + fc, tk)]);
        const float4 wv = *reinterpret_cast<const float4*>(&Wl[tk]);
        const float a0 = kv.x * wv.x, a1 = kv.y * wv.y, a2 = kv.z * wv.z, a3 = kv.w * wv.w;
#pragma unroll
        for (int ct = 0; ct < kNT; ++ct) {
          const float4 dv = *reinterpret_cast<const float4*>(&dt[16 * ct + fc][tk]);
          acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, dv.x, acc[ct], 0, 0, 0);
          acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, dv.y, acc[ct], 0, 0, 0);
          acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(a2, dv.z, acc[ct], 0, 0, 0);
          acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(a3, dv.w, acc[ct], 0, 0, 0);
        }
      }
#pragma unroll
      for (int ct = 0; ct < kNT; ++ct)
        *reinterpret_cast<float4*>(&st[16 * ct + fc][r0 + 4 * fq]) = make_float4(acc[ct][0], acc[ct][1], acc[ct][2], acc[ct][3]);
    }
    halo::LdsSync();
  }
#pragma unroll
  for (int i = 0; i < kNT; ++i) {
    const std::uint32_t r = tid / (kNC / 4) + (2048 / kNC) * i, p = tid % (kNC / 4);
    *reinterpret_cast<float4*>(Sg + static_cast<std::size_t>(r) * kD + j0 + 4 * p) =
        make_float4(st[4 * p][r], st[4 * p + 1][r], st[4 * p + 2][r], st[4 * p + 3][r]);
  }
}

extern "C" __global__ void __launch_bounds__(512)
    halo_gdn_wy_prep(const std::uint16_t* __restrict__ q, const std::uint16_t* __restrict__ k,
                     const std::uint16_t* __restrict__ v, const float* __restrict__ g, const float* __restrict__ beta,
                     const std::uint32_t* __restrict__ chunks, float* __restrict__ wy, float* __restrict__ Gc,
                     std::uint32_t Hv, std::uint32_t Hk) {
  WyPrep(q, k, v, g, beta, chunks, wy, Gc, Hv, Hk);
}
extern "C" __global__ void __launch_bounds__(512)
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
  WyScan<std::uint16_t, 32>(k, wy, Gc, chunks, seqs, state, o, Hv, Hk);
}
extern "C" __global__ void __launch_bounds__(512)
    halo_gdn_wy_scan_f32(const float* __restrict__ k, const float* __restrict__ wy, const float* __restrict__ Gc,
                         const std::uint32_t* __restrict__ chunks, const std::uint32_t* __restrict__ seqs,
                         float* __restrict__ state, float* __restrict__ o, std::uint32_t Hv, std::uint32_t Hk) {
  WyScan<float, 32>(k, wy, Gc, chunks, seqs, state, o, Hv, Hk);
}
// 16 value columns per block (eight blocks per head): for batches with too few (sequence, head) pairs to fill the
// CUs at 32 columns, halving each block's matrix work on the chunk-serial path
extern "C" __global__ void __launch_bounds__(512)
    halo_gdn_wy_scan_n16(const std::uint16_t* __restrict__ k, const float* __restrict__ wy, const float* __restrict__ Gc,
                         const std::uint32_t* __restrict__ chunks, const std::uint32_t* __restrict__ seqs,
                         float* __restrict__ state, float* __restrict__ o, std::uint32_t Hv, std::uint32_t Hk) {
  WyScan<std::uint16_t, 16>(k, wy, Gc, chunks, seqs, state, o, Hv, Hk);
}
extern "C" __global__ void __launch_bounds__(512)
    halo_gdn_wy_scan_f32_n16(const float* __restrict__ k, const float* __restrict__ wy, const float* __restrict__ Gc,
                             const std::uint32_t* __restrict__ chunks, const std::uint32_t* __restrict__ seqs,
                             float* __restrict__ state, float* __restrict__ o, std::uint32_t Hv, std::uint32_t Hk) {
  WyScan<float, 16>(k, wy, Gc, chunks, seqs, state, o, Hv, Hk);
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
// halo_gdn_step_q8 takes K <= 4 (the ring slots in registers, loaded before the state), _kn any K <= 8.
namespace {
template <bool kSmallK>
__device__ __forceinline__ void GdnStepQ8(
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
  HALO_PHASE(0, 0);
  // prologue: threads 0..383 take the q, k and v channels of this head (128 each: waves 0-1, 2-3, 4-5). With K <= 4
  // every ring slot is loaded before the position arrives, so the ring loads do not wait for nkv; the slots are
  // selected by position afterwards.
  const std::uint32_t seg = t / kD, i = t % kD;
  const std::uint32_t ch = seg == 0 ? kh * kD + i : seg == 1 ? Dk + kh * kD + i : 2 * Dk + h * kD + min(i, kD - 1);
  float* rs = ring + static_cast<std::size_t>(s) * K * C;
  const std::uint32_t pos = nkv[s] - 1;
  const float zg = z[static_cast<std::size_t>(s) * Dv + h * kD + min(t, static_cast<std::uint32_t>(kD - 1))];  // t < kD
  float y = 0.0f;
  // the prologue's loads are issued before the state's (64 KB per block, eight 16-byte loads per thread), so the conv
  // and norms below run while the state streams in
  // (unconditional loads from clamped addresses, selected afterwards: a load under a branch would wait at the join
  // for every load issued before it, the state's included)
  const float x = qkv[static_cast<std::size_t>(s) * C + ch];
  float slot[4], w[4];
#pragma unroll
  for (std::uint32_t j = 0; j < 4; ++j) {
    const std::uint32_t jj = min(j, K - 1);
    slot[j] = rs[static_cast<std::size_t>(jj) * C + ch];
    w[j] = conv_w[static_cast<std::size_t>(ch) * K + jj];
  }
  const float ga = a[h], gdt = dt[h], galpha = ab[static_cast<std::size_t>(s) * 2 * Hv + h],
              gbeta = ab[static_cast<std::size_t>(s) * 2 * Hv + Hv + h];
  __builtin_amdgcn_sched_barrier(0);  // keep the issue order
  // Measured: the state issued only once the prologue's inputs have landed streams in ~2 us and leaves the conv and
  // norms free to run; issued right behind them, the wave stalls on issuing it (until ~2.7 us) with the conv waiting.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  float4 row[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) row[r] = *reinterpret_cast<const float4*>(St + static_cast<std::size_t>(i0 + r) * kD + j0);
  __builtin_amdgcn_sched_barrier(0);
  // the conv in every thread (waves 6-7 on a clamped channel, discarded), so the loads above stay where they are
  float acc;
  if constexpr (kSmallK) {
    acc = w[K - 1] * x;
#pragma unroll
    for (std::uint32_t j = 0; j < 3; ++j)
      if (j + 1 < K) acc += w[j] * slot[(pos + 1 + j) % K];
  } else {
    acc = conv_w[static_cast<std::size_t>(ch) * K + K - 1] * x;
    for (std::uint32_t j = 0; j + 1 < K; ++j)
      acc += conv_w[static_cast<std::size_t>(ch) * K + j] * rs[static_cast<std::size_t>((pos + 1 + j) % K) * C + ch];
  }
  if (seg < 3) {
    if (seg == 2 || h < Hk) rs[static_cast<std::size_t>(pos % K) * C + ch] = x;
    y = halo::Silu(acc);
  }
  const float ss = halo::GroupSum(y * y);
  if (lane == 0) part[wave] = ss;
  const float g0 = ga * halo::Softplus(galpha + gdt), g1 = halo::Sigmoid(gbeta);
  if (t == 0) {
    gates[0] = g0;
    gates[1] = g1;
  }
  __syncthreads();
  HALO_PHASE(0, 1);
  if (seg < 2) {
    const float sc = 1.0f / sqrtf(part[2 * seg] + part[2 * seg + 1] + eps);
    (seg == 0 ? sq : sk)[i] = y * sc;
  } else if (seg == 2) {
    sv[i] = y;
  }
  __syncthreads();
  HALO_PHASE(0, 2);
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
  HALO_PHASE(0, 3);
  if (t < kD) {
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc += red[r][t];
    dl[t] = (sv[t] - acc) * bt;
  }
  __syncthreads();
  HALO_PHASE(0, 4);
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
  HALO_PHASE(0, 5);
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
  HALO_PHASE(0, 6);
  if (t < kD) {
    const float sc = 1.0f / sqrtf((part[0] + part[1]) / static_cast<float>(kD) + eps);
    const std::size_t off = static_cast<std::size_t>(s) * Dv + h * kD + t;
    const float v = o * sc * norm_w[t] * halo::Sigmoid(zg);
    const float amax = halo::GroupMax<32>(fabsf(v));
    const float scale = amax / 127.0f;
    oq[off] = static_cast<std::int8_t>(scale > 0.0f ? static_cast<int>(rintf(v / scale)) : 0);
    if (t % 32 == 0) os[off / 32] = scale;
  }
  HALO_PHASE(0, 7);
}
}  // namespace

extern "C" __global__ void __launch_bounds__(512) halo_gdn_step_q8(
    const float* qkv, const float* z, const float* ab, float* ring, const float* conv_w, const float* a,
    const float* dt, const float* norm_w, float* state, const std::uint32_t* nkv, std::int8_t* oq, float* os,
    std::uint32_t Hk, std::uint32_t Hv, std::uint32_t K, float eps) {
  GdnStepQ8<true>(qkv, z, ab, ring, conv_w, a, dt, norm_w, state, nkv, oq, os, Hk, Hv, K, eps);
}
extern "C" __global__ void __launch_bounds__(512) halo_gdn_step_q8_kn(
    const float* qkv, const float* z, const float* ab, float* ring, const float* conv_w, const float* a,
    const float* dt, const float* norm_w, float* state, const std::uint32_t* nkv, std::int8_t* oq, float* os,
    std::uint32_t Hk, std::uint32_t Hv, std::uint32_t K, float eps) {
  GdnStepQ8<false>(qkv, z, ab, ring, conv_w, a, dt, norm_w, state, nkv, oq, os, Hk, Hv, K, eps);
}
