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
