// Per-token glue of the hybrid decode step (gfx950, wave64): norms fused with the activation quantizer, the
// DeltaNet conv / L2-norm / decay prologue, the gated output norm, q/k norm + RoPE + KV append, embedding lookup,
// greedy argmax and the device-side step advance (so one captured graph replays at every position).
//
// Reference semantics: cpu::RmsNorm / L2Norm / Rope / Silu / Softplus (src/model/cpu_ops.cpp:134-185),
// ReferenceModel::LinearAttention conv + norms + gate (src/model/reference.cpp:278-366), ReferenceModel::Attention
// q/gate split, q/k norm, NEOX rope (src/model/reference.cpp:368-416), HaloStepParam (src/kernels/step_params.h).
#include <type_traits>

#include "common.h"
#include "halo_sample.h"

using halo::kWave;

namespace {
// Quantizes 32 consecutive values held one per lane of a half wave (amax / 127, round half to even).
__device__ __forceinline__ void Quant32(float v, std::int8_t* xq, float* xs, std::uint32_t blk) {
  const std::uint32_t lane = threadIdx.x % 32;
  const float amax = halo::GroupMax<32>(fabsf(v));
  const float scale = amax / 127.0f;
  xq[blk * 32 + lane] = static_cast<std::int8_t>(scale > 0.0f ? static_cast<int>(rintf(v / scale)) : 0);
  if (lane == 0) xs[blk] = scale;
}
}  // namespace

// grid (S), block 256 (H <= 8192, H % 32 == 0). res [S][H] += delta [S][H] (delta may be null), then
// xn = RMSNorm(res) * w (fp32, may be null) and its Q8 quantization xq [S][H], xs [S][H / 32] (may be null).
// The row decomposition is the canonical one (halo::RmsNormRow8), shared with the projection prologues.
extern "C" __global__ void __launch_bounds__(256)
    halo_add_rmsnorm_q8(float* __restrict__ res, const float* __restrict__ delta, const float* __restrict__ w,
                        float* __restrict__ xn, std::int8_t* __restrict__ xq, float* __restrict__ xs,
                        std::uint32_t H, float eps) {
  __shared__ float red[4];
  const std::size_t s = blockIdx.x;
  // the row and the weights are loaded together (one round trip); rows of at most 2048 take one chunk per thread
  auto body = [&](auto kc) {
    constexpr int KC = decltype(kc)::value;
    halo::Row8<KC> r, wr;
    halo::LoadRow8(res + s * H, delta != nullptr ? delta + s * H : nullptr, H, r);
    if (w != nullptr) {
      halo::LoadRow8(w, nullptr, H, wr);
    } else {
#pragma unroll
      for (int k = 0; k < KC; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) wr.v[k][e] = 1.0f;  // v * scale * 1 = v * scale
    }
    if (delta != nullptr) halo::StoreRow8(res + s * H, H, r);
    halo::RmsNormRow8W(r, wr, H, eps, red);
    if (xn != nullptr) halo::StoreRow8(xn + s * H, H, r);
    if (xq != nullptr) halo::QuantRow8(r, H, xq + s * H, xs + s * (H / 32));
  };
  if (H <= 2048)
    body(std::integral_constant<int, 1>{});
  else
    body(std::integral_constant<int, 4>{});
}

// grid (S, C / 256), block 256: the DeltaNet prologue for one token per session, one channel per thread.
//   qkv [S][C] (C = 2 Dk + Dv channels: q | k | v), conv_state [S][K-1][C] (oldest first), conv_w [C][K];
//   conv = SiLU(w[K-1] x + sum_{k<K-1} w[k] state[k]); the state shifts in x. q, k per key head L2-normalized
//   (eps = rms eps); ab [S][2 Hv] (alpha | beta logits), a [Hv] (negative), dt [Hv]:
//   g = a * softplus(alpha + dt) (log decay), beta = sigmoid(beta logit).
//   Outputs q, k [S][Hk][d], v [S][Hv][d], g, beta [S][Hv]. d = 128: a block covers two heads.
extern "C" __global__ void __launch_bounds__(256) halo_gdn_prep_decode(
    const float* __restrict__ qkv, float* __restrict__ conv_state, const float* __restrict__ conv_w,
    const float* __restrict__ ab, const float* __restrict__ a, const float* __restrict__ dt, float* __restrict__ q,
    float* __restrict__ k, float* __restrict__ v, float* __restrict__ g, float* __restrict__ beta, std::uint32_t Hk,
    std::uint32_t Hv, std::uint32_t d, std::uint32_t K, float eps) {
  __shared__ float part[4];
  const std::size_t s = blockIdx.x;
  const std::uint32_t Dk = Hk * d, Dv = Hv * d, C = 2 * Dk + Dv;
  const std::uint32_t ch = blockIdx.y * blockDim.x + threadIdx.x;
  const float x = qkv[s * C + ch];
  float* st = conv_state + s * (K - 1) * C;
  float acc = conv_w[static_cast<std::size_t>(ch) * K + K - 1] * x;
  for (std::uint32_t j = 0; j + 1 < K; ++j) acc += conv_w[static_cast<std::size_t>(ch) * K + j] * st[j * C + ch];
  for (std::uint32_t j = 0; j + 2 < K; ++j) st[j * C + ch] = st[(j + 1) * C + ch];
  if (K > 1) st[(K - 2) * C + ch] = x;
  const float y = halo::Silu(acc);
  // the block's 256 channels are two heads of 128 (two waves each)
  const std::uint32_t wave = threadIdx.x / kWave;
  const float ss = halo::GroupSum(y * y);
  if (threadIdx.x % kWave == 0) part[wave] = ss;
  __syncthreads();
  const std::uint32_t head = ch / d;
  if (ch < 2 * Dk) {
    const std::uint32_t w0 = (wave / 2) * 2;
    const float sc = 1.0f / sqrtf(part[w0] + part[w0 + 1] + eps);
    float* dst = head < Hk ? q + (s * Hk + head) * d : k + (s * Hk + head - Hk) * d;
    dst[ch % d] = y * sc;
  } else {
    v[s * Dv + ch - 2 * Dk] = y;
  }
  if (blockIdx.y == 0 && threadIdx.x < Hv) {
    const std::uint32_t h = threadIdx.x;
    g[s * Hv + h] = a[h] * halo::Softplus(ab[s * 2 * Hv + h] + dt[h]);
    beta[s * Hv + h] = halo::Sigmoid(ab[s * 2 * Hv + Hv + h]);
  }
}

// grid (S), block 256: per 128-value head RMSNorm(o_h) * w (d weights shared by heads) * sigmoid(z_h), then the
// Q8 quantization: o, z [S][Hv][d] -> xq [S][Hv d], xs [S][Hv d / 32]. d = 128, Hv d <= 8192. The row
// decomposition is the canonical one (halo::GatedNormRow8), shared with the output projection's prologue.
extern "C" __global__ void __launch_bounds__(256)
    halo_gated_rmsnorm_q8(const float* __restrict__ o, const float* __restrict__ z, const float* __restrict__ w,
                          std::int8_t* __restrict__ xq, float* __restrict__ xs, std::uint32_t Hv, std::uint32_t d,
                          float eps) {
  const std::size_t s = blockIdx.x;
  const std::uint32_t D = Hv * d;
  halo::Row8<4> r;
  halo::LoadRow8(o + s * D, nullptr, D, r);
  halo::GatedNormRow8(r, z + s * D, w, D, eps);
  halo::QuantRow8(r, D, xq + s * D, xs + s * (D / 32));
}

// grid (S, Hq + 2 Hkv), block 64 (one wave per head): attention prologue for one token per session (or, with tok_sess
// / tok_pos non-null, for each token of a prefill batch at its own session and position). qg [S][Hq][2 d] (per head: q | gate),
// kin, vin [S][Hkv][d]; RMSNorm of every q head (wq) and k head (wk); NEOX rope on the first `rot` dims at position
// nkv[s] - 1; q, gate [S][Hq][d] out; k, v appended to the paged pools at that position. d = 256.
extern "C" __global__ void __launch_bounds__(256) halo_attn_prep_decode(
    const float* __restrict__ qg, const float* __restrict__ kin, const float* __restrict__ vin,
    const float* __restrict__ wq, const float* __restrict__ wk, float* __restrict__ q, float* __restrict__ gate,
    float* __restrict__ kpool, float* __restrict__ vpool, const std::uint32_t* __restrict__ pages,
    const std::uint32_t* __restrict__ nkv, std::uint32_t Hq, std::uint32_t Hkv, std::uint32_t max_pages,
    std::uint32_t rot, float theta, float eps, const std::uint32_t* __restrict__ tok_sess,
    const std::uint32_t* __restrict__ tok_pos) {
  constexpr std::uint32_t d = 256, kPage = 16;
  // row s of the inputs / outputs; its session and position: per token in a prefill batch, else session s at nkv - 1
  const std::size_t s = blockIdx.x;
  const std::uint32_t lane = threadIdx.x % kWave;
  const std::size_t sess = tok_pos != nullptr ? tok_sess[s] : s;
  const std::uint32_t pos = tok_pos != nullptr ? tok_pos[s] : nkv[s] - 1;
  const std::uint32_t pg = pages[sess * max_pages + pos / kPage];
  {
    const std::uint32_t hh = blockIdx.y;
    // hh < Hq: q head; Hq <= hh < Hq + Hkv: k head; else v head (copied)
    float x[4];
    const float* src;
    if (hh < Hq)
      src = qg + (s * Hq + hh) * 2 * d;
    else if (hh < Hq + Hkv)
      src = kin + (s * Hkv + (hh - Hq)) * d;
    else
      src = vin + (s * Hkv + (hh - Hq - Hkv)) * d;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = src[lane + 64 * i];
    if (hh >= Hq + Hkv) {
      const std::uint32_t kvh = hh - Hq - Hkv;
      float* dst = vpool + ((static_cast<std::size_t>(pg) * Hkv + kvh) * kPage + pos % kPage) * d;
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[lane + 64 * i] = x[i];
      return;
    }
    float out[4], wv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wv[i] = (hh < Hq ? wq : wk)[lane + 64 * i];
    halo::NormRopeHead(x, wv, halo::RopeAngles(pos, rot, theta), rot, eps, out);
    if (hh < Hq) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        q[(s * Hq + hh) * d + lane + 64 * i] = out[i];
        gate[(s * Hq + hh) * d + lane + 64 * i] = src[d + lane + 64 * i];
      }
    } else {
      const std::uint32_t kvh = hh - Hq;
      float* dst = kpool + ((static_cast<std::size_t>(pg) * Hkv + kvh) * kPage + pos % kPage) * d;
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[lane + 64 * i] = out[i];
    }
  }
}

// grid (S), block 256: x [S][H] = dequantized embedding row tokens[s] of a repacked Q8_0 table.
extern "C" __global__ void __launch_bounds__(256)
    halo_embed_q8(const std::int8_t* __restrict__ qs, const std::uint16_t* __restrict__ d,
                  const std::uint32_t* __restrict__ tokens, float* __restrict__ x, std::uint32_t H,
                  std::uint32_t qstride) {
  const std::size_t s = blockIdx.x, t = tokens[s];
  for (std::uint32_t i = threadIdx.x; i < H; i += blockDim.x)
    x[s * H + i] = halo::F16(d[t * (H / 32) + i / 32]) * static_cast<float>(qs[t * qstride + i]);
}

// grid (S, 64), block 256: partial argmax of each 1/64 slice of the V logits of session s (ties to the lower id)
// -> part [S][64] as (value, id) pairs; halo_step_advance finishes the reduction.
extern "C" __global__ void __launch_bounds__(256)
    halo_argmax_part(const float* __restrict__ logits, float* __restrict__ pv, std::uint32_t* __restrict__ pi,
                     std::uint32_t V) {
  __shared__ float bv[4];
  __shared__ std::uint32_t bi[4];
  const std::size_t s = blockIdx.x;
  const std::uint32_t per = (V + gridDim.y - 1) / gridDim.y, lo = blockIdx.y * per, hi = min(V, lo + per);
  float v = -INFINITY;
  std::uint32_t at = 0xFFFFFFFFu;
  for (std::uint32_t i = lo + threadIdx.x; i < hi; i += blockDim.x) {
    const float x = logits[s * V + i];
    if (x > v) {  // ascending i per thread: the first maximum wins
      v = x;
      at = i;
    }
  }
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, kWave);
    const std::uint32_t oi = __shfl_xor(at, o, kWave);
    if (ov > v || (ov == v && oi < at)) {
      v = ov;
      at = oi;
    }
  }
  const std::uint32_t wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    bv[wave] = v;
    bi[wave] = at;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (std::uint32_t w = 1; w < blockDim.x / kWave; ++w)
      if (bv[w] > v || (bv[w] == v && bi[w] < at)) {
        v = bv[w];
        at = bi[w];
      }
    pv[s * gridDim.y + blockIdx.y] = v;
    pi[s * gridDim.y + blockIdx.y] = at;
  }
}

// grid 1, block 64: end of a decode step. For each session s < S: the produced token is the argmax over the
// `parts` partial maxima of halo_argmax_part (ties to the lower id); it is recorded at history[s][nkv[s]]; the
// next input token is the prompt token at that position when it exists (teacher forcing), otherwise the produced
// one; nkv[s] advances by one. prompt [S][prompt_stride], prompt_len [S].
extern "C" __global__ void __launch_bounds__(1024)
    halo_step_advance(const float* __restrict__ pv, const std::uint32_t* __restrict__ pi,
                      const std::uint32_t* __restrict__ prompt, const std::uint32_t* __restrict__ prompt_len,
                      std::uint32_t* __restrict__ tokens, std::uint32_t* __restrict__ nkv,
                      std::uint32_t* __restrict__ history, std::uint32_t* __restrict__ produced, std::uint32_t S,
                      std::uint32_t parts, std::uint32_t prompt_stride, std::uint32_t history_stride,
                      std::uint32_t max_context) {
  // one wave per session: lane p reduces partial maxima p, p + 64, ...; then a wave reduction (ties to the lower id)
  const std::uint32_t s = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (s >= S) return;
  float v = -INFINITY;
  std::uint32_t at = 0xFFFFFFFFu;
  for (std::uint32_t p = lane; p < parts; p += kWave) {
    const float x = pv[s * parts + p];
    const std::uint32_t i = pi[s * parts + p];
    if (x > v || (x == v && i < at)) {
      v = x;
      at = i;
    }
  }
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, kWave);
    const std::uint32_t oi = __shfl_xor(at, o, kWave);
    if (ov > v || (ov == v && oi < at)) {
      v = ov;
      at = oi;
    }
  }
  if (lane != 0) return;
  produced[s] = at;
  const std::uint32_t n = nkv[s];  // positions now in the cache, the produced token goes at index n
  if (n < history_stride) history[static_cast<std::size_t>(s) * history_stride + n] = at;
  tokens[s] = n < prompt_len[s] ? prompt[static_cast<std::size_t>(s) * prompt_stride + n] : at;
  nkv[s] = min(n + 1, max_context);
}

// The advance after device sampling: out[s] holds session s's drawn token and RNG state (halo_sample_final). The
// token is recorded at history[s][nkv[s]] as in halo_step_advance; a sampler code (no finite logit, bad
// parameters: token >= vocab) is recorded as is and token 0 fed next, so the step never indexes past the
// embedding. The RNG state goes back into params[s] for the next step.
extern "C" __global__ void __launch_bounds__(64)
    halo_step_advance_sampled(const HaloSampleOut* __restrict__ out, HaloSampleParams* __restrict__ params,
                              const std::uint32_t* __restrict__ prompt, const std::uint32_t* __restrict__ prompt_len,
                              std::uint32_t* __restrict__ tokens, std::uint32_t* __restrict__ nkv,
                              std::uint32_t* __restrict__ history, std::uint32_t* __restrict__ produced,
                              std::uint32_t S, std::uint32_t vocab, std::uint32_t prompt_stride,
                              std::uint32_t history_stride, std::uint32_t max_context) {
  const std::uint32_t s = threadIdx.x;
  if (s >= S) return;
  const HaloSampleOut o = out[s];
  params[s].rng = o.rng;
  produced[s] = o.token;
  const std::uint32_t n = nkv[s];
  if (n < history_stride) history[static_cast<std::size_t>(s) * history_stride + n] = o.token;
  tokens[s] = n < prompt_len[s] ? prompt[static_cast<std::size_t>(s) * prompt_stride + n]
                                : (o.token < vocab ? o.token : 0u);
  nkv[s] = min(n + 1, max_context);
}

// ---- batched prefill glue ------------------------------------------------------------------------------------------
// A prefill batch is T tokens; token t is position tok_pos[t] of session tok_sess[t] (runs of consecutive positions per
// session, laid out back to back). seg_start[t] is the first position of t's run in this batch.

// grid (T), block 256: x [T][H] = dequantized embedding rows of prompt[tok_sess[t]][tok_pos[t]].
extern "C" __global__ void __launch_bounds__(256)
    halo_embed_prompt_q8(const std::int8_t* __restrict__ qs, const std::uint16_t* __restrict__ d,
                         const std::uint32_t* __restrict__ prompt, std::uint32_t prompt_stride,
                         const std::uint32_t* __restrict__ tok_sess, const std::uint32_t* __restrict__ tok_pos,
                         float* __restrict__ x, std::uint32_t H, std::uint32_t qstride) {
  const std::size_t t = blockIdx.x;
  const std::size_t tok = prompt[static_cast<std::size_t>(tok_sess[t]) * prompt_stride + tok_pos[t]];
  for (std::uint32_t i = threadIdx.x; i < H; i += blockDim.x)
    x[t * H + i] = halo::F16(d[tok * (H / 32) + i / 32]) * static_cast<float>(qs[tok * qstride + i]);
}

// grid (ceil(T / 16), C / 256), block 64: the DeltaNet prologue of halo_gdn_prep_decode for every token of a prefill
// batch. The conv taps at positions below the token's run come from the session's conv ring (slot p % K), inside
// the run from the batch's own projection rows, below 0 they are zero. Outputs for the chunked recurrence: q, k
// [T][Hk][d] and v [T][Hv][d], g, beta [T][Hv], all fp32 as the decode step computes them. Lane l of block (b, c)
// owns channels 256 c + 4 l .. + 3 (16-byte loads and stores) for the block's 16 consecutive batch tokens; a q / k
// head of 128 channels is 32 lanes, its sum of squares one 32-lane reduction. The tap rows of a token are the rows
// the block just loaded for the tokens before it (L1 / L2 hits). d = 128, C % 256 == 0, K <= 8.
namespace {
// The outputs of one token of the prefill prologue from its four conv results y (channels ch .. ch + 3 of lane
// `lane`): q / k L2-normalized per 128-channel head, v as is; blocks of column 0 also write the token's g and beta.
__device__ __forceinline__ void GdnPrepOut(const float (&y)[4], std::uint32_t t, std::uint32_t ch, std::uint32_t lane,
                                           const float* __restrict__ ab, const float* __restrict__ a,
                                           const float* __restrict__ dt, float* __restrict__ q, float* __restrict__ k,
                                           float* __restrict__ v, float* __restrict__ g, float* __restrict__ beta,
                                           std::uint32_t Hk, std::uint32_t Hv, float eps) {
  constexpr std::uint32_t kD = 128;
  const std::uint32_t Dk = Hk * kD, Dv = Hv * kD;
  if (ch < 2 * Dk) {
    const float ss = halo::GroupSum<32>((y[0] * y[0] + y[1] * y[1]) + (y[2] * y[2] + y[3] * y[3]));
    const float sc = 1.0f / sqrtf(ss + eps);
    const std::uint32_t head = ch / kD;
    float* dst = head < Hk ? q + (static_cast<std::size_t>(t) * Hk + head) * kD
                           : k + (static_cast<std::size_t>(t) * Hk + head - Hk) * kD;
    *reinterpret_cast<float4*>(dst + ch % kD) = make_float4(y[0] * sc, y[1] * sc, y[2] * sc, y[3] * sc);
  } else {
    *reinterpret_cast<float4*>(v + static_cast<std::size_t>(t) * Dv + ch - 2 * Dk) = make_float4(y[0], y[1], y[2], y[3]);
  }
  if (blockIdx.y == 0)
    for (std::uint32_t h = lane; h < Hv; h += 64) {
      g[static_cast<std::size_t>(t) * Hv + h] = a[h] * halo::Softplus(ab[static_cast<std::size_t>(t) * 2 * Hv + h] + dt[h]);
      beta[static_cast<std::size_t>(t) * Hv + h] = halo::Sigmoid(ab[static_cast<std::size_t>(t) * 2 * Hv + Hv + h]);
    }
}
}  // namespace

extern "C" __global__ void __launch_bounds__(64) halo_gdn_prep_prefill(
    const float* __restrict__ qkv, const float* __restrict__ ring, const float* __restrict__ conv_w,
    const float* __restrict__ ab, const float* __restrict__ a, const float* __restrict__ dt,
    const std::uint32_t* __restrict__ tok_sess, const std::uint32_t* __restrict__ tok_pos,
    const std::uint32_t* __restrict__ seg_start, float* __restrict__ q, float* __restrict__ k,
    float* __restrict__ v, float* __restrict__ g, float* __restrict__ beta, std::uint32_t T, std::uint32_t Hk,
    std::uint32_t Hv, std::uint32_t K, float eps) {
  constexpr std::uint32_t kD = 128, kTok = 16, kMaxK = 8;
  const std::uint32_t Dk = Hk * kD, Dv = Hv * kD, C = 2 * Dk + Dv;
  const std::uint32_t lane = threadIdx.x, ch = blockIdx.y * 256 + 4 * lane;
  const std::uint32_t t0 = blockIdx.x * kTok, t1 = min(t0 + kTok, T);
  float w[4][kMaxK];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (std::uint32_t j = 0; j < kMaxK; ++j) w[c][j] = j < K ? conv_w[static_cast<std::size_t>(ch + c) * K + j] : 0.0f;
  for (std::uint32_t t = t0; t < t1; ++t) {
    const std::uint32_t s = tok_sess[t], p = tok_pos[t], p0 = seg_start[t];
    const float4 x = *reinterpret_cast<const float4*>(qkv + static_cast<std::size_t>(t) * C + ch);
    float acc[4] = {w[0][K - 1] * x.x, w[1][K - 1] * x.y, w[2][K - 1] * x.z, w[3][K - 1] * x.w};
    for (std::uint32_t j = 0; j + 1 < K; ++j) {
      // tap j reads position p - (K - 1) + j
      const std::int64_t pp = static_cast<std::int64_t>(p) - static_cast<std::int64_t>(K - 1) + j;
      float4 xv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (pp >= static_cast<std::int64_t>(p0))
        xv = *reinterpret_cast<const float4*>(qkv + (static_cast<std::size_t>(t) - (p - static_cast<std::uint32_t>(pp))) * C + ch);
      else if (pp >= 0)
        xv = *reinterpret_cast<const float4*>(ring + (static_cast<std::size_t>(s) * K + static_cast<std::uint32_t>(pp) % K) * C + ch);
      acc[0] += w[0][j] * xv.x;
      acc[1] += w[1][j] * xv.y;
      acc[2] += w[2][j] * xv.z;
      acc[3] += w[3][j] * xv.w;
    }
    float y[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) y[c] = halo::Silu(acc[c]);
    GdnPrepOut(y, t, ch, lane, ab, a, dt, q, k, v, g, beta, Hk, Hv, eps);
  }
}

// The same prologue for conv kernel K = 4 with the block's rows in registers: the 16 tokens' rows and the 3 before
// them are loaded at once (19 independent 16-byte loads per lane), so the taps cost no further loads and no load
// waits on the previous token's; ring rows (taps below a run's first position in this batch) are loaded where
// needed. Same operations in the same order as halo_gdn_prep_prefill, so the results are bitwise equal.
extern "C" __global__ void __launch_bounds__(64) halo_gdn_prep_prefill_k4(
    const float* __restrict__ qkv, const float* __restrict__ ring, const float* __restrict__ conv_w,
    const float* __restrict__ ab, const float* __restrict__ a, const float* __restrict__ dt,
    const std::uint32_t* __restrict__ tok_sess, const std::uint32_t* __restrict__ tok_pos,
    const std::uint32_t* __restrict__ seg_start, float* __restrict__ q, float* __restrict__ k,
    float* __restrict__ v, float* __restrict__ g, float* __restrict__ beta, std::uint32_t T, std::uint32_t Hk,
    std::uint32_t Hv, std::uint32_t K, float eps) {
  constexpr std::uint32_t kD = 128, kTok = 16, kK = 4;
  const std::uint32_t C = 2 * Hk * kD + Hv * kD;
  const std::uint32_t lane = threadIdx.x, ch = blockIdx.y * 256 + 4 * lane;
  const std::uint32_t t0 = blockIdx.x * kTok;
  float w[4][kK];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (std::uint32_t j = 0; j < kK; ++j) w[c][j] = conv_w[static_cast<std::size_t>(ch + c) * K + j];
  // xr[r] = row t0 - 3 + r (clamped into [0, T): rows outside are loaded but never used)
  float4 xr[kTok + kK - 1];
#pragma unroll
  for (std::uint32_t r = 0; r < kTok + kK - 1; ++r) {
    const std::int64_t row = static_cast<std::int64_t>(t0) - static_cast<std::int64_t>(kK - 1) + r;
    const std::uint32_t rc = static_cast<std::uint32_t>(row < 0 ? 0 : (row >= T ? T - 1 : row));
    xr[r] = *reinterpret_cast<const float4*>(qkv + static_cast<std::size_t>(rc) * C + ch);
  }
#pragma unroll
  for (std::uint32_t i = 0; i < kTok; ++i) {
    const std::uint32_t t = t0 + i;
    if (t >= T) break;
    const std::uint32_t s = tok_sess[t], p = tok_pos[t], p0 = seg_start[t];
    const float4 x = xr[i + kK - 1];
    float acc[4] = {w[0][kK - 1] * x.x, w[1][kK - 1] * x.y, w[2][kK - 1] * x.z, w[3][kK - 1] * x.w};
#pragma unroll
    for (std::uint32_t j = 0; j + 1 < kK; ++j) {
      // tap j reads position p - 3 + j: row t - 3 + j when inside the run
      const std::int64_t pp = static_cast<std::int64_t>(p) - static_cast<std::int64_t>(kK - 1) + j;
      float4 xv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (pp >= static_cast<std::int64_t>(p0))
        xv = xr[i + j];
      else if (pp >= 0)
        xv = *reinterpret_cast<const float4*>(ring + (static_cast<std::size_t>(s) * kK + static_cast<std::uint32_t>(pp) % kK) * C + ch);
      acc[0] += w[0][j] * xv.x;
      acc[1] += w[1][j] * xv.y;
      acc[2] += w[2][j] * xv.z;
      acc[3] += w[3][j] * xv.w;
    }
    float y[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) y[c] = halo::Silu(acc[c]);
    GdnPrepOut(y, t, ch, lane, ab, a, dt, q, k, v, g, beta, Hk, Hv, eps);
  }
}

// grid (nseg, C / 256), block 256: after a prefill batch, each run's last K positions go to its session's conv ring
// (slot p % K). segs [nseg][4] = {session, start, length, first token}.
extern "C" __global__ void __launch_bounds__(256)
    halo_gdn_ring_update(const float* __restrict__ qkv, float* __restrict__ ring,
                         const std::uint32_t* __restrict__ segs, std::uint32_t K, std::uint32_t C) {
  const std::uint32_t* sg = segs + 4 * static_cast<std::size_t>(blockIdx.x);
  const std::uint32_t s = sg[0], start = sg[1], len = sg[2], first = sg[3];
  const std::uint32_t ch = blockIdx.y * blockDim.x + threadIdx.x;
  for (std::uint32_t j = 0; j < K && j < len; ++j) {
    const std::uint32_t p = start + len - 1 - j;
    ring[(static_cast<std::size_t>(s) * K + p % K) * C + ch] = qkv[(static_cast<std::size_t>(first) + len - 1 - j) * C + ch];
  }
}

// grid (nseg), block 256: copies the quantized final-norm row of each run's last token to row i of a small batch
// for the LM head. xq [T][H], xs [T][H / 32] -> lq [nseg][H], ls [nseg][H / 32].
extern "C" __global__ void __launch_bounds__(256)
    halo_prefill_gather_last(const std::int8_t* __restrict__ xq, const float* __restrict__ xs,
                             const std::uint32_t* __restrict__ segs, std::int8_t* __restrict__ lq,
                             float* __restrict__ ls, std::uint32_t H) {
  const std::uint32_t* sg = segs + 4 * static_cast<std::size_t>(blockIdx.x);
  const std::size_t t = static_cast<std::size_t>(sg[3]) + sg[2] - 1, i = blockIdx.x;
  for (std::uint32_t c = threadIdx.x; c < H; c += blockDim.x) lq[i * H + c] = xq[t * H + c];
  for (std::uint32_t c = threadIdx.x; c < H / 32; c += blockDim.x) ls[i * (H / 32) + c] = xs[t * (H / 32) + c];
}

// grid 1, block 64: end of a prefill batch, per run i (thread): the produced token is the argmax over the `parts`
// partial maxima of row i (ties to the lower id); history[s][start + len] = it; the next input token is the prompt
// token at start + len when the prompt goes on, else the produced one; nkv[s] = start + len + 1 (the next decode
// step processes position start + len).
extern "C" __global__ void __launch_bounds__(64)
    halo_prefill_advance(const float* __restrict__ pv, const std::uint32_t* __restrict__ pi,
                         const std::uint32_t* __restrict__ segs, const std::uint32_t* __restrict__ prompt,
                         const std::uint32_t* __restrict__ prompt_len, std::uint32_t* __restrict__ tokens,
                         std::uint32_t* __restrict__ nkv, std::uint32_t* __restrict__ history,
                         std::uint32_t* __restrict__ produced, std::uint32_t nseg, std::uint32_t parts,
                         std::uint32_t stride, std::uint32_t max_context) {
  const std::uint32_t i = threadIdx.x;
  if (i >= nseg) return;
  float v = -INFINITY;
  std::uint32_t at = 0xFFFFFFFFu;
  for (std::uint32_t p = 0; p < parts; ++p) {
    const float x = pv[i * parts + p];
    const std::uint32_t id = pi[i * parts + p];
    if (x > v || (x == v && id < at)) {
      v = x;
      at = id;
    }
  }
  const std::uint32_t* sg = segs + 4 * static_cast<std::size_t>(i);
  const std::uint32_t s = sg[0], n = sg[1] + sg[2];
  produced[s] = at;
  if (n < stride) history[static_cast<std::size_t>(s) * stride + n] = at;
  tokens[s] = n < prompt_len[s] ? prompt[static_cast<std::size_t>(s) * stride + n] : at;
  nkv[s] = min(n + 1, max_context);
}
