// Reference-named decode kernels: the names, parameter lists and grid conventions of the reference's generic
// decode kernels (src/kernels/core.hip:259-586, 2621-2650, 3003-3063), so engine code that launches them by name
// runs unchanged; the bodies are gfx950 implementations (wave64 reductions, coalesced row accesses). The model's own
// step uses the fused MI355X kernels instead (model.hip, gdn.hip, attn.hip); these serve the kernel-level drop-in.
//
// Reductions over a block accept any block size that is a multiple of 64 (the reference launches 128 or 256).
#include "common.h"

namespace halo::refk {

using halo::kWave;

// Sum / maximum over the block; every thread gets the result. `red` holds one entry per wave.
__device__ __forceinline__ float BlockSumAny(float v, float* red) {
  v = halo::GroupSum(v);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float r = 0.0f;
  for (std::uint32_t i = 0; i < (blockDim.x + kWave - 1) / kWave; ++i) r += red[i];
  __syncthreads();
  return r;
}
__device__ __forceinline__ float BlockMaxAny(float v, float* red) {
  v = halo::GroupMax(v);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float r = -INFINITY;
  for (std::uint32_t i = 0; i < (blockDim.x + kWave - 1) / kWave; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

// Row normalisation helpers shared by the norm kernels: one block per row of d values. Both passes use 16-byte
// accesses when the row and d allow them (scalar otherwise); the sum of squares keeps two fused chains per thread
// (even / odd lanes of each float4) and then BlockSumAny. Every read of the first pass precedes the block sum's
// barriers, so the second pass may write in place.
__device__ __forceinline__ bool Vec4Ok(const void* p, std::uint32_t d) {
  return (d & 3u) == 0 && (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0;
}
__device__ __forceinline__ float RowSumSq(const float* v, std::uint32_t d, float* red) {
  float a0 = 0.0f, a1 = 0.0f;
  if (Vec4Ok(v, d)) {
    const float4* v4 = reinterpret_cast<const float4*>(v);
    for (std::uint32_t i = threadIdx.x; i < d / 4; i += blockDim.x) {
      const float4 f = v4[i];
      a0 = __builtin_fmaf(f.x, f.x, a0);
      a1 = __builtin_fmaf(f.y, f.y, a1);
      a0 = __builtin_fmaf(f.z, f.z, a0);
      a1 = __builtin_fmaf(f.w, f.w, a1);
    }
  } else {
    for (std::uint32_t i = threadIdx.x; i < d; i += blockDim.x) a0 = __builtin_fmaf(v[i], v[i], a0);
  }
  return BlockSumAny(a0 + a1, red);
}
// y[i] = fn(i, x[i]) for i < d.
template <typename Fn>
__device__ __forceinline__ void RowApply(const float* x, float* y, std::uint32_t d, Fn fn) {
  if (Vec4Ok(x, d) && Vec4Ok(y, d)) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float4* y4 = reinterpret_cast<float4*>(y);
    for (std::uint32_t i = threadIdx.x; i < d / 4; i += blockDim.x) {
      const float4 f = x4[i];
      y4[i] = make_float4(fn(4 * i, f.x), fn(4 * i + 1, f.y), fn(4 * i + 2, f.z), fn(4 * i + 3, f.w));
    }
  } else {
    for (std::uint32_t i = threadIdx.x; i < d; i += blockDim.x) y[i] = fn(i, x[i]);
  }
}
__device__ __forceinline__ float RmsScale(const float* v, std::uint32_t d, float eps, float* red) {
  return 1.0f / sqrtf(RowSumSq(v, d, red) / static_cast<float>(d) + eps);
}

// NEOX rotation of the first rotary_dim values of one head: pairs (i, i + rotary_dim / 2) rotate by
// pos * theta^(-2 i / rotary_dim).
__device__ __forceinline__ void RotateHead(float* v, std::uint32_t rotary_dim, std::uint32_t pos, float theta) {
  const std::uint32_t half = rotary_dim / 2;
  for (std::uint32_t i = threadIdx.x; i < half; i += blockDim.x) {
    const float ang = static_cast<float>(pos) * powf(theta, -2.0f * static_cast<float>(i) / static_cast<float>(rotary_dim));
    const float cs = cosf(ang), sn = sinf(ang);
    const float x0 = v[i], x1 = v[i + half];
    v[i] = x0 * cs - x1 * sn;
    v[i + half] = x0 * sn + x1 * cs;
  }
}

// Softmax(q . K^T / sqrt(hd)) V * sigmoid(gate) for one query head over n rows of a contiguous cache
// [pos][num_kv_heads][hd]: rows [0, n), or rows visible[0 .. n) when `visible` is given; sc is the head's score
// scratch (global, n entries). Scores: one wave per position, its lanes across hd (coalesced rows); weighted V:
// threads across hd.
__device__ void AttendHead(const float* qh, const float* kc, const float* vc, const float* gh, float* oh, float* sc,
                           std::uint32_t kvh, std::uint32_t num_kv_heads, std::uint32_t hd, std::uint32_t n,
                           float* red, const std::uint32_t* visible = nullptr) {
  const auto row = [&](std::uint32_t p) -> std::size_t {
    return (static_cast<std::size_t>(visible ? visible[p] : p) * num_kv_heads + kvh) * hd;
  };
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, nw = blockDim.x / kWave;
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));
  float mx = -INFINITY;
  for (std::uint32_t p = wave; p < n; p += nw) {
    const float* kp = kc + row(p);
    float dot = 0.0f;
    for (std::uint32_t i = lane; i < hd; i += kWave) dot += qh[i] * kp[i];
    dot = halo::GroupSum(dot) * scale;
    if (lane == 0) sc[p] = dot;
    mx = fmaxf(mx, dot);
  }
  mx = BlockMaxAny(mx, red);  // its barriers also publish sc to the block
  float den = 0.0f;
  for (std::uint32_t p = threadIdx.x; p < n; p += blockDim.x) {
    const float e = expf(sc[p] - mx);
    sc[p] = e;
    den += e;
  }
  den = BlockSumAny(den, red);
  for (std::uint32_t i = threadIdx.x; i < hd; i += blockDim.x) {
    float acc = 0.0f;
    for (std::uint32_t p = 0; p < n; ++p) acc += sc[p] * vc[row(p) + i];
    oh[i] = acc / den * halo::Sigmoid(gh[i]);
  }
}

}  // namespace halo::refk

using namespace halo::refk;

// y_b = x_b * w_b / rms(x_b), one block per vector b of d values; w_b = w_all + b * w_stride (core.hip:259).
extern "C" __global__ void halo_rmsnorm(const float* x, const float* w_all, float* y, std::uint32_t d, float eps,
                                        std::uint32_t w_stride) {
  __shared__ float red[16];
  const std::size_t b = blockIdx.x;
  const float* w = w_all + b * w_stride;
  const float inv = RmsScale(x + b * d, d, eps, red);
  RowApply(x + b * d, y + b * d, d, [&](std::uint32_t i, float v) { return v * inv * w[i]; });
}

// x_b /= sqrt(sum x_b^2 + eps) in place, one block per vector (core.hip:265).
extern "C" __global__ void halo_l2norm(float* x, std::uint32_t d, float eps) {
  __shared__ float red[16];
  float* xv = x + static_cast<std::size_t>(blockIdx.x) * d;
  const float inv = 1.0f / sqrtf(RowSumSq(xv, d, red) + eps);
  RowApply(xv, xv, d, [&](std::uint32_t, float v) { return v * inv; });
}

// NEOX RoPE in place, one block per head of head_dim values (core.hip:289-306): at position pos; rows of `heads`
// heads per token at pos0 + token; at params[slot] * scale.
extern "C" __global__ void halo_rope_neox(float* x, std::uint32_t head_dim, std::uint32_t rotary_dim, std::uint32_t pos,
                                          float theta) {
  RotateHead(x + static_cast<std::size_t>(blockIdx.x) * head_dim, rotary_dim, pos, theta);
}
extern "C" __global__ void halo_rope_neox_rows(float* x, std::uint32_t head_dim, std::uint32_t rotary_dim,
                                               std::uint32_t pos0, std::uint32_t heads, float theta) {
  RotateHead(x + static_cast<std::size_t>(blockIdx.x) * head_dim, rotary_dim, pos0 + blockIdx.x / heads, theta);
}
extern "C" __global__ void halo_rope_neox_p(float* x, const std::uint32_t* params, std::uint32_t head_dim,
                                            std::uint32_t rotary_dim, std::uint32_t slot, std::uint32_t scale,
                                            float theta) {
  RotateHead(x + static_cast<std::size_t>(blockIdx.x) * head_dim, rotary_dim, params[slot] * scale, theta);
}

// Grid-stride elementwise kernels (core.hip:313-362).
#define HALO_GRID_STRIDE(i, n) \
  for (std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += gridDim.x * blockDim.x)
extern "C" __global__ void halo_add(float* y, const float* x, std::uint32_t n) {
  HALO_GRID_STRIDE(i, n) y[i] += x[i];
}
extern "C" __global__ void halo_axpy(float* y, const float* x, float a, std::uint32_t n) {
  HALO_GRID_STRIDE(i, n) y[i] += a * x[i];
}
extern "C" __global__ void halo_silu_mul(float* g, const float* up, std::uint32_t n) {
  HALO_GRID_STRIDE(i, n) g[i] = halo::Silu(g[i]) * up[i];
}
extern "C" __global__ void halo_sigmoid_gate(float* x, const float* gate, std::uint32_t n) {
  HALO_GRID_STRIDE(i, n) x[i] *= halo::Sigmoid(gate[i]);
}
extern "C" __global__ void halo_copy(float* dst, const float* src, std::uint32_t n) {
  HALO_GRID_STRIDE(i, n) dst[i] = src[i];
}
// dst[params[slot] * stride + i] = src[i]: one row appended to a cache at the step's position.
extern "C" __global__ void halo_copy_at(float* dst, const float* src, const std::uint32_t* params, std::uint32_t slot,
                                        std::uint32_t stride, std::uint32_t n) {
  float* row = dst + static_cast<std::size_t>(params[slot]) * stride;
  HALO_GRID_STRIDE(i, n) row[i] = src[i];
}
#undef HALO_GRID_STRIDE

// [heads][2 hd] (q | gate per head) -> q [heads][hd], gate [heads][hd]; one block per head (core.hip:364).
extern "C" __global__ void halo_split_qgate(const float* qg, float* q, float* gate, std::uint32_t hd) {
  const std::size_t h = blockIdx.x;
  for (std::uint32_t i = threadIdx.x; i < hd; i += blockDim.x) {
    q[h * hd + i] = qg[h * 2 * hd + i];
    gate[h * hd + i] = qg[h * 2 * hd + hd + i];
  }
}

// ---- depthwise causal conv (DeltaNet q/k/v channels) -------------------------------------------------------------
// One arithmetic for every conv kernel below, so stepping, the one-token-per-block prefill and the eight-token prefill
// give the same bits: the taps of a channel against its window (oldest input first, the current input last) as one
// fused multiply-add chain starting from the oldest tap, then SiLU; the L2 norm of a head (d channels) from lane
// partials p_l = sum over m of v[l + 64 m]^2 (fused, m ascending) reduced over the wave (GroupSum).
// Conv state layout: [kern - 1][channels], slot j holds the input kern - 1 - j steps back (oldest first).
namespace halo::refk {
constexpr std::uint32_t kMaxTaps = 9;

__device__ __forceinline__ float ConvSilu(const float* wc, const float (&win)[kMaxTaps], std::uint32_t kern) {
  float acc = 0.0f;
#pragma unroll
  for (std::uint32_t j = 0; j < kMaxTaps; ++j)
    if (j < kern) acc = __builtin_fmaf(wc[j], win[j], acc);
  return halo::Silu(acc);
}

// Input i of a chunk's conv stream: i >= 0 is row i of the chunk, i < 0 the state slot kern - 1 + i.
__device__ __forceinline__ float ConvInput(const float* in, const float* state, std::int64_t i, std::uint32_t ch,
                                           std::uint32_t channels, std::uint32_t kern) {
  return i >= 0 ? in[static_cast<std::size_t>(i) * channels + ch]
                : state[static_cast<std::size_t>(i + kern - 1) * channels + ch];
}

// One decode step of channel ch: the window is the state then x; the state moves one slot (x becomes the newest).
__device__ __forceinline__ float ConvStep(const float* in, float* state, const float* w, std::uint32_t ch,
                                          std::uint32_t channels, std::uint32_t kern) {
  const float x = in[ch];
  float win[kMaxTaps];
#pragma unroll
  for (std::uint32_t j = 0; j < kMaxTaps; ++j)
    win[j] = j + 1 < kern ? state[static_cast<std::size_t>(j) * channels + ch] : (j + 1 == kern ? x : 0.0f);
#pragma unroll
  for (std::uint32_t j = 0; j + 1 < kMaxTaps; ++j)
    if (j + 1 < kern) state[static_cast<std::size_t>(j) * channels + ch] = win[j + 1];
  return ConvSilu(w + static_cast<std::size_t>(ch) * kern, win, kern);
}

// Sum of squares of a head whose channel i is thread i's y (block = one head, <= 256 threads): staged in LDS, then
// every wave forms the canonical lane partials and reduces them itself (identical bits in all waves).
__device__ __forceinline__ float HeadSumSq(float y, float* sh) {
  sh[threadIdx.x] = y;
  __syncthreads();
  const std::uint32_t lane = threadIdx.x % kWave;
  float p = 0.0f;
  for (std::uint32_t i = lane; i < blockDim.x; i += kWave) p = __builtin_fmaf(sh[i], sh[i], p);
  return halo::GroupSum(p);
}

// Block = one head of blockDim channels; heads that start below l2_channels are L2-normalised (block-uniform).
__device__ __forceinline__ void ConvL2norm(const float* in, float* state, const float* w, float* out,
                                           std::uint32_t channels, std::uint32_t kern, std::uint32_t l2_channels,
                                           float eps, float* sh) {
  const std::uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x;
  float y = ch < channels ? ConvStep(in, state, w, ch, channels, kern) : 0.0f;
  if (blockIdx.x * blockDim.x < l2_channels) y *= 1.0f / sqrtf(HeadSumSq(y, sh) + eps);
  if (ch < channels) out[ch] = y;
}
}  // namespace halo::refk

// Conv step + SiLU, one thread per channel; kern <= 9 (core.hip:447). grid (ceil(channels / blockDim)).
extern "C" __global__ void halo_conv_step(const float* in, float* state, const float* w, float* out,
                                          std::uint32_t channels, std::uint32_t kern) {
  const std::uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch < channels) out[ch] = ConvStep(in, state, w, ch, channels, kern);
}
// The conv step and the per-head L2 norm of q and k (core.hip:3003-3028). grid (ceil(channels / d)), block d <= 256.
extern "C" __global__ void halo_conv_l2norm(const float* in, float* state, const float* w, float* out,
                                            std::uint32_t channels, std::uint32_t kern, std::uint32_t l2_channels,
                                            float eps) {
  __shared__ float sh[256];
  ConvL2norm(in, state, w, out, channels, kern, l2_channels, eps, sh);
}

// One Gated DeltaNet decode step for any head size d <= 256 (core.hip:463), one block per value head h (key head
// h % num_k_heads), any block size that is a multiple of 64 (threads loop over value columns j). Single pass over the
// key-major state [h][i][j], in the algebraic form the d = 128 kernels use: with A = sum_i S_ij k_i and
// B = sum_i S_ij q_i over the old state, delta_j = (v_j - decay A) b, S'_ij = decay S_ij + k_i delta_j and
// o_j = (decay B + delta_j (k . q)) / sqrt(d); decay = exp(a softplus(alpha + dt)), b = sigmoid(beta).
extern "C" __global__ void halo_gdn_step(const float* q, const float* k, const float* v, const float* alpha,
                                         const float* beta, const float* a, const float* dt, float* state, float* out,
                                         std::uint32_t num_k_heads, std::uint32_t d) {
  __shared__ float kl[256], ql[256], red[16];
  const std::uint32_t h = blockIdx.x, kh = h % num_k_heads;
  float kq = 0.0f;
  for (std::uint32_t i = threadIdx.x; i < d; i += blockDim.x) {
    const float ki = k[static_cast<std::size_t>(kh) * d + i], qi = q[static_cast<std::size_t>(kh) * d + i];
    kl[i] = ki;
    ql[i] = qi;
    kq = __builtin_fmaf(ki, qi, kq);
  }
  kq = BlockSumAny(kq, red);  // its barriers publish kl / ql
  const float decay = expf(a[h] * halo::Softplus(alpha[h] + dt[h])), b = halo::Sigmoid(beta[h]);
  const float inv_sqrt_d = 1.0f / sqrtf(static_cast<float>(d));
  float* sh = state + static_cast<std::size_t>(h) * d * d;
  for (std::uint32_t j = threadIdx.x; j < d; j += blockDim.x) {
    float A0 = 0.0f, A1 = 0.0f, B0 = 0.0f, B1 = 0.0f;  // even / odd key rows: two independent chains each
    std::uint32_t i = 0;
    for (; i + 1 < d; i += 2) {
      const float s0 = sh[static_cast<std::size_t>(i) * d + j], s1 = sh[static_cast<std::size_t>(i + 1) * d + j];
      A0 = __builtin_fmaf(s0, kl[i], A0);
      B0 = __builtin_fmaf(s0, ql[i], B0);
      A1 = __builtin_fmaf(s1, kl[i + 1], A1);
      B1 = __builtin_fmaf(s1, ql[i + 1], B1);
    }
    if (i < d) {
      const float s0 = sh[static_cast<std::size_t>(i) * d + j];
      A0 = __builtin_fmaf(s0, kl[i], A0);
      B0 = __builtin_fmaf(s0, ql[i], B0);
    }
    const float delta = (v[static_cast<std::size_t>(h) * d + j] - decay * (A0 + A1)) * b;
    for (std::uint32_t r = 0; r < d; ++r) {
      float* s = sh + static_cast<std::size_t>(r) * d + j;
      *s = __builtin_fmaf(kl[r], delta, decay * *s);
    }
    out[static_cast<std::size_t>(h) * d + j] = (decay * (B0 + B1) + delta * kq) * inv_sqrt_d;
  }
}

namespace {
// The single-pass d = 128 step (core.hip:2621-2650): A = S k and B = S q over the old state, delta = (v - decay A) b,
// S' = decay S + delta k^T, o = (decay B + delta (k . q)) / sqrt(d). Block 128, thread j = value column; the column
// is held in registers between the read and the write.
__device__ __forceinline__ float GdnStepD128(const float* q, const float* k, const float* v, const float* alpha,
                                             const float* beta, const float* a, const float* dt, float* state,
                                             std::uint32_t num_k_heads, float* kl, float* ql, float* red) {
  constexpr std::uint32_t d = 128;
  const std::uint32_t h = blockIdx.x, j = threadIdx.x, kh = h % num_k_heads;
  const float kj = k[static_cast<std::size_t>(kh) * d + j], qj = q[static_cast<std::size_t>(kh) * d + j];
  kl[j] = kj;
  ql[j] = qj;
  float* col = state + static_cast<std::size_t>(h) * d * d + j;
  const float kq = BlockSumAny(kj * qj, red);  // its barriers publish kl / ql
  const float decay = expf(a[h] * halo::Softplus(alpha[h] + dt[h])), b = halo::Sigmoid(beta[h]);
  // A and B over the old column (16 loads in flight per chunk), then the update reads it again (an L2 hit) and
  // writes it once
  float A = 0.0f, B = 0.0f;
#pragma unroll 1
  for (std::uint32_t i0 = 0; i0 < d; i0 += 16) {
    float s[16];
#pragma unroll
    for (std::uint32_t i = 0; i < 16; ++i) s[i] = col[(i0 + i) * d];
#pragma unroll
    for (std::uint32_t i = 0; i < 16; ++i) {
      A += s[i] * kl[i0 + i];
      B += s[i] * ql[i0 + i];
    }
  }
  const float delta = (v[static_cast<std::size_t>(h) * d + j] - decay * A) * b;
#pragma unroll 1
  for (std::uint32_t i0 = 0; i0 < d; i0 += 16) {
    float s[16];
#pragma unroll
    for (std::uint32_t i = 0; i < 16; ++i) s[i] = col[(i0 + i) * d];
#pragma unroll
    for (std::uint32_t i = 0; i < 16; ++i) col[(i0 + i) * d] = decay * s[i] + delta * kl[i0 + i];
  }
  return (decay * B + delta * kq) / sqrtf(static_cast<float>(d));
}
}  // namespace

extern "C" __global__ void __launch_bounds__(128)
    halo_gdn_step_d128(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                       const float* a, const float* dt, float* state, float* out, std::uint32_t num_k_heads) {
  __shared__ float kl[128], ql[128], red[2];
  const float o = GdnStepD128(q, k, v, alpha, beta, a, dt, state, num_k_heads, kl, ql, red);
  out[static_cast<std::size_t>(blockIdx.x) * 128 + threadIdx.x] = o;
}

// The d = 128 step with the per-head gated RMSNorm in the epilogue: o * w / rms(o) * (silu(z) for mode 0, sigmoid(z)
// for mode 1) (core.hip:3030-3063).
extern "C" __global__ void __launch_bounds__(128)
    halo_gdn_step_d128_norm(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                            const float* a, const float* dt, float* state, const float* norm_w, const float* z,
                            float* out, std::uint32_t num_k_heads, float eps, std::uint32_t mode) {
  __shared__ float kl[128], ql[128], red[2];
  const float o = GdnStepD128(q, k, v, alpha, beta, a, dt, state, num_k_heads, kl, ql, red);
  const float inv = 1.0f / sqrtf(BlockSumAny(o * o, red) / 128.0f + eps);
  const std::size_t at = static_cast<std::size_t>(blockIdx.x) * 128 + threadIdx.x;
  const float zv = z[at];
  out[at] = o * inv * norm_w[threadIdx.x] * (mode == 0 ? halo::Silu(zv) : halo::Sigmoid(zv));
}

// Per-head RMSNorm * w * (silu(z) mode 0, sigmoid(z) mode 1), in place; one block per head (core.hip:497).
extern "C" __global__ void halo_gated_norm(float* o, const float* w, const float* z, std::uint32_t d, float eps,
                                           std::uint32_t mode) {
  __shared__ float red[16];
  float* ov = o + static_cast<std::size_t>(blockIdx.x) * d;
  const float* zv = z + static_cast<std::size_t>(blockIdx.x) * d;
  const float inv = RmsScale(ov, d, eps, red);
  if (mode == 0)
    RowApply(ov, ov, d, [&](std::uint32_t i, float v) { return v * inv * w[i] * halo::Silu(zv[i]); });
  else
    RowApply(ov, ov, d, [&](std::uint32_t i, float v) { return v * inv * w[i] * halo::Sigmoid(zv[i]); });
}

// Decode attention over positions [0, n) of a contiguous cache [pos][num_kv_heads][hd], one block per query head
// (kv head = h / (num_heads / num_kv_heads)), output gated by sigmoid(gate); scores [num_heads][max_n] scratch
// (core.hip:514).
extern "C" __global__ void halo_attention_decode(const float* q, const float* kc, const float* vc, const float* gate,
                                                 float* out, float* scores, std::uint32_t num_heads,
                                                 std::uint32_t num_kv_heads, std::uint32_t hd, std::uint32_t n,
                                                 std::uint32_t max_n) {
  __shared__ float red[16];
  const std::uint32_t h = blockIdx.x, kvh = h / (num_heads / num_kv_heads);
  const std::size_t row = static_cast<std::size_t>(h) * hd;
  AttendHead(q + row, kc, vc, gate + row, out + row, scores + static_cast<std::size_t>(h) * max_n, kvh, num_kv_heads,
             hd, n, red);
}

// The same for a chunk of T queries (grid (num_heads, T)): query t at position pos0 + t attends to [0, pos0 + t]
// (core.hip:551). q, gate, out [T][num_heads][hd]; scores [T][num_heads][max_n].
extern "C" __global__ void halo_attention_prefill(const float* q, const float* kc, const float* vc, const float* gate,
                                                  float* out, float* scores, std::uint32_t num_heads,
                                                  std::uint32_t num_kv_heads, std::uint32_t hd, std::uint32_t pos0,
                                                  std::uint32_t max_n) {
  __shared__ float red[16];
  const std::uint32_t h = blockIdx.x, t = blockIdx.y, kvh = h / (num_heads / num_kv_heads);
  const std::size_t row = (static_cast<std::size_t>(t) * num_heads + h) * hd;
  AttendHead(q + row, kc, vc, gate + row, out + row,
             scores + (static_cast<std::size_t>(t) * num_heads + h) * max_n, kvh, num_kv_heads, hd, pos0 + t + 1, red);
}

// Attention over a list of visible cache rows (core.hip:783-820, 898-903, 909-918): n = params[5] (the step
// parameters' visible count), rows visible[0 .. n) of the contiguous cache, one block per query head; scores
// [num_heads][max_n]. _b is the same kernel under the name the decode engine launches; _rows takes token t =
// blockIdx.y with q, gate, out [T][num_heads][hd], visible lists max_n apart, scores num_heads * max_n apart and
// step parameters 16 words apart.
#define HALO_ATTN_SELECT(NAME)                                                                                     \
  extern "C" __global__ void __launch_bounds__(256)                                                              \
      NAME(const float* q, const float* kc, const float* vc, const float* gate, const std::uint32_t* visible,    \
           float* out, float* scores, const std::uint32_t* params, std::uint32_t num_heads,                      \
           std::uint32_t num_kv_heads, std::uint32_t hd, std::uint32_t max_n) {                                  \
    __shared__ float red[16];                                                                                    \
    const std::uint32_t h = blockIdx.x, kvh = h / (num_heads / num_kv_heads);                                    \
    const std::size_t row = static_cast<std::size_t>(h) * hd;                                                    \
    AttendHead(q + row, kc, vc, gate + row, out + row, scores + static_cast<std::size_t>(h) * max_n, kvh,        \
               num_kv_heads, hd, params[5], red, visible);                                                       \
  }
HALO_ATTN_SELECT(halo_attention_select)
HALO_ATTN_SELECT(halo_attention_select_b)
#undef HALO_ATTN_SELECT
extern "C" __global__ void __launch_bounds__(256)
    halo_attention_select_rows(const float* q, const float* kc, const float* vc, const float* gate,
                               const std::uint32_t* visible, float* out, float* scores, const std::uint32_t* params,
                               std::uint32_t num_heads, std::uint32_t num_kv_heads, std::uint32_t hd,
                               std::uint32_t max_n) {
  __shared__ float red[16];
  const std::uint32_t h = blockIdx.x, t = blockIdx.y, kvh = h / (num_heads / num_kv_heads);
  const std::size_t row = (static_cast<std::size_t>(t) * num_heads + h) * hd;
  AttendHead(q + row, kc, vc, gate + row, out + row,
             scores + (static_cast<std::size_t>(t) * num_heads + h) * max_n, kvh, num_kv_heads, hd,
             params[static_cast<std::size_t>(t) * 16 + 5], red, visible + static_cast<std::size_t>(t) * max_n);
}

// ---- Q8_0 GEMV variants, expert GEMVs, MoE down/combine, few-row fp32 matvecs (reference names) -------------
// reference src/kernels/core.hip:2183-2211, 2362-2378, 2436-2458, 2988-3000, 3313-3330, 9263-9285, 9401-9416,
// 9642-9700. Grids as the reference launches them: the Q8 GEMVs take ceil(rows / 8) blocks of 256 (ceil(rows / 32)
// for the _r4 / _r4n variants), the MoE down kernels a second grid dimension over the expert slots, the rowblock
// matvecs one block per output row. Repacked experts are stacked [experts][rows][qstride] int8 + [experts][rows]
// [cols / 32] fp16. The fp32-x GEMV body is GemvQ8rF32 (wave64: two rows per wave per pass, x from the vector
// cache, so no column limit of an LDS copy of x).
extern "C" __global__ void __launch_bounds__(256)
    halo_gemv_q8r_wide(const std::int8_t* qs, const std::uint16_t* d, const float* x, float* y, std::uint32_t rows,
                       std::uint32_t cols, std::uint32_t qstride) {
  GemvQ8rF32<1>(qs, d, x, y, rows, cols, qstride);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_gemv_q8r_r4n(const std::int8_t* qs, const std::uint16_t* d, const float* x, float* y, std::uint32_t rows,
                      std::uint32_t cols, std::uint32_t qstride) {
  GemvQ8rF32<4>(qs, d, x, y, rows, cols, qstride);
}
// Expert ids[slot] of the stacked tensor.
extern "C" __global__ void __launch_bounds__(256)
    halo_gemv_q8r_expert(const std::int8_t* qs, const std::uint16_t* d, const std::uint32_t* ids, const float* x,
                         float* y, std::uint32_t slot, std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride) {
  const std::size_t e = ids[slot];
  GemvQ8rF32<1>(qs + e * rows * qstride, d + e * rows * (cols / 32), x, y, rows, cols, qstride);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_gemv_q8r_expert_r4(const std::int8_t* qs, const std::uint16_t* d, const std::uint32_t* ids,
                            const float* x, float* y, std::uint32_t slot, std::uint32_t rows, std::uint32_t cols,
                            std::uint32_t qstride) {
  const std::size_t e = ids[slot];
  GemvQ8rF32<4>(qs + e * rows * qstride, d + e * rows * (cols / 32), x, y, rows, cols, qstride);
}
// Down projections of every routed slot in one launch: grid.y = slots; h [slots][cols] -> part [slots][rows].
extern "C" __global__ void __launch_bounds__(256)
    halo_moe_down_q8r(const std::int8_t* qs, const std::uint16_t* d, const std::uint32_t* ids, const float* h,
                      float* part, std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride) {
  const std::size_t slot = blockIdx.y, e = ids[slot];
  GemvQ8rF32<1>(qs + e * rows * qstride, d + e * rows * (cols / 32), h + slot * cols, part + slot * rows, rows, cols,
                qstride);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_moe_down_q8r_r4(const std::int8_t* qs, const std::uint16_t* d, const std::uint32_t* ids, const float* h,
                         float* part, std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride) {
  const std::size_t slot = blockIdx.y, e = ids[slot];
  GemvQ8rF32<4>(qs + e * rows * qstride, d + e * rows * (cols / 32), h + slot * cols, part + slot * rows, rows, cols,
                qstride);
}

namespace halo::refk {
// out[i] = sum over slots s, in slot order, of weights[s] * part[s][i] (fused multiply-add chain). Grid-stride.
template <bool kUnrolled>
__device__ __forceinline__ void Combine(const float* part, const float* weights, float* out, std::uint32_t slots,
                                        std::uint32_t n) {
  for (std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    float acc = 0.0f;
    if constexpr (kUnrolled) {
      float p[16];  // every slot's load issued before the chain
#pragma unroll
      for (std::uint32_t s = 0; s < 16; ++s) p[s] = s < slots ? part[static_cast<std::size_t>(s) * n + i] : 0.0f;
#pragma unroll
      for (std::uint32_t s = 0; s < 16; ++s)
        if (s < slots) acc = __builtin_fmaf(weights[s], p[s], acc);
    } else {
      for (std::uint32_t s = 0; s < slots; ++s)
        acc = __builtin_fmaf(weights[s], part[static_cast<std::size_t>(s) * n + i], acc);
    }
    out[i] = acc;
  }
}
// y = row . x for one row per block. 16-byte loads when cols and the row allow them: each thread takes float4 pairs
// (two loads in flight, two fused chains), then BlockSumAny.
__device__ __forceinline__ float RowDot(const float* row, const float* x, std::uint32_t cols, float* red) {
  float a0 = 0.0f, a1 = 0.0f;
  if (Vec4Ok(row, cols) && Vec4Ok(x, cols)) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const std::uint32_t n4 = cols / 4;
    std::uint32_t i = threadIdx.x;
    for (; i + blockDim.x < n4; i += 2 * blockDim.x) {
      const float4 p = r4[i], u = x4[i], p2 = r4[i + blockDim.x], u2 = x4[i + blockDim.x];
      a0 = __builtin_fmaf(p.w, u.w, __builtin_fmaf(p.z, u.z, __builtin_fmaf(p.y, u.y, __builtin_fmaf(p.x, u.x, a0))));
      a1 = __builtin_fmaf(p2.w, u2.w,
                          __builtin_fmaf(p2.z, u2.z, __builtin_fmaf(p2.y, u2.y, __builtin_fmaf(p2.x, u2.x, a1))));
    }
    if (i < n4) {
      const float4 p = r4[i], u = x4[i];
      a0 = __builtin_fmaf(p.w, u.w, __builtin_fmaf(p.z, u.z, __builtin_fmaf(p.y, u.y, __builtin_fmaf(p.x, u.x, a0))));
    }
  } else {
    for (std::uint32_t c = threadIdx.x; c < cols; c += blockDim.x) a0 = __builtin_fmaf(row[c], x[c], a0);
  }
  return BlockSumAny(a0 + a1, red);
}

// The rowblock matvecs: block b computes row b % rows of matrix b / rows (kMats matrices with the same x).
template <int kMats>
__device__ __forceinline__ void RowblockMatvec(const float* const (&w)[kMats], const float* x, float* const (&y)[kMats],
                                               std::uint32_t rows, std::uint32_t cols) {
  __shared__ float red[16];
  const std::uint32_t m = blockIdx.x / rows, r = blockIdx.x % rows;
  if (m >= static_cast<std::uint32_t>(kMats)) return;  // block-uniform
  const float acc = RowDot(w[m] + static_cast<std::size_t>(r) * cols, x, cols, red);
  if (threadIdx.x == 0) y[m][r] = acc;
}
}  // namespace halo::refk

// n <= any; grid-stride over the n outputs.
extern "C" __global__ void __launch_bounds__(256)
    halo_moe_combine(const float* part, const float* weights, float* out, std::uint32_t slots, std::uint32_t n) {
  halo::refk::Combine<false>(part, weights, out, slots, n);
}
// slots <= 16.
extern "C" __global__ void __launch_bounds__(256)
    halo_moe_combine_u(const float* part, const float* weights, float* out, std::uint32_t slots, std::uint32_t n) {
  halo::refk::Combine<true>(part, weights, out, slots, n);
}
// grid (rows), any multiple of 64 threads: y[r] = w[r] . x (core.hip:2193, 9264).
extern "C" __global__ void __launch_bounds__(256)
    halo_matvec_f32_rowblock(const float* w, const float* x, float* y, std::uint32_t rows, std::uint32_t cols) {
  RowblockMatvec<1>({w}, x, {y}, rows, cols);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_matvec_f32_rowblock_u(const float* w, const float* x, float* y, std::uint32_t rows, std::uint32_t cols) {
  RowblockMatvec<1>({w}, x, {y}, rows, cols);
}
// grid (2 rows): blocks [0, rows) compute ya = wa x, blocks [rows, 2 rows) yb = wb x.
extern "C" __global__ void __launch_bounds__(256)
    halo_matvec_f32_rowblock2(const float* wa, const float* wb, const float* x, float* ya, float* yb,
                              std::uint32_t rows, std::uint32_t cols) {
  RowblockMatvec<2>({wa, wb}, x, {ya, yb}, rows, cols);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_matvec_f32_rowblock2_u(const float* wa, const float* wb, const float* x, float* ya, float* yb,
                                std::uint32_t rows, std::uint32_t cols) {
  RowblockMatvec<2>({wa, wb}, x, {ya, yb}, rows, cols);
}
// Per token and 32 values (amax / 127, round half to even, as halo_quantize_q8_rows), K-blocked (core.hip:3317-3331):
// x [T][cols] -> xq [cols / 64][T][64], xd [cols / 32][T]. A lane quantizes 4 values from one 16-byte load; 8 lanes
// form a Q8_0 block (QuantQuad) and store their codes as one 32-byte run. grid (T), any multiple of 64 threads;
// cols % 64 == 0.
extern "C" __global__ void __launch_bounds__(256)
    halo_quantize_q8_kblocked(const float* x, std::int8_t* xq, float* xd, std::uint32_t cols, std::uint32_t tokens) {
  const std::size_t t = blockIdx.x;
  const float4* row = reinterpret_cast<const float4*>(x + t * cols);
  for (std::uint32_t g = threadIdx.x; g < cols / 4; g += blockDim.x) {  // groups of 8 lanes stay whole (cols % 32)
    float scale;
    const std::uint32_t word = halo::QuantQuad(row[g], scale), c = 4 * g;
    *reinterpret_cast<std::uint32_t*>(xq + (static_cast<std::size_t>(c / 64) * tokens + t) * 64 + c % 64) = word;
    if (g % 8 == 0) xd[static_cast<std::size_t>(c / 32) * tokens + t] = scale;
  }
}
// halo_router_topk's results (softmax, top k in (probability desc, index asc) order, weights renormalized in slot
// order) with the reference's 256-thread launch: the first wave does the work. n <= 1024, k <= 16.
extern "C" __global__ void __launch_bounds__(256)
    halo_router_topk_w(const float* logits, std::uint32_t* ids, float* weights, std::uint32_t n, std::uint32_t k) {
  __shared__ std::uint32_t scratch[64];
  __shared__ float wscratch[64];
  __shared__ TopKScratch sc;
  if (threadIdx.x >= kWave) return;
  WaveTopK<16>(logits, n, k, ids, weights, scratch, wscratch, sc);
}

// ---- DeltaNet prefill helpers and the chunk-stepped d = 128 step (reference names) ------------------------------
// core.hip:3480-3500, 3586-3597, 3612-3662, 9590-9636.

// halo_gdn_step_d128_norm under the name of the reference's two-pass variant (this implementation is two-pass).
extern "C" __global__ void __launch_bounds__(128)
    halo_gdn_step_d128_norm_r(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                              const float* a, const float* dt, float* state, const float* norm_w, const float* z,
                              float* out, std::uint32_t num_k_heads, float eps, std::uint32_t mode) {
  __shared__ float kl[128], ql[128], red[2];
  const float o = GdnStepD128(q, k, v, alpha, beta, a, dt, state, num_k_heads, kl, ql, red);
  const float inv = 1.0f / sqrtf(BlockSumAny(o * o, red) / 128.0f + eps);
  const std::size_t at = static_cast<std::size_t>(blockIdx.x) * 128 + threadIdx.x;
  const float zv = z[at];
  out[at] = o * inv * norm_w[threadIdx.x] * (mode == 0 ? halo::Silu(zv) : halo::Sigmoid(zv));
}

// halo_gdn_step_d128_norm over T tokens in one launch, token by token with the same arithmetic (each token's output
// and the final state equal T single steps bit for bit). Row t of q and k at t * qk_stride, of v at t * v_stride, of
// z and out at t * zo_stride; alpha, beta [T][heads]. grid (heads), block 128.
extern "C" __global__ void __launch_bounds__(128)
    halo_gdn_prefill_d128_norm(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                               const float* a, const float* dt, float* state, const float* norm_w, const float* z,
                               float* out, std::uint32_t num_k_heads, float eps, std::uint32_t mode,
                               std::uint32_t tokens, std::uint32_t qk_stride, std::uint32_t v_stride,
                               std::uint32_t zo_stride) {
  __shared__ float kl[128], ql[128], red[2];
  const std::uint32_t heads = gridDim.x;
  const float wj = norm_w[threadIdx.x];
  for (std::uint32_t t = 0; t < tokens; ++t) {
    const std::size_t qk = static_cast<std::size_t>(t) * qk_stride, ab = static_cast<std::size_t>(t) * heads;
    // the previous token's last block sum ends with barriers after every read of kl / ql
    const float o = GdnStepD128(q + qk, k + qk, v + static_cast<std::size_t>(t) * v_stride, alpha + ab, beta + ab, a,
                                dt, state, num_k_heads, kl, ql, red);
    const float inv = 1.0f / sqrtf(BlockSumAny(o * o, red) / 128.0f + eps);
    const std::size_t at = static_cast<std::size_t>(t) * zo_stride + static_cast<std::size_t>(blockIdx.x) * 128 +
                           threadIdx.x;
    const float zv = z[at];
    out[at] = o * inv * wj * (mode == 0 ? halo::Silu(zv) : halo::Sigmoid(zv));
  }
}

// halo_conv_l2norm for T tokens at once (core.hip:3480-3508): token t's window is inputs t - kern + 1 .. t of the
// chunk, reaching back into the conv state before the chunk; same arithmetic as stepping, so every output equals the
// step's bits. The state is only read (halo_conv_state_advance moves it after the chunk).
//   in, out [T][channels]; grid (ceil(channels / d), T), block d <= 256 (one head).
extern "C" __global__ void halo_conv_l2norm_prefill(const float* in, const float* state, const float* w, float* out,
                                                    std::uint32_t channels, std::uint32_t kern,
                                                    std::uint32_t l2_channels, float eps) {
  __shared__ float sh[256];
  const std::uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x;
  const std::int64_t t = blockIdx.y;
  float y = 0.0f;
  if (ch < channels) {
    float win[kMaxTaps];
#pragma unroll
    for (std::uint32_t j = 0; j < kMaxTaps; ++j)
      win[j] = j < kern ? ConvInput(in, state, t - static_cast<std::int64_t>(kern - 1 - j), ch, channels, kern) : 0.0f;
    y = ConvSilu(w + static_cast<std::size_t>(ch) * kern, win, kern);
  }
  if (blockIdx.x * blockDim.x < l2_channels) y *= 1.0f / sqrtf(HeadSumSq(y, sh) + eps);
  if (ch < channels) out[static_cast<std::size_t>(t) * channels + ch] = y;
}

// The conv state after a chunk of T inputs (core.hip:3586-3597): slot j becomes stream input T - kern + 1 + j. Slots
// are rewritten in ascending order, so a slot that moves down within the state is read before it is overwritten.
// grid (ceil(channels / blockDim)); kern <= 9.
extern "C" __global__ void halo_conv_state_advance(const float* in, float* state, std::uint32_t channels,
                                                   std::uint32_t kern, std::uint32_t tokens) {
  const std::uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= channels) return;
  for (std::uint32_t j = 0; j + 1 < kern; ++j) {
    const std::int64_t i = static_cast<std::int64_t>(tokens) + j - (kern - 1);
    state[static_cast<std::size_t>(j) * channels + ch] = ConvInput(in, state, i, ch, channels, kern);
  }
}

// ---- router with the expert activations quantized, shared expert (reference names) --------------------------------
// core.hip:2657-2661, 9196-9230, 9284-9343, 9418-9446.
namespace halo::refk {
// Q8_0 row r of [rows][qstride] int8 + [rows][cols / 32] fp16 dotted with fp32 x (cols % 1024 == 0 not required:
// cols % 16 == 0); every lane of the wave gets the sum.
__device__ __forceinline__ float Q8RowDot(const std::int8_t* qs, const std::uint16_t* d, const float* x,
                                          std::uint32_t r, std::uint32_t cols, std::uint32_t qstride) {
  const std::uint32_t lane = threadIdx.x % kWave, nblk = cols / 32;
  float acc = 0.0f;
  for (std::uint32_t c = lane * 16; c < cols; c += kWave * 16) {
    const int4 qv = *reinterpret_cast<const int4*>(qs + static_cast<std::size_t>(r) * qstride + c);
    const std::int8_t* q8 = reinterpret_cast<const std::int8_t*>(&qv);
    const float4* xp = reinterpret_cast<const float4*>(x + c);
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 xv = xp[i];
      part += static_cast<float>(q8[4 * i]) * xv.x + static_cast<float>(q8[4 * i + 1]) * xv.y +
              static_cast<float>(q8[4 * i + 2]) * xv.z + static_cast<float>(q8[4 * i + 3]) * xv.w;
    }
    acc += halo::F16(d[static_cast<std::size_t>(r) * nblk + c / 32]) * part;
  }
  return halo::GroupSum(acc);
}

// The shared expert's gate/up: h[r] = SiLU(gate_r . x) * (up_r . x), 16 rows per block (4 per wave); block 0 also
// writes sgate[0] = gate_inp . x.
__device__ __forceinline__ void ShexpGateUp(const std::int8_t* gq, const std::uint16_t* gd, const std::int8_t* uq,
                                            const std::uint16_t* ud, const float* gate_inp, const float* x, float* h,
                                            float* sgate, std::uint32_t rows, std::uint32_t cols,
                                            std::uint32_t qstride, float* red) {
  if (blockIdx.x == 0) {
    const float s = RowDot(gate_inp, x, cols, red);
    if (threadIdx.x == 0) sgate[0] = s;
  }
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const std::uint32_t per_wave = 16 / (blockDim.x / kWave);
  for (std::uint32_t k = 0; k < per_wave; ++k) {
    const std::uint32_t r = blockIdx.x * 16 + wave * per_wave + k;
    if (r >= rows) break;
    const float g = Q8RowDot(gq, gd, x, r, cols, qstride), u = Q8RowDot(uq, ud, x, r, cols, qstride);
    if (lane == 0) h[r] = halo::Silu(g) * u;
  }
}

// out[r] = sum over slots s, in slot order, of weights[s] * part[s][r], + sigmoid(sgate[0]) * (down_r . hin); 32 rows
// per block (8 per wave).
__device__ __forceinline__ void ShexpDownCombine(const std::int8_t* dq, const std::uint16_t* dd, const float* hin,
                                                 const float* sgate, const float* part, const float* weights,
                                                 std::uint32_t slots, float* out, std::uint32_t rows,
                                                 std::uint32_t cols, std::uint32_t qstride) {
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const std::uint32_t per_wave = 32 / (blockDim.x / kWave);
  const float s = halo::Sigmoid(sgate[0]);
  for (std::uint32_t k = 0; k < per_wave; ++k) {
    const std::uint32_t r = blockIdx.x * 32 + wave * per_wave + k;
    if (r >= rows) break;
    const float y = Q8RowDot(dq, dd, hin, r, cols, qstride);
    if (lane == 0) {
      float acc = 0.0f;
      for (std::uint32_t sl = 0; sl < slots; ++sl)
        acc = __builtin_fmaf(weights[sl], part[static_cast<std::size_t>(sl) * rows + r], acc);
      out[r] = acc + s * y;
    }
  }
}
}  // namespace halo::refk

// grid (ceil(rows / 16)), block 256.
extern "C" __global__ void __launch_bounds__(256)
    halo_shexp_gate_up(const std::int8_t* gq, const std::uint16_t* gd, const std::int8_t* uq, const std::uint16_t* ud,
                       const float* gate_inp, const float* x, float* h, float* sgate, std::uint32_t rows,
                       std::uint32_t cols, std::uint32_t qstride) {
  __shared__ float red[16];
  ShexpGateUp(gq, gd, uq, ud, gate_inp, x, h, sgate, rows, cols, qstride, red);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_shexp_gate_up_u(const std::int8_t* gq, const std::uint16_t* gd, const std::int8_t* uq,
                         const std::uint16_t* ud, const float* gate_inp, const float* x, float* h, float* sgate,
                         std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride) {
  __shared__ float red[16];
  ShexpGateUp(gq, gd, uq, ud, gate_inp, x, h, sgate, rows, cols, qstride, red);
}
// grid (ceil(rows / 32)), block 256; _u: slots <= 32.
extern "C" __global__ void __launch_bounds__(256)
    halo_shexp_down_combine(const std::int8_t* dq, const std::uint16_t* dd, const float* hin, const float* sgate,
                            const float* part, const float* weights, std::uint32_t slots, float* out,
                            std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride) {
  ShexpDownCombine(dq, dd, hin, sgate, part, weights, slots, out, rows, cols, qstride);
}
extern "C" __global__ void __launch_bounds__(256)
    halo_shexp_down_combine_u(const std::int8_t* dq, const std::uint16_t* dd, const float* hin, const float* sgate,
                              const float* part, const float* weights, std::uint32_t slots, float* out,
                              std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride) {
  ShexpDownCombine(dq, dd, hin, sgate, part, weights, slots, out, rows, cols, qstride);
}

// Router logits y[r] = w_r . x (block r < rows) and, in blocks b < cols / 32, the Q8 activation record of x's 32-value
// block b (core.hip:9315-9343; act: int8 codes [4096] four to a little-endian word, fp32 scale [128] = amax / 127,
// fp32 block sum [128]; cols <= 4096). The record takes lanes 0-7 of the first wave, one 16-byte load each: the codes
// come from QuantQuad, the sum is each lane's (x0 + x1) + (x2 + x3) added across the 8 lanes by Group8Sum.
// grid (max(rows, cols / 32)), block 256.
extern "C" __global__ void __launch_bounds__(256)
    halo_router_rowblock_q8act(const float* w, const float* x, float* y, std::uint32_t rows, std::uint32_t cols,
                               void* act) {
  __shared__ float red[16];
  const std::uint32_t blk = blockIdx.x;
  if (blk < cols / 32 && threadIdx.x < 8) {
    std::uint32_t* aq = static_cast<std::uint32_t*>(act);
    float* ascale = reinterpret_cast<float*>(aq + 1024);
    const float4 v = reinterpret_cast<const float4*>(x + blk * 32)[threadIdx.x];
    float scale;
    aq[blk * 8 + threadIdx.x] = halo::QuantQuad(v, scale);
    const float sum = halo::Group8Sum((v.x + v.y) + (v.z + v.w));
    if (threadIdx.x == 0) {
      ascale[blk] = scale;
      ascale[128 + blk] = sum;
    }
  }
  if (blk >= rows) return;  // block-uniform
  const float acc = RowDot(w + static_cast<std::size_t>(blk) * cols, x, cols, red);
  if (threadIdx.x == 0) y[blk] = acc;
}

// ---- prefill int8 GEMMs (reference names) ---------------------------------------------------------------------
// core.hip:3103-3153, 3303-3311, 3466-3476: y[t][r] = sum over Q8_0 blocks of the exact int32 block product scaled by
// d_w[r] s_x[t] (y [T][rows], ystride = rows), on the LDS-tiled int8 MFMA template. The _wmma kernels read
// activations as halo_quantize_q8_rows writes them (xq [T][cols], xd [T][cols / 32]); the q8a8 kernels read the
// K-blocked layout of halo_quantize_q8_kblocked (xq [cols / 64][T][64], xd [cols / 32][T]). Grids as the reference
// launches them: (ceil(T / BN), ceil(rows / BM)). Every tile here is a whole number of 32 x 32 MFMA tiles, so
// cols % 64 == 0 (every matrix of the model; the reference itself needs cols % 32 == 0 for _wmma).
#define HALO_REF_GEMM(NAME, BLOCK, BM, BN, WR, MT, WT, KB)                                                      \
  extern "C" __global__ void __launch_bounds__(BLOCK)                                                          \
      NAME(const std::int8_t* qs, const std::uint16_t* d, const std::int8_t* xq, const float* xd, float* y,   \
           std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride, std::uint32_t tokens) {             \
    if (threadIdx.x >= WR * WT * 64) return; /* tiles that need fewer waves than the reference's block */      \
    const std::uint32_t t0 = blockIdx.x * BN;                                                                  \
    halo::GemmTileQ8<WR, MT, WT, 1, false, KB>(qs, d, nullptr, nullptr, rows, qstride, blockIdx.y * BM, xq, xd, \
                                               nullptr, t0, min(static_cast<std::uint32_t>(BN), tokens - t0),  \
                                               cols, y, t0, rows, tokens);                                    \
  }
HALO_REF_GEMM(halo_gemm_q8r_wmma, 128, 64, 64, 1, 2, 2, false)
HALO_REF_GEMM(halo_gemm_q8r_wmma_t, 256, 128, 128, 1, 4, 4, false)
HALO_REF_GEMM(halo_gemm_q8a8_128x128, 256, 128, 128, 1, 4, 4, true)
HALO_REF_GEMM(halo_gemm_q8a8_128x64, 256, 128, 64, 2, 2, 2, true)
HALO_REF_GEMM(halo_gemm_q8a8_320x64, 256, 320, 64, 2, 5, 2, true)
HALO_REF_GEMM(halo_gemm_q8a8_160x64, 256, 160, 64, 1, 5, 2, true)
HALO_REF_GEMM(halo_gemm_q8a8_256x128, 256, 256, 128, 1, 8, 4, true)
#undef HALO_REF_GEMM

// Two Q8_0 matrices with the same fp32 input in one launch (core.hip:2960-2985, DeltaNet qkv and z): row blocks
// [0, blocks1) take matrix 1, the rest matrix 2; 32 rows per block of 256. x is read through the vector cache (no
// column limit).
extern "C" __global__ void __launch_bounds__(256)
    halo_gemv_q8r_dual(const std::int8_t* q1, const std::uint16_t* d1, float* y1, std::uint32_t rows1,
                       std::uint32_t qstride1, const std::int8_t* q2, const std::uint16_t* d2, float* y2,
                       std::uint32_t rows2, std::uint32_t qstride2, const float* x, std::uint32_t cols,
                       std::uint32_t blocks1) {
  const bool first = blockIdx.x < blocks1;
  GemvQ8rF32At<4>(first ? q1 : q2, first ? d1 : d2, x, first ? y1 : y2, first ? rows1 : rows2, cols,
                  first ? qstride1 : qstride2, first ? blockIdx.x : blockIdx.x - blocks1);
}

// ---- routed experts across session columns, grouped by expert (reference names) -----------------------------
// batch_decode.hip:415-446, 646-697.

// ids [n = NB k] (column b's slot s at b k + s; an expert at most once a column) -> ucount, the distinct experts
// uexp[u] in order of first appearance, their pair counts unum[u] and pairs upair[u * 8 + j] in pair order. One block
// of 128 threads (n <= 128).
extern "C" __global__ void __launch_bounds__(128)
    halo_moe_bucket_b(const std::uint32_t* ids, std::uint32_t n, std::uint32_t* ucount, std::uint32_t* uexp,
                      std::uint32_t* unum, std::uint32_t* upair) {
  __shared__ std::uint32_t lid[128], wfirst[2];
  const std::uint32_t p = threadIdx.x, lane = p % kWave, wave = p / kWave;
  const std::uint32_t e = p < n ? ids[p] : 0xFFFFFFFFu;
  lid[p] = e;
  __syncthreads();
  bool first = p < n;
  for (std::uint32_t q = 0; q < p && first; ++q) first = lid[q] != e;
  const std::uint64_t m = __ballot(first);
  if (lane == 0) wfirst[wave] = static_cast<std::uint32_t>(__builtin_popcountll(m));
  __syncthreads();
  // u = first appearances before p: the earlier wave's count plus this wave's lanes below
  const std::uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<std::uint32_t>(m >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(static_cast<std::uint32_t>(m), 0u));
  if (first) {
    const std::uint32_t u = (wave ? wfirst[0] : 0u) + below;
    uexp[u] = e;
    std::uint32_t cnt = 0;
    for (std::uint32_t q = p; q < n; ++q)
      if (lid[q] == e) upair[u * 8 + cnt++] = q;
    unum[u] = cnt;
  }
  if (p == 0) *ucount = wfirst[0] + wfirst[1];
}

// The down projection of every pair of distinct expert u = blockIdx.y (blocks past ucount exit), 32 rows per block:
// part[pair][r] = down_e[r] . h[pair] (h [pairs][cols], part [pairs][rows]). NB bounds the pairs of one expert.
template <int NB>
__device__ __forceinline__ void MoeDownBucket(const std::int8_t* qs, const std::uint16_t* d, const std::uint32_t* ucount,
                                              const std::uint32_t* uexp, const std::uint32_t* unum,
                                              const std::uint32_t* upair, const float* h, float* part,
                                              std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride) {
  const std::uint32_t u = blockIdx.y;
  if (u >= *ucount) return;
  const std::uint32_t m = min(unum[u], static_cast<std::uint32_t>(NB));
  std::uint32_t pair[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) pair[j] = upair[u * 8 + min(static_cast<std::uint32_t>(j), m - 1)];
  const std::size_t e = uexp[u];
  const std::int8_t* q8 = qs + e * rows * qstride;
  const std::uint16_t* dd = d + e * rows * (cols / 32);
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, nblk = cols / 32;
  const std::uint32_t per_wave = 32 / (blockDim.x / kWave);
  for (std::uint32_t k = 0; k < per_wave; ++k) {
    const std::uint32_t r = blockIdx.x * 32 + wave * per_wave + k;
    if (r >= rows) break;
    float acc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = 0.0f;
    for (std::uint32_t c = lane * 16; c < cols; c += kWave * 16) {
      const int4 qv = *reinterpret_cast<const int4*>(q8 + static_cast<std::size_t>(r) * qstride + c);
      const std::int8_t* v = reinterpret_cast<const std::int8_t*>(&qv);
      const float s = halo::F16(dd[static_cast<std::size_t>(r) * nblk + c / 32]);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const float4* xp = reinterpret_cast<const float4*>(h + static_cast<std::size_t>(pair[j]) * cols + c);
        float pp = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 xv = xp[i];
          pp += static_cast<float>(v[4 * i]) * xv.x + static_cast<float>(v[4 * i + 1]) * xv.y +
                static_cast<float>(v[4 * i + 2]) * xv.z + static_cast<float>(v[4 * i + 3]) * xv.w;
        }
        acc[j] += s * pp;
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const float a = halo::GroupSum(acc[j]);
      if (lane == 0 && static_cast<std::uint32_t>(j) < m) part[static_cast<std::size_t>(pair[j]) * rows + r] = a;
    }
  }
}
#define HALO_MOE_DOWN_BUCKET(NB)                                                                                 \
  extern "C" __global__ void __launch_bounds__(256) halo_moe_down_q8r_r4_b##NB(                                 \
      const std::int8_t* qs, const std::uint16_t* d, const std::uint32_t* ucount, const std::uint32_t* uexp,     \
      const std::uint32_t* unum, const std::uint32_t* upair, const float* h, float* part, std::uint32_t rows,     \
      std::uint32_t cols, std::uint32_t qstride) {                                                               \
    MoeDownBucket<NB>(qs, d, ucount, uexp, unum, upair, h, part, rows, cols, qstride);                           \
  }
HALO_MOE_DOWN_BUCKET(1)
HALO_MOE_DOWN_BUCKET(2)
HALO_MOE_DOWN_BUCKET(3)
HALO_MOE_DOWN_BUCKET(4)
HALO_MOE_DOWN_BUCKET(5)
HALO_MOE_DOWN_BUCKET(6)
HALO_MOE_DOWN_BUCKET(7)
HALO_MOE_DOWN_BUCKET(8)
#undef HALO_MOE_DOWN_BUCKET

// ---- prefill pair grouping by expert (reference names) ------------------------------------------------------------
// core.hip:4725-4864. (token, slot) pairs p with expert ids[p] -> sorted (pairs grouped by expert, pair order within
// an expert), pos[p] (p's sorted position), work tiles of up to 64 pairs of one expert, tiles[3 i .. 3 i + 2] =
// (expert, first, count), in expert order, and ntiles. experts <= 1024.
namespace halo::refk {
constexpr std::uint32_t kPairTile = 64, kPairChunk = 1024, kNoKey = 0xFFFFFFFFu;
// Expert offsets (exclusive scan of totals in expert order), tiles and ntiles, from total[e] in LDS; block 1024.
__device__ __forceinline__ void BucketTiles(const std::uint32_t* total, std::uint32_t experts, std::uint32_t* poff,
                                            std::uint32_t* tiles, std::uint32_t* ntiles, std::uint32_t* wave_tot) {
  const std::uint32_t e = threadIdx.x;
  const std::uint32_t n = e < experts ? total[e] : 0u, nt = (n + kPairTile - 1) / kPairTile;
  std::uint32_t ptot, ttot;
  const std::uint32_t p0 = halo::sample::BlockExclScan<std::uint32_t>(n, wave_tot, &ptot);
  const std::uint32_t t0 = halo::sample::BlockExclScan<std::uint32_t>(nt, wave_tot, &ttot);
  if (e < experts) poff[e] = p0;
  for (std::uint32_t i = 0; i < nt; ++i) {
    tiles[3 * (t0 + i)] = e;
    tiles[3 * (t0 + i) + 1] = p0 + i * kPairTile;
    tiles[3 * (t0 + i) + 2] = min(kPairTile, n - i * kPairTile);
  }
  if (e == 0) *ntiles = ttot;
}

// Stable rank of this thread's key among the block's lower-numbered threads holding the same key (keys < nkeys;
// kNoKey takes no part and gets 0). Inside a wave the lanes of one key are found together by a ballot against the
// lowest pending lane's key, one key per round; wave w's count of each key goes to tab[w * nkeys + key], so the rank
// adds the counts of the earlier waves. tab holds (blockDim / 64) * nkeys words; it stays valid until the caller's
// next barrier-separated reuse (callers read per-key block totals from it).
__device__ __forceinline__ std::uint32_t BlockKeyRank(std::uint32_t key, std::uint32_t nkeys, std::uint32_t* tab) {
  const std::uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
  for (std::uint32_t i = threadIdx.x; i < waves * nkeys; i += blockDim.x) tab[i] = 0;
  __syncthreads();
  const std::uint64_t below = (std::uint64_t{1} << lane) - 1;
  std::uint64_t todo = __ballot(key != kNoKey);
  std::uint32_t rank = 0;
  while (todo) {
    const std::uint32_t leader = static_cast<std::uint32_t>(__builtin_ctzll(todo));
    const std::uint32_t lk = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), leader));
    const std::uint64_t same = __ballot(key == lk);
    if (key == lk) rank = static_cast<std::uint32_t>(__builtin_popcountll(same & below));
    if (lane == leader) tab[wave * nkeys + lk] = static_cast<std::uint32_t>(__builtin_popcountll(same));
    todo &= ~same;
  }
  __syncthreads();
  if (key != kNoKey)
    for (std::uint32_t w = 0; w < wave; ++w) rank += tab[w * nkeys + key];
  return rank;
}
}  // namespace halo::refk

// One block of 1024 threads does all of it (small chunks): counts, offsets and tiles, then chunk by chunk each pair's
// position = its expert's running offset + its rank in the chunk; the running offsets then add the chunk's counts.
extern "C" __global__ void __launch_bounds__(1024)
    halo_moe_bucket(const std::uint32_t* ids, std::uint32_t pairs, std::uint32_t experts, std::uint32_t* sorted,
                    std::uint32_t* pos, std::uint32_t* tiles, std::uint32_t* ntiles) {
  __shared__ std::uint32_t cnt[1024], run[1024], wave_tot[16], tab[16 * 1024];
  const std::uint32_t tid = threadIdx.x;
  cnt[tid] = 0;
  __syncthreads();
  for (std::uint32_t p = tid; p < pairs; p += blockDim.x) atomicAdd(&cnt[ids[p]], 1u);
  __syncthreads();
  BucketTiles(cnt, experts, run, tiles, ntiles, wave_tot);
  const std::uint32_t waves = blockDim.x / kWave;
  for (std::uint32_t base = 0; base < pairs; base += blockDim.x) {
    const std::uint32_t p = base + tid;
    const std::uint32_t e = p < pairs ? ids[p] : kNoKey;
    const std::uint32_t rank = BlockKeyRank(e, experts, tab);  // its first barrier also publishes run[]
    if (e != kNoKey) {
      const std::uint32_t at = run[e] + rank;
      sorted[at] = p;
      pos[p] = at;
    }
    __syncthreads();  // every read of run[] for this chunk is done
    for (std::uint32_t x = tid; x < experts; x += blockDim.x) {
      std::uint32_t add = 0;
      for (std::uint32_t w = 0; w < waves; ++w) add += tab[w * experts + x];
      run[x] += add;
    }
    __syncthreads();  // run[] updated and tab[] free before the next chunk
  }
}
// 1. per chunk of 1024 pairs, per-expert counts [chunks][experts]. grid (chunks), block 1024.
extern "C" __global__ void __launch_bounds__(1024)
    halo_moe_bucket_count(const std::uint32_t* ids, std::uint32_t pairs, std::uint32_t experts,
                          std::uint32_t* counts) {
  __shared__ std::uint32_t c[1024];
  const std::uint32_t tid = threadIdx.x, p = blockIdx.x * kPairChunk + tid;
  c[tid] = 0;
  __syncthreads();
  if (p < pairs) atomicAdd(&c[ids[p]], 1u);
  __syncthreads();
  if (tid < experts) counts[static_cast<std::size_t>(blockIdx.x) * experts + tid] = c[tid];
}
// 2. counts become exclusive chunk offsets per expert; expert offsets base[e], tiles, ntiles. grid (1), block 1024.
extern "C" __global__ void __launch_bounds__(1024)
    halo_moe_bucket_scan(std::uint32_t* counts, std::uint32_t chunks, std::uint32_t experts, std::uint32_t* tiles,
                         std::uint32_t* ntiles, std::uint32_t* base) {
  __shared__ std::uint32_t total[1024], wave_tot[16];
  const std::uint32_t e = threadIdx.x;
  if (e < experts) {
    std::uint32_t acc = 0;
    for (std::uint32_t ch = 0; ch < chunks; ++ch) {
      std::uint32_t* c = counts + static_cast<std::size_t>(ch) * experts + e;
      const std::uint32_t v = *c;
      *c = acc;
      acc += v;
    }
    total[e] = acc;
  }
  __syncthreads();
  BucketTiles(total, experts, base, tiles, ntiles, wave_tot);
}
// 3. sorted position = expert base + the chunk's offset for the expert + the pair's rank inside the chunk
// (BlockKeyRank). grid (chunks), block 1024.
extern "C" __global__ void __launch_bounds__(1024)
    halo_moe_bucket_scatter(const std::uint32_t* ids, std::uint32_t pairs, std::uint32_t experts,
                            const std::uint32_t* chunk_off, const std::uint32_t* base, std::uint32_t* sorted,
                            std::uint32_t* pos) {
  __shared__ std::uint32_t tab[16 * 1024];
  const std::uint32_t p = blockIdx.x * kPairChunk + threadIdx.x;
  const std::uint32_t e = p < pairs ? ids[p] : kNoKey;
  const std::uint32_t rank = BlockKeyRank(e, experts, tab);
  if (e == kNoKey) return;
  const std::uint32_t at = base[e] + chunk_off[static_cast<std::size_t>(blockIdx.x) * experts + e] + rank;
  sorted[at] = p;
  pos[p] = at;
}

// ---- decode / prefill glue: fused norm + RoPE rows, batched-column variants, small elementwise (reference names)
// core.hip:308-311, 372-440, 587-590, 1123-1133, 4045-4055, 4708-4715; batch_decode.hip:1680-1705.
namespace halo::refk {
// v [d] in LDS (d <= 256, one value per thread at threadIdx.x < d) <- x * w / rms(x); then NEOX RoPE on v at pos.
__device__ __forceinline__ void NormRopeLds(float xi, const float* w, float eps, std::uint32_t d,
                                            std::uint32_t rotary_dim, std::uint32_t pos, float theta, float* v,
                                            float* red) {
  const std::uint32_t i = threadIdx.x;
  const float ss = BlockSumAny(i < d ? xi * xi : 0.0f, red);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
  if (i < d) v[i] = xi * inv * w[i];
  __syncthreads();
  RotateHead(v, rotary_dim, pos, theta);
  __syncthreads();
}
}  // namespace halo::refk

// Pooled blocks b0, b0 + 1, ... at positions (b0 + b) * ratio. grid (nblocks).
extern "C" __global__ void halo_rope_neox_blocks(float* x, std::uint32_t head_dim, std::uint32_t rotary_dim,
                                                 std::uint32_t b0, std::uint32_t ratio, float theta) {
  RotateHead(x + static_cast<std::size_t>(blockIdx.x) * head_dim, rotary_dim, (b0 + blockIdx.x) * ratio, theta);
}
// halo_split_qgate, the q rows' RMSNorm (shared w) and RoPE in one pass: token t = blockIdx.x / heads at pos0 + t.
// gate may be null. grid (T * heads), block hd (<= 256).
extern "C" __global__ void __launch_bounds__(256)
    halo_split_qgate_norm_rope(const float* qg, float* q, float* gate, const float* w, float eps,
                               std::uint32_t rotary_dim, std::uint32_t pos0, std::uint32_t heads, float theta) {
  __shared__ float red[16], v[256];
  const std::uint32_t hd = blockDim.x, i = threadIdx.x;
  const float* src = qg + static_cast<std::size_t>(blockIdx.x) * 2 * hd;
  if (gate) gate[static_cast<std::size_t>(blockIdx.x) * hd + i] = src[hd + i];
  NormRopeLds(src[i], w, eps, hd, rotary_dim, pos0 + blockIdx.x / heads, theta, v, red);
  q[static_cast<std::size_t>(blockIdx.x) * hd + i] = v[i];
}
// RMSNorm (shared w, d <= 256) then RoPE on rows of `heads` heads per token at pos0 + blockIdx.x / heads, in place;
// with cache non-null the rotated row is also written there (cache row blockIdx.x). grid (T * heads), block 256.
extern "C" __global__ void __launch_bounds__(256)
    halo_norm_rope_rows(float* x, const float* w, float eps, std::uint32_t d, std::uint32_t rotary_dim,
                        std::uint32_t pos0, std::uint32_t heads, float theta, float* cache) {
  __shared__ float red[16], v[256];
  const std::uint32_t i = threadIdx.x;
  float* row = x + static_cast<std::size_t>(blockIdx.x) * d;
  NormRopeLds(i < d ? row[i] : 0.0f, w, eps, d, rotary_dim, pos0 + blockIdx.x / heads, theta, v, red);
  if (i < d) {
    row[i] = v[i];
    if (cache) cache[static_cast<std::size_t>(blockIdx.x) * d + i] = v[i];
  }
}
// RMSNorm of T * hc vectors whose gammas repeat every w_period vectors (vector b uses w_all + (b % w_period) *
// w_stride). grid (vectors).
extern "C" __global__ void halo_rmsnorm_rows(const float* x, const float* w_all, float* y, std::uint32_t d, float eps,
                                             std::uint32_t w_stride, std::uint32_t w_period) {
  __shared__ float red[16];
  const std::size_t b = blockIdx.x;
  const float* w = w_all + (b % w_period) * w_stride;
  const float inv = RmsScale(x + b * d, d, eps, red);
  RowApply(x + b * d, y + b * d, d, [&](std::uint32_t i, float v) { return v * inv * w[i]; });
}

// Batched-column variants: column (session entry) e = blockIdx.y, its data `stride` floats apart.
// grid (heads, B)
extern "C" __global__ void halo_split_qgate_y(const float* qg, float* q, float* gate, std::uint32_t hd,
                                              std::uint32_t qg_stride, std::uint32_t q_stride) {
  const std::size_t h = blockIdx.x, e = blockIdx.y;
  const float* src = qg + e * qg_stride + h * 2 * hd;
  for (std::uint32_t i = threadIdx.x; i < hd; i += blockDim.x) {
    q[e * q_stride + h * hd + i] = src[i];
    gate[e * q_stride + h * hd + i] = src[hd + i];
  }
}
// In place; grid (vectors, B)
extern "C" __global__ void halo_rmsnorm_y(float* x, const float* w_all, std::uint32_t d, float eps,
                                          std::uint32_t w_stride, std::uint32_t stride) {
  __shared__ float red[16];
  float* xv = x + static_cast<std::size_t>(blockIdx.y) * stride + static_cast<std::size_t>(blockIdx.x) * d;
  const float* w = w_all + static_cast<std::size_t>(blockIdx.x) * w_stride;
  const float inv = RmsScale(xv, d, eps, red);
  RowApply(xv, xv, d, [&](std::uint32_t i, float v) { return v * inv * w[i]; });
}
// grid (heads, B): column e's position params[e * pstride + slot] * scale.
extern "C" __global__ void halo_rope_neox_p_y(float* x, const std::uint32_t* params, std::uint32_t head_dim,
                                              std::uint32_t rotary_dim, std::uint32_t slot, std::uint32_t scale,
                                              float theta, std::uint32_t stride, std::uint32_t pstride) {
  const std::size_t e = blockIdx.y;
  RotateHead(x + e * stride + static_cast<std::size_t>(blockIdx.x) * head_dim, rotary_dim,
             params[e * pstride + slot] * scale, theta);
}
// Column e's destination is the pointer tab[e * tstride + tslot]. grid (ceil(n / 256), B)
extern "C" __global__ void halo_copy_at_y(const std::uint64_t* tab, std::uint32_t tstride, std::uint32_t tslot,
                                          const float* src, const std::uint32_t* params, std::uint32_t slot,
                                          std::uint32_t stride, std::uint32_t n, std::uint32_t src_stride,
                                          std::uint32_t pstride) {
  const std::size_t e = blockIdx.y;
  float* dst = reinterpret_cast<float*>(tab[e * tstride + tslot]);
  float* row = dst + static_cast<std::size_t>(params[e * pstride + slot]) * stride;
  const float* s = src + e * src_stride;
  for (std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) row[i] = s[i];
}

// y += weights[slot] x; y += sigmoid(g[0]) x; for T rows y [T][n] += sigmoid(g[t]) x [T][n]; x = silu(x scale).
extern "C" __global__ void halo_axpy_slot(float* y, const float* x, const float* weights, std::uint32_t slot,
                                          std::uint32_t n) {
  const float a = weights[slot];
  for (std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) y[i] += a * x[i];
}
extern "C" __global__ void halo_axpy_sigmoid(float* y, const float* x, const float* g, std::uint32_t n) {
  const float a = halo::Sigmoid(g[0]);
  for (std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) y[i] += a * x[i];
}
extern "C" __global__ void halo_axpy_sigmoid_rows(float* y, const float* x, const float* g, std::uint32_t n,
                                                  std::uint32_t tokens) {
  const std::size_t total = static_cast<std::size_t>(tokens) * n;
  for (std::size_t i = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
    y[i] += halo::Sigmoid(g[i / n]) * x[i];
}
extern "C" __global__ void halo_scale_silu(float* x, float scale, std::uint32_t n) {
  for (std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    x[i] = halo::Silu(x[i] * scale);
}

// ---- fp32 GEMMs for prefill routers and small projections, shared-expert add, batched top-k (reference names) --
// core.hip:2938-2956, 3767-3800, 5605-5680, 8975-9000; batch_decode.hip:1157-1165. y [T][rows] = x [T][cols] W^T.

// 64 rows x 64 tokens per block on fp32 MFMA: the tile body of halo_gemm_f32_nt (v_mfma_f32_32x32x2f32, K staged
// 32 at a time through LDS, the next stage prefetched into registers), with the reference's grid. cols % 16 == 0
// (a trailing half stage is zero-filled). grid (ceil(T / 64), ceil(rows / 64)), block 256.
extern "C" __global__ void __launch_bounds__(256)
    halo_gemm_f32_tiled(const float* w, const float* x, float* y, std::uint32_t rows, std::uint32_t cols,
                        std::uint32_t tokens) {
  halo::GemmF32NtTile(x, w, nullptr, y, nullptr, tokens, rows, cols, rows, blockIdx.y * 64, blockIdx.x * 64);
}
// One wave per output row (2 rows per wave of the block's 8), lanes across columns. grid (ceil(rows / 8), T).
extern "C" __global__ void __launch_bounds__(256)
    halo_gemm_f32_rows(const float* w, const float* x, float* y, std::uint32_t rows, std::uint32_t cols) {
  const std::uint32_t t = blockIdx.y, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const float* xr = x + static_cast<std::size_t>(t) * cols;
  for (std::uint32_t k = 0; k < 2; ++k) {
    const std::uint32_t r = blockIdx.x * 8 + wave * 2 + k;
    if (r >= rows) break;
    const float* wr = w + static_cast<std::size_t>(r) * cols;
    float acc = 0.0f;
    for (std::uint32_t c = lane; c < cols; c += kWave) acc = __builtin_fmaf(wr[c], xr[c], acc);
    acc = halo::GroupSum(acc);
    if (lane == 0) y[static_cast<std::size_t>(t) * rows + r] = acc;
  }
}
// Few columns (core.hip:3771-3782): one output row per thread, the token's x row in LDS. W is staged through LDS in
// 256-row x 32-column tiles read along the rows (32 consecutive floats per row, coalesced), so no thread walks its
// own row in HBM; each thread then sums its tile row in ascending k (one fused chain).
// grid (ceil(rows / 256), T), block 256; cols <= 8192.
extern "C" __global__ void __launch_bounds__(256)
    halo_gemm_f32_narrow(const float* w, const float* x, float* y, std::uint32_t rows, std::uint32_t cols) {
  constexpr std::uint32_t BK = 32;
  __shared__ float xs[8192];
  __shared__ float tile[256][BK + 1];
  const std::uint32_t tid = threadIdx.x, r0 = blockIdx.x * 256;
  const std::size_t t = blockIdx.y;
  for (std::uint32_t i = tid; i < cols; i += 256) xs[i] = x[t * cols + i];
  float acc = 0.0f;
  for (std::uint32_t k0 = 0; k0 < cols; k0 += BK) {
    __syncthreads();  // the previous tile is consumed (and, the first time, xs is written)
    for (std::uint32_t e = tid; e < 256 * BK; e += 256) {
      const std::uint32_t rr = e / BK, kk = e % BK, r = r0 + rr, k = k0 + kk;
      tile[rr][kk] = r < rows && k < cols ? w[static_cast<std::size_t>(r) * cols + k] : 0.0f;
    }
    __syncthreads();
    const std::uint32_t kn = min(BK, cols - k0);
    for (std::uint32_t kk = 0; kk < kn; ++kk) acc = __builtin_fmaf(tile[tid][kk], xs[k0 + kk], acc);
  }
  if (r0 + tid < rows) y[t * rows + r0 + tid] = acc;
}
// Few rows (<= 16; core.hip:8975-9000): each wave takes two of the block's 8 tokens in turn, all 64 lanes across the
// token's row (16-byte loads when the row allows), every weight row against it (the few weight rows stay in cache),
// then one wave reduction per row. grid (ceil(T / 8)), block 256.
extern "C" __global__ void __launch_bounds__(256)
    halo_gemm_f32_skinny(const float* w, const float* x, float* y, std::uint32_t rows, std::uint32_t cols,
                         std::uint32_t tokens) {
  const std::uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  for (std::uint32_t tt = 0; tt < 2; ++tt) {
    const std::uint32_t t = blockIdx.x * 8 + wave * 2 + tt;
    if (t >= tokens) break;  // wave-uniform
    const float* xr = x + static_cast<std::size_t>(t) * cols;
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    const bool vec = Vec4Ok(xr, cols) && Vec4Ok(w, cols);
    const std::uint32_t nv = vec ? cols / 4 : 0;
    for (std::uint32_t c4 = lane; c4 < nv; c4 += kWave) {
      const float4 xv = reinterpret_cast<const float4*>(xr)[c4];
#pragma unroll
      for (std::uint32_t r = 0; r < 16; ++r)
        if (r < rows) {
          const float4 wv = reinterpret_cast<const float4*>(w + static_cast<std::size_t>(r) * cols)[c4];
          acc[r] = __builtin_fmaf(wv.w, xv.w,
                                  __builtin_fmaf(wv.z, xv.z, __builtin_fmaf(wv.y, xv.y, __builtin_fmaf(wv.x, xv.x, acc[r]))));
        }
    }
    for (std::uint32_t c = 4 * nv + lane; c < cols; c += kWave) {  // scalar path (unaligned rows)
      const float xv = xr[c];
#pragma unroll
      for (std::uint32_t r = 0; r < 16; ++r)
        if (r < rows) acc[r] = __builtin_fmaf(w[static_cast<std::size_t>(r) * cols + c], xv, acc[r]);
    }
#pragma unroll
    for (std::uint32_t r = 0; r < 16; ++r) {
      const float sum = halo::GroupSum(acc[r]);
      if (lane == 0 && r < rows) y[static_cast<std::size_t>(t) * rows + r] = sum;
    }
  }
}

// out[r] += sigmoid(sgate[0]) * (down_r . hin); 32 rows per block. grid (ceil(rows / 32)), block 256.
extern "C" __global__ void __launch_bounds__(256)
    halo_shexp_down_add(const std::int8_t* dq, const std::uint16_t* dd, const float* hin, const float* sgate,
                        float* out, std::uint32_t rows, std::uint32_t cols, std::uint32_t qstride) {
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const std::uint32_t per_wave = 32 / (blockDim.x / kWave);
  const float s = halo::Sigmoid(sgate[0]);
  for (std::uint32_t k = 0; k < per_wave; ++k) {
    const std::uint32_t r = blockIdx.x * 32 + wave * per_wave + k;
    if (r >= rows) break;
    const float yv = Q8RowDot(dq, dd, hin, r, cols, qstride);
    if (lane == 0) out[r] += s * yv;
  }
}

// halo_router_topk_w for the columns of a batch: column b = blockIdx.y reads logits + b * lstride and writes
// k ids / weights at b * k. grid (1, B), block 256.
extern "C" __global__ void __launch_bounds__(256)
    halo_router_topk_w_y(const float* logits, std::uint32_t* ids, float* weights, std::uint32_t n, std::uint32_t k,
                         std::uint32_t lstride) {
  __shared__ std::uint32_t scratch[64];
  __shared__ float wscratch[64];
  __shared__ TopKScratch sc;
  if (threadIdx.x >= kWave) return;
  const std::size_t b = blockIdx.y;
  WaveTopK<16>(logits + b * lstride, n, k, ids + b * k, weights + b * k, scratch, wscratch, sc);
}

// ---- batched columns through a pointer table (reference names; batch_decode.hip:1727-1748) ----------------------
// Column e = blockIdx.y: its KV cache (rows kslot, kslot + 1) or conv state (slot tslot) is the pointer
// tab[e * tstride + slot]; its other data sit `stride` floats apart.
// grid (num_heads, B), block 256
extern "C" __global__ void __launch_bounds__(256)
    halo_attention_select_b_y(const float* q, const std::uint64_t* tab, std::uint32_t tstride, std::uint32_t kslot,
                              const float* gate, const std::uint32_t* visible, float* out, float* scores,
                              const std::uint32_t* params, std::uint32_t num_heads, std::uint32_t num_kv_heads,
                              std::uint32_t hd, std::uint32_t max_n, std::uint32_t q_stride,
                              std::uint32_t visible_stride, std::uint32_t scores_stride, std::uint32_t pstride) {
  __shared__ float red[16];
  const std::size_t e = blockIdx.y;
  const float* kc = reinterpret_cast<const float*>(tab[e * tstride + kslot]);
  const float* vc = reinterpret_cast<const float*>(tab[e * tstride + kslot + 1]);
  const std::uint32_t h = blockIdx.x, kvh = h / (num_heads / num_kv_heads);
  const std::size_t row = e * q_stride + static_cast<std::size_t>(h) * hd;
  AttendHead(q + row, kc, vc, gate + row, out + row, scores + e * scores_stride + static_cast<std::size_t>(h) * max_n,
             kvh, num_kv_heads, hd, params[e * pstride + 5], red, visible + e * visible_stride);
}
// grid (channels / 128, B), block 128
extern "C" __global__ void halo_conv_l2norm_y(const float* in, const std::uint64_t* tab, std::uint32_t tstride,
                                              std::uint32_t tslot, const float* w, float* out, std::uint32_t channels,
                                              std::uint32_t kern, std::uint32_t l2_channels, float eps,
                                              std::uint32_t stride) {
  __shared__ float sh[256];
  const std::size_t e = blockIdx.y;
  ConvL2norm(in + e * stride, reinterpret_cast<float*>(tab[e * tstride + tslot]), w, out + e * stride, channels, kern,
             l2_channels, eps, sh);
}

// halo_conv_l2norm_prefill for kern = 4 over tiles of 128 channels x 8 tokens (the reference's grid, core.hip:
// 3512-3570), mapped wave64-first: wave w takes tokens t0 + 4 w .. t0 + 4 w + 3 of the whole head, lane l its channels
// l and l + 64, so a token's L2 sum is one wave's reduction (no LDS, no barrier). Each channel's 7-input window is
// loaded once for its four tokens. Arithmetic as stepping: the same bits as halo_conv_l2norm_prefill.
//   grid (ceil(channels / 128), ceil(T / 8)), block 128.
extern "C" __global__ void __launch_bounds__(128)
    halo_conv_l2norm_prefill8(const float* in, const float* state, const float* w, float* out, std::uint32_t channels,
                              std::uint32_t tokens, std::uint32_t l2_channels, float eps) {
  constexpr std::uint32_t K = 4, TW = 4;
  const std::uint32_t lane = threadIdx.x % kWave, c0 = blockIdx.x * 128;
  const std::int64_t tb = static_cast<std::int64_t>(blockIdx.y) * 8 + (threadIdx.x / kWave) * TW;
  float v[2][TW];
#pragma unroll
  for (std::uint32_t half = 0; half < 2; ++half) {
    const std::uint32_t ch = c0 + half * kWave + lane;
    const bool live = ch < channels;
    const std::uint32_t c = live ? ch : 0;
    float x[TW + K - 1];  // inputs tb - 3 .. tb + 3
#pragma unroll
    for (std::uint32_t j = 0; j < TW + K - 1; ++j) {
      const std::int64_t i = tb - static_cast<std::int64_t>(K - 1) + j;
      x[j] = i < static_cast<std::int64_t>(tokens) ? ConvInput(in, state, i, c, channels, K) : 0.0f;
    }
    const float* wc = w + static_cast<std::size_t>(c) * K;
#pragma unroll
    for (std::uint32_t t = 0; t < TW; ++t) {
      float win[kMaxTaps] = {x[t], x[t + 1], x[t + 2], x[t + 3]};
      v[half][t] = live ? ConvSilu(wc, win, K) : 0.0f;
    }
  }
  if (c0 < l2_channels) {  // block-uniform
#pragma unroll
    for (std::uint32_t t = 0; t < TW; ++t) {
      const float ss = halo::GroupSum(__builtin_fmaf(v[1][t], v[1][t], __builtin_fmaf(v[0][t], v[0][t], 0.0f)));
      const float inv = 1.0f / sqrtf(ss + eps);
      v[0][t] *= inv;
      v[1][t] *= inv;
    }
  }
#pragma unroll
  for (std::uint32_t half = 0; half < 2; ++half) {
    const std::uint32_t ch = c0 + half * kWave + lane;
#pragma unroll
    for (std::uint32_t t = 0; t < TW; ++t)
      if (ch < channels && tb + t < tokens) out[static_cast<std::size_t>(tb + t) * channels + ch] = v[half][t];
  }
}
