// MoE decode layer for T <= 16 tokens (gfx950, wave64): router, softmax/top-k with the session union of experts,
// grouped gate/up + SwiGLU over the active experts, and the down projection with the routed combine.
//
// Reference semantics: ReferenceModel::Moe (src/model/reference.cpp:530-578), cpu::RouteTopK
// (src/model/cpu_ops.cpp:187-207), GPU RouterTopk (src/kernels/core.hip:1053-1108), session-union bucketing
// halo_moe_bucket_b (src/kernels/batch_decode.hip:417-446).
//
// Launches (all take device buffers only, so one captured graph replays for any routing):
//   1. halo_moe_router     logits[t][e] = W_r[e] . x[t] (fp32), shared-gate logit, x quantized per 32 (int8);
//      or halo_moe_router_n_* (T <= 4), which also forms x = RMSNorm(res + delta) * w itself (the FFN norm).
//   2. halo_moe_topk_w*    one wave per token: softmax, top-k (ties -> lower id), renormalized weights (the block
//                          kernel halo_moe_topk serves prefill batches); at T = 1 folded into the gate/up launch
//                          instead (halo_moe_gate_up_topk_q8_*: 3 launches).
//   3. halo_moe_gate_up_q8 block (routed pair, 4 ff rows): the first token that selected an expert computes it for
//                          every token that selected it (the union of experts: weights streamed once), h =
//                          SiLU(g) * u in fp32. One more block column is the shared expert.
//   4. halo_moe_down_q8    block (8 output rows, token): one wave per slot quantizes its h per 32 and streams
//                          4 KB of its expert; the slots are combined in slot order in LDS, then
//                          + sigmoid(shared gate) * shared.
#include "common.h"

using halo::Dot16;
using halo::F16;
using halo::kWave;

namespace {
constexpr int kMoeMaxT = 16;
}

// grid (E + 1 + ceil(T * H / 32 / 8)), block 256. router [E][H], sgate [H] (may be null), x [T][H] fp32.
extern "C" __global__ void __launch_bounds__(256)
    halo_moe_router(const float* __restrict__ router, const float* __restrict__ sgate, const float* __restrict__ x,
                    float* __restrict__ logits, float* __restrict__ sgl, std::int8_t* __restrict__ xq,
                    float* __restrict__ xs, std::uint32_t E, std::uint32_t H, std::uint32_t T) {
  const std::uint32_t bid = blockIdx.x;
  if (bid > E) {
    // quantization blocks: one 32-value block of one token per half wave
    const std::uint32_t hw = (bid - E - 1) * (blockDim.x / 32) + threadIdx.x / 32;
    const std::uint32_t nblk = H / 32;
    if (hw >= T * nblk) return;
    const std::uint32_t t = hw / nblk, b = hw % nblk, lane = threadIdx.x % 32;
    const float v = x[static_cast<std::size_t>(t) * H + b * 32 + lane];
    const float amax = halo::GroupMax<32>(fabsf(v));
    const float scale = amax / 127.0f;
    const int q = scale > 0.0f ? static_cast<int>(rintf(v / scale)) : 0;
    xq[static_cast<std::size_t>(t) * H + b * 32 + lane] = static_cast<std::int8_t>(q);
    if (lane == 0) xs[static_cast<std::size_t>(t) * nblk + b] = scale;
    return;
  }
  const float* row = bid < E ? router + static_cast<std::size_t>(bid) * H : sgate;
  if (row == nullptr) return;
  __shared__ float part[kMoeMaxT][4];
  float acc[kMoeMaxT];
#pragma unroll
  for (int t = 0; t < kMoeMaxT; ++t) acc[t] = 0.0f;
  for (std::uint32_t c = threadIdx.x * 4; c < H; c += blockDim.x * 4) {
    const float4 w = *reinterpret_cast<const float4*>(row + c);
#pragma unroll
    for (int t = 0; t < kMoeMaxT; ++t)
      if (t < static_cast<int>(T)) {
        const float4 xv = *reinterpret_cast<const float4*>(x + static_cast<std::size_t>(t) * H + c);
        acc[t] += w.x * xv.x + w.y * xv.y + w.z * xv.z + w.w * xv.w;
      }
  }
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
#pragma unroll
  for (int t = 0; t < kMoeMaxT; ++t)
    if (t < static_cast<int>(T)) {
      const float s = halo::GroupSum(acc[t]);
      if (lane == 0) part[t][wave] = s;
    }
  __syncthreads();
  if (threadIdx.x < T) {
    const float s = part[threadIdx.x][0] + part[threadIdx.x][1] + part[threadIdx.x][2] + part[threadIdx.x][3];
    if (bid < E)
      logits[static_cast<std::size_t>(threadIdx.x) * E + bid] = s;
    else
      sgl[threadIdx.x] = s;
  }
}

// The router with the FFN input norm in its prologue, for T <= 4 tokens (T * H <= 8192, H a multiple of 2048):
// x_t = RMSNorm(res[t] + delta[t]) * norm_w in the canonical row layout of halo_add_rmsnorm_q8 (same bits), so the
// norm launch before the MoE disappears. Every block normalizes the T rows itself (L2 reads); block 0 also writes
// res_out[t] = res[t] + delta[t] (a different buffer from res: the other blocks still read res) and the Q8
// quantization xq / xs of x_t for the experts. Wave w of block b dots router row r = 4 b + w (r = E: the shared gate
// row, skipped when null) with x_t from LDS.
//   grid (ceil((E + 1) / 4)), block 256. router [E][H] fp32, logits [T][E], sgl [T].
template <int KC, int kMaxT>
__device__ __forceinline__ void MoeRouterN(const float* __restrict__ router, const float* __restrict__ sgate,
                                           const float* __restrict__ res, const float* __restrict__ delta,
                                           const float* __restrict__ norm_w, float* __restrict__ res_out,
                                           float* __restrict__ logits, float* __restrict__ sgl,
                                           std::int8_t* __restrict__ xq, float* __restrict__ xs, std::uint32_t E,
                                           std::uint32_t T, float eps) {
  constexpr std::uint32_t H = KC * 2048, kF4 = H / 256;  // float4 chunks of a row per lane
  __shared__ __attribute__((aligned(16))) float xl[kMaxT * H < 8192 ? kMaxT * H : 8192];  // T * H <= 8192
  __shared__ float red[kMaxT][4];
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const std::uint32_t r = blockIdx.x * 4 + wave;
  const float* row = r < E ? router + static_cast<std::size_t>(r) * H : sgate;
  const bool live = r < E || (r == E && sgate != nullptr);
  const float* rowc = live ? row : router;  // a valid address either way; the result is dropped
  HALO_PHASE(4, 0);
  float4 w[kF4];
#pragma unroll
  for (int i = 0; i < static_cast<int>(kF4); ++i) w[i] = reinterpret_cast<const float4*>(rowc)[lane + kWave * i];
  halo::Row8<KC> x[kMaxT], nw;
#pragma unroll
  for (int t = 0; t < static_cast<int>(kMaxT); ++t) {
    const std::uint32_t tt = min(static_cast<std::uint32_t>(t), T - 1);
    halo::LoadRow8(res + static_cast<std::size_t>(tt) * H, delta + static_cast<std::size_t>(tt) * H, H, x[t]);
  }
  halo::LoadRow8(norm_w, nullptr, H, nw);
  if (blockIdx.x == 0)
#pragma unroll
    for (int t = 0; t < static_cast<int>(kMaxT); ++t)
      if (t < static_cast<int>(T)) halo::StoreRow8(res_out + static_cast<std::size_t>(t) * H, H, x[t]);
  // the sums of squares of every token, one barrier (the arithmetic of halo::RmsNormRow8W)
#pragma unroll
  for (int t = 0; t < static_cast<int>(kMaxT); ++t) {
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < KC; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(x[t].v[k][e], x[t].v[k][e], ss);
    ss = halo::GroupSum(ss);
    if (lane == 0) red[t][wave] = ss;
  }
  __syncthreads();
  HALO_PHASE(4, 1);
#pragma unroll
  for (int t = 0; t < static_cast<int>(kMaxT); ++t) {
    const float ss = ((red[t][0] + red[t][1]) + red[t][2]) + red[t][3];
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
#pragma unroll
    for (int k = 0; k < KC; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[t].v[k][e] = x[t].v[k][e] * scale * nw.v[k][e];
  }
  if (blockIdx.x == 0)
#pragma unroll
    for (int t = 0; t < static_cast<int>(kMaxT); ++t)
      if (t < static_cast<int>(T))
        halo::QuantRow8(x[t], H, xq + static_cast<std::size_t>(t) * H, xs + static_cast<std::size_t>(t) * (H / 32));
  // x_t to LDS: chunk c = thread + 256 k holds elements 8 c .. 8 c + 7
#pragma unroll
  for (int t = 0; t < static_cast<int>(kMaxT); ++t)
    if (t < static_cast<int>(T))
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const std::uint32_t c = threadIdx.x + 256u * k;
      float4* dst = reinterpret_cast<float4*>(xl + t * H + 8 * c);
      dst[0] = make_float4(x[t].v[k][0], x[t].v[k][1], x[t].v[k][2], x[t].v[k][3]);
      dst[1] = make_float4(x[t].v[k][4], x[t].v[k][5], x[t].v[k][6], x[t].v[k][7]);
    }
  __syncthreads();
  HALO_PHASE(4, 2);
  if (!live) return;
  for (std::uint32_t t = 0; t < T; ++t) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < static_cast<int>(kF4); ++i) {
      const float4 xv = reinterpret_cast<const float4*>(xl + t * H)[lane + kWave * i];
      acc += w[i].x * xv.x + w[i].y * xv.y + w[i].z * xv.z + w[i].w * xv.w;
    }
    acc = halo::GroupSum(acc);
    if (lane == 0) {
      if (r < E)
        logits[static_cast<std::size_t>(t) * E + r] = acc;
      else
        sgl[t] = acc;
    }
  }
  HALO_PHASE(4, 3);
}

// _n: T <= 4; _n1: T = 1 (one residual row loaded, not four).
#define HALO_MOE_ROUTER_N(NAME, KC, NT)                                                                            \
  extern "C" __global__ void __launch_bounds__(256)                                                               \
      NAME(const float* router, const float* sgate, const float* res, const float* delta, const float* norm_w,     \
           float* res_out, float* logits, float* sgl, std::int8_t* xq, float* xs, std::uint32_t E, std::uint32_t T, \
           float eps) {                                                                                            \
    MoeRouterN<KC, NT>(router, sgate, res, delta, norm_w, res_out, logits, sgl, xq, xs, E, T, eps);               \
  }
HALO_MOE_ROUTER_N(halo_moe_router_n_h2048, 1, 4)
HALO_MOE_ROUTER_N(halo_moe_router_n_h4096, 2, 4)
HALO_MOE_ROUTER_N(halo_moe_router_n1_h2048, 1, 1)
HALO_MOE_ROUTER_N(halo_moe_router_n1_h4096, 2, 1)
#undef HALO_MOE_ROUTER_N

namespace {
// Softmax over E logits and top-k of the probabilities for one token, one wave (src/model/cpu_ops.cpp:187-207):
// the k ids in descending probability (ties to the lower id) and the weights renormalized by max(sum, 2^-14),
// the sum accumulated in slot order. Selection: a threshold tau at or below the k-th largest of the 64 lane maxima
// bounds the k-th largest probability from below, so the top k are among the candidates p >= tau (a few per
// selected lane); each candidate's rank among the candidates, by (probability desc, id asc), is its slot. Results go
// to lds_ids (k entries) and, when lds_w is non-null, the weights to lds_w and, when non-null, ids / weights to
// global memory (a caller that needs only the ids passes lds_w = ids = weights = null and skips the renormalization).
constexpr int kCandMax = 256;

struct TopKScratch {
  // candidate keys (probability bits << 32 | ~id), 8 pad keys past the last, and a spare slot per lane
  std::uint64_t ck[kCandMax + 8 + 64];
  float sum;
};

// Orders this wave's LDS accesses: everything before is visible to every lane after.
__device__ __forceinline__ void WaveSync() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ std::uint32_t LanesBelow(std::uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<std::uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<std::uint32_t>(mask), 0u));
}

template <int kPer>
__device__ __forceinline__ void WaveTopK(const float* logits, std::uint32_t E, std::uint32_t k, std::uint32_t* ids, float* weights,
                         std::uint32_t* lds_ids, float* lds_w, TopKScratch& sc) {
  const std::uint32_t lane = threadIdx.x % kWave;
  float p[kPer];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const std::uint32_t e = lane + kWave * i;
    const float lv = logits[min(e, E - 1)];
    p[i] = e < E ? lv : -INFINITY;
    mx = fmaxf(mx, p[i]);
  }
  mx = halo::GroupMax(mx);
  float den = 0.0f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const std::uint32_t e = lane + kWave * i;
    p[i] = e < E ? expf(p[i] - mx) : 0.0f;
    den += p[i];
  }
  den = halo::GroupSum(den);
  float lm = -1.0f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const std::uint32_t e = lane + kWave * i;
    p[i] = e < E ? p[i] / den : -1.0f;
    lm = fmaxf(lm, p[i]);
  }
  HALO_PHASE(3, 5);
  // tau from a bitwise search over the lane keys (probability bits + 1, 0 for a lane without experts; probabilities
  // are in [0, 1], so their bit patterns order like the values and stay below 2^30). The search keeps the largest thr
  // with at least k keys >= thr, deciding bits 29 .. 18 only: thr is then the k-th largest key with its low 18 bits
  // cleared (within 2^-5 of it), still a lower bound, in 6 dependent steps instead of 31 at the cost of a few
  // more candidates. Every probability is >= 0, so tau = -1 admits all when k > 64.
  float tau = -1.0f;
  if (k <= kWave) {
    const std::uint32_t key = lm >= 0.0f ? __float_as_uint(lm) + 1u : 0u;
    std::uint32_t thr = 0;
    // two bits per step (three independent ballots; the counts fall as the digit rises, so the largest digit
    // whose count reaches k is the one two single-bit steps would pick): half the dependent ballot chain
#pragma unroll
    for (int bit = 28; bit >= 18; bit -= 2) {
      const std::uint32_t c1 = thr | (1u << bit), c2 = thr | (2u << bit), c3 = thr | (3u << bit);
      const std::uint32_t n1 = static_cast<std::uint32_t>(__builtin_popcountll(__ballot(key >= c1)));
      const std::uint32_t n2 = static_cast<std::uint32_t>(__builtin_popcountll(__ballot(key >= c2)));
      const std::uint32_t n3 = static_cast<std::uint32_t>(__builtin_popcountll(__ballot(key >= c3)));
      thr = n3 >= k ? c3 : n2 >= k ? c2 : n1 >= k ? c1 : thr;
    }
    tau = thr == 0 ? -1.0f : __uint_as_float(thr - 1u);
  }
  HALO_PHASE(3, 6);
  // candidates p >= tau as 64-bit keys, probability bits above and ~id below: a larger key is an earlier slot (ties
  // in probability to the lower id; ids are distinct, so keys are). Every lane stores, a non-candidate (or one past
  // the scratch) into its own spare slot, so no store waits on an exec mask.
  std::uint32_t n = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const std::uint32_t e = lane + kWave * i;
    const bool f = e < E && p[i] >= tau;
    const std::uint64_t m = __ballot(f);
    const std::uint32_t pos = n + LanesBelow(m);
    sc.ck[f && pos < kCandMax ? pos : kCandMax + 8 + lane] =
        (static_cast<std::uint64_t>(__float_as_uint(p[i])) << 32) | static_cast<std::uint32_t>(~e);
    n += static_cast<std::uint32_t>(__builtin_popcountll(m));
  }
  if (lane < 8 && n <= kCandMax) sc.ck[n + lane] = 0;  // pad keys below every candidate: reads past n count nothing
  WaveSync();
  HALO_PHASE(3, 7);
  if (n <= kCandMax) {
    // candidate c in lane c % 64: its rank = the number of larger keys, read 8 at a time (4 loads in flight)
    for (std::uint32_t c0 = 0; c0 < n; c0 += kWave) {
      const std::uint32_t c = c0 + lane;
      const std::uint64_t key = sc.ck[min(c, n - 1)];
      std::uint32_t rank = 0;
      for (std::uint32_t j = 0; j < n; j += 8) {
        const ulonglong2 k0 = *reinterpret_cast<const ulonglong2*>(&sc.ck[j]);
        const ulonglong2 k1 = *reinterpret_cast<const ulonglong2*>(&sc.ck[j + 2]);
        const ulonglong2 k2 = *reinterpret_cast<const ulonglong2*>(&sc.ck[j + 4]);
        const ulonglong2 k3 = *reinterpret_cast<const ulonglong2*>(&sc.ck[j + 6]);
        rank += ((k0.x > key) + (k0.y > key)) + ((k1.x > key) + (k1.y > key)) + ((k2.x > key) + (k2.y > key)) +
                ((k3.x > key) + (k3.y > key));
      }
      if (c < n && rank < k) {
        lds_ids[rank] = ~static_cast<std::uint32_t>(key);
        if (lds_w != nullptr) lds_w[rank] = __uint_as_float(static_cast<std::uint32_t>(key >> 32));
      }
    }
  } else {
    // more candidates than the scratch holds (massive ties): repeated arg-max
    std::uint32_t taken = 0;
    for (std::uint32_t s = 0; s < k; ++s) {
      float v = -2.0f;
      std::uint32_t at = 0xFFFFFFFFu;
#pragma unroll
      for (int i = 0; i < kPer; ++i)
        if (!((taken >> i) & 1u) && p[i] > v) {
          v = p[i];
          at = lane + kWave * i;
        }
#pragma unroll
      for (int o = kWave / 2; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const std::uint32_t oi = __shfl_xor(at, o, kWave);
        if (ov > v || (ov == v && oi < at)) {
          v = ov;
          at = oi;
        }
      }
      if (at % kWave == lane) taken |= 1u << (at / kWave);
      if (lane == 0) {
        lds_ids[s] = at;
        if (lds_w != nullptr) lds_w[s] = v;
      }
    }
  }
  WaveSync();
  if (lds_w == nullptr) return;
  if (k <= static_cast<std::uint32_t>(kWave)) {
    // slot s in lane s; the sum in slot order, read across lanes
    const float ws = lds_w[min(lane, k - 1)];
    float sum = 0.0f;
    for (std::uint32_t s = 0; s < k; ++s)
      sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ws), s));
    sum = fmaxf(sum, 6.103515625e-5f);
    if (lane < k) {
      const float w = ws / sum;
      lds_w[lane] = w;
      if (ids != nullptr) {
        ids[lane] = lds_ids[lane];
        weights[lane] = w;
      }
    }
    WaveSync();
    return;
  }
  if (lane == 0) {
    float sum = 0.0f;
    for (std::uint32_t s = 0; s < k; ++s) sum += lds_w[s];
    sc.sum = fmaxf(sum, 6.103515625e-5f);
  }
  WaveSync();
  const float sum = sc.sum;
  for (std::uint32_t s = lane; s < k; s += kWave) {
    const float w = lds_w[s] / sum;
    lds_w[s] = w;
    if (ids != nullptr) {
      ids[s] = lds_ids[s];
      weights[s] = w;
    }
  }
  WaveSync();
}
}  // namespace

namespace {
// Block-wide max / sum over blockDim.x threads (a multiple of 64, <= 1024); red holds 16 floats.
__device__ __forceinline__ float BlockMax16(float v, float* red) {
  v = halo::GroupMax(v);
  const std::uint32_t wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
  if (threadIdx.x % kWave == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (std::uint32_t w = 1; w < waves; ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ float BlockSum16(float v, float* red) {
  v = halo::GroupSum(v);
  const std::uint32_t wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
  if (threadIdx.x % kWave == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (std::uint32_t w = 1; w < waves; ++w) r += red[w];
  __syncthreads();
  return r;
}
}  // namespace

// Routing of T tokens, one block per token, one thread per expert (blockDim.x = E rounded up to 64, <= 1024):
// softmax over the E logits, top-k by probability (ties to the lower id), weights renormalized by max(sum, 2^-14)
// with the sum in slot order (src/model/cpu_ops.cpp:187-207). Selection: groups of 8 consecutive experts; tau,
// the k-th largest group maximum, bounds the k-th largest probability from below, so the top k are among the
// candidates p >= tau; a candidate's rank among the candidates by (probability desc, id asc) is its slot.
//   logits [T][E] -> ids [T][k], weights [T][k]
extern "C" __global__ void __launch_bounds__(1024)
    halo_moe_topk(const float* __restrict__ logits, std::uint32_t* __restrict__ ids, float* __restrict__ weights,
                  std::uint32_t E, std::uint32_t k) {
  constexpr int kCand = 256;
  __shared__ float red[16];
  __shared__ float gmax[128];
  __shared__ float cp[kCand];
  __shared__ std::uint32_t ci[kCand];
  __shared__ float selp[32];
  __shared__ std::uint32_t seli[32];
  __shared__ float pall[1024];
  __shared__ float tau_s;
  __shared__ std::uint32_t ncand;
  const std::uint32_t t = blockIdx.x, e = threadIdx.x;
  const bool valid = e < E;
  const float lv = logits[static_cast<std::size_t>(t) * E + min(e, E - 1)];
  const float l = valid ? lv : -INFINITY;
  if (e == 0) {
    tau_s = -1.0f;
    ncand = 0;
  }
  const float mx = BlockMax16(l, red);
  const float ex = valid ? expf(l - mx) : 0.0f;
  const float den = BlockSum16(ex, red);
  const float p = valid ? ex / den : -1.0f;
  pall[e] = p;
  // group-of-8 maxima
  float g = fmaxf(p, halo::Dpp<0xB1>(p));
  g = fmaxf(g, halo::Dpp<0x4E>(g));
  g = fmaxf(g, halo::Dpp<0x141>(g));
  const std::uint32_t G = (E + 7) / 8;
  if (e % 8 == 0 && e / 8 < G) gmax[e / 8] = g;
  __syncthreads();
  if (k <= G && G <= kWave) {
    // tau = the k-th largest group maximum, by a bitwise search over the keys in wave 0 (probability bits + 1;
    // probabilities are >= 0, so their bit patterns order like the values; 0 marks a lane without a group)
    if (e < kWave) {
      const std::uint32_t key = e < G ? __float_as_uint(gmax[e]) + 1u : 0u;
      std::uint32_t thr = 0;
      for (int bit = 30; bit >= 0; --bit) {
        const std::uint32_t cand = thr | (1u << bit);
        if (static_cast<std::uint32_t>(__builtin_popcountll(__ballot(key >= cand))) >= k) thr = cand;
      }
      if (e == 0) tau_s = __uint_as_float(thr - 1u);
    }
  } else if (k <= G && e < G) {
    const float mine = gmax[e];
    std::uint32_t r = 0;
    for (std::uint32_t j = 0; j < G; ++j) {
      const float gj = gmax[j];
      r += (gj > mine) || (gj == mine && j < e);
    }
    if (r == k - 1) tau_s = mine;
  }
  __syncthreads();
  const float tau = tau_s;
  const bool cand = valid && p >= tau;
  if (cand) {
    const std::uint32_t pos = atomicAdd(&ncand, 1u);
    if (pos < kCand) {
      cp[pos] = p;
      ci[pos] = e;
    }
  }
  __syncthreads();
  const std::uint32_t n = ncand;
  if (n <= kCand) {
    if (cand) {
      std::uint32_t r = 0;
#pragma unroll 8
      for (std::uint32_t j = 0; j < n; ++j) {
        const float pj = cp[j];
        r += (pj > p) || (pj == p && ci[j] < e);
      }
      if (r < k) {
        selp[r] = p;
        seli[r] = e;
      }
    }
  } else if (cand) {
    // more candidates than the scratch holds (massive ties): rank against every expert
    std::uint32_t r = 0;
    for (std::uint32_t j = 0; j < E; ++j) {
      const float pj = pall[j];
      r += (pj > p) || (pj == p && j < e);
    }
    if (r < k) {
      selp[r] = p;
      seli[r] = e;
    }
  }
  __syncthreads();
  if (e == 0) {
    float sum = 0.0f;
    for (std::uint32_t s = 0; s < k; ++s) sum += selp[s];
    red[0] = fmaxf(sum, 6.103515625e-5f);
  }
  __syncthreads();
  if (e < k) {
    ids[static_cast<std::size_t>(t) * k + e] = seli[e];
    weights[static_cast<std::size_t>(t) * k + e] = selp[e] / red[0];
  }
}

// The same routing with one wave per token (WaveTopK: kPer 8 for E <= 512, 16 for E <= 1024), k <= 64: grid (T),
// block 64. Shorter than the block kernel above for decode batches (no block-wide reductions, no atomics).
//   logits [T][E] -> ids [T][k], weights [T][k]
#define HALO_MOE_TOPK_W(NAME, PER)                                                                                 \
  extern "C" __global__ void __launch_bounds__(64) NAME(const float* __restrict__ logits,                          \
                                                        std::uint32_t* __restrict__ ids, float* __restrict__ weights, \
                                                        std::uint32_t E, std::uint32_t k) {                        \
    __shared__ std::uint32_t lids[kWave];                                                                          \
    __shared__ float lw[kWave];                                                                                    \
    __shared__ TopKScratch sc;                                                                                     \
    const std::size_t t = blockIdx.x;                                                                              \
    WaveTopK<PER>(logits + t * E, E, k, ids + t * k, weights + t * k, lids, lw, sc);                               \
  }
HALO_MOE_TOPK_W(halo_moe_topk_w512, 8)
HALO_MOE_TOPK_W(halo_moe_topk_w1024, 16)
#undef HALO_MOE_TOPK_W

// grid (T * k + 1, ceil(max(ff, sff) / 4)), block 256: wave w computes ff row j = 4 * blockIdx.y + w of gate and
// up (two rows of H int8, kSteps = H / 1024 loads each per lane). Block x < T * k is routed pair x (token x / k,
// slot x % k); the block of the first token that selected an expert computes that expert for every token that
// selected it (weights streamed once), the others exit: the union of experts over tokens without a separate
// bucketing pass. Block x = T * k is the shared expert for all tokens. Gate/up [E][ff][H] repacked Q8_0 (row
// stride H), shared gate/up [sff][H]. Output h = SiLU(gate) * up in fp32: h [T * k + T][hstride] (row t * k + s for
// routed pairs, T * k + t for the shared expert).
// kTopKPer > 0 (one token): the routing is done here, not by a halo_moe_topk launch before. Every routed block runs
// WaveTopK from the logits in its first wave (the shared expert's blocks skip it) and block (0, 0) also writes ids /
// weights for the down launch; the other blocks need only the ids and skip the renormalization. At one token the
// redundant ranking (one wave per block) costs less than a launch.
template <int kSteps, int kTopKPer = 0>
__device__ __forceinline__ void MoeGateUp(
    const std::int8_t* __restrict__ gq, const std::uint16_t* __restrict__ gd, const std::int8_t* __restrict__ uq,
    const std::uint16_t* __restrict__ ud, const std::int8_t* __restrict__ sgq, const std::uint16_t* __restrict__ sgd,
    const std::int8_t* __restrict__ suq, const std::uint16_t* __restrict__ sud, const std::int8_t* __restrict__ xq,
    const float* __restrict__ xs, const std::uint32_t* __restrict__ ids_in, float* __restrict__ h, std::uint32_t T,
    std::uint32_t ff, std::uint32_t sff, std::uint32_t k, std::uint32_t hstride,
    const float* __restrict__ logits = nullptr, std::uint32_t E = 0, std::uint32_t* __restrict__ ids_out = nullptr,
    float* __restrict__ w_out = nullptr) {
  constexpr std::uint32_t H = kSteps * kWave * 16;
  constexpr std::uint32_t nblk = H / 32;
  const std::uint32_t px = blockIdx.x;
  const bool shared = px == T * k;
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const std::uint32_t j = blockIdx.y * (blockDim.x / kWave) + wave;
  __shared__ std::uint32_t rows_s[kMoeMaxT];  // h row of each pair, ascending token
  __shared__ std::uint32_t tokmask;
  __shared__ std::uint32_t owner;
  __shared__ std::uint32_t ids_l[kTopKPer > 0 ? 16 : 1];
  __shared__ float w_l[kTopKPer > 0 ? 16 : 1];
  __shared__ TopKScratch tsc[1];
  std::uint32_t np, f;
  std::size_t e = 0;
  const std::uint32_t* ids = ids_in;
  // the activation pieces of the block's first row (its pair's token; token 0 for the shared expert) do not depend
  // on the routing: loaded first, they land while the routing and the ownership check run
  int4 x0[kSteps];
  float s0[kSteps];
  // likewise this thread's entry of the pair ids (several tokens: the ownership check reads them all)
  std::uint32_t idpre = 0;
  if constexpr (kTopKPer == 0) idpre = ids_in[min(static_cast<std::uint32_t>(threadIdx.x), T * k - 1)];
  {
    const std::uint32_t tok0 = shared ? 0u : px / k;
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      const std::uint32_t c = st * kWave * 16 + lane * 16;
      x0[st] = *reinterpret_cast<const int4*>(xq + static_cast<std::size_t>(tok0) * H + c);
      s0[st] = xs[static_cast<std::size_t>(tok0) * nblk + c / 32];
    }
  }
  if (shared) {
    if (sgq == nullptr || blockIdx.y * (blockDim.x / kWave) >= sff) return;
    np = T;
    f = sff;
  } else {
    if (blockIdx.y * (blockDim.x / kWave) >= ff) return;
    if constexpr (kTopKPer > 0) {
      HALO_PHASE(3, 0);
      if (wave == 0) {
        const bool first = blockIdx.x == 0 && blockIdx.y == 0;
        WaveTopK<kTopKPer>(logits, E, k, first ? ids_out : nullptr, first ? w_out : nullptr, ids_l, first ? w_l : nullptr,
                           tsc[0]);
        HALO_PHASE(3, 1);
      }
      __syncthreads();
      HALO_PHASE(3, 2);
      ids = ids_l;
    }
    e = ids[px];
    np = 0;
    f = ff;
  }
  const std::int8_t* q0 = shared ? sgq : gq + e * ff * H;
  const std::uint16_t* d0 = shared ? sgd : gd + e * ff * nblk;
  const std::int8_t* q1 = shared ? suq : uq + e * ff * H;
  const std::uint16_t* d1 = shared ? sud : ud + e * ff * nblk;
  // the two weight rows, issued before the ownership check (the check only decides whether to use them)
  const std::uint32_t jr = min(j, f - 1);
  int4 w[2][kSteps];
  float sw[2][kSteps];
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {
    const std::uint32_t c = st * kWave * 16 + lane * 16;
    w[0][st] = __builtin_bit_cast(int4, __builtin_nontemporal_load(
                                           reinterpret_cast<const halo::V4i*>(q0 + static_cast<std::size_t>(jr) * H + c)));
    w[1][st] = __builtin_bit_cast(int4, __builtin_nontemporal_load(
                                           reinterpret_cast<const halo::V4i*>(q1 + static_cast<std::size_t>(jr) * H + c)));
    sw[0][st] = F16(d0[static_cast<std::size_t>(jr) * nblk + c / 32]);
    sw[1][st] = F16(d1[static_cast<std::size_t>(jr) * nblk + c / 32]);
  }
  std::uint32_t row1 = 0;  // T = 1: the one h row (the k experts of one token are distinct: no union to form)
  if (T == 1) {
    np = 1;
    row1 = shared ? k : px;
  } else if (shared) {
    if (threadIdx.x < T) rows_s[threadIdx.x] = T * k + threadIdx.x;
  } else {
    const std::uint32_t t = px / k;
    if (threadIdx.x == 0) {
      tokmask = 0;
      owner = 1;
    }
    __syncthreads();
    for (std::uint32_t i = threadIdx.x; i < T * k; i += blockDim.x)
      if ((i == threadIdx.x ? idpre : ids[i]) == e) {
        if (i / k < t) owner = 0;
        atomicOr(&tokmask, 1u << (i / k));
      }
    __syncthreads();
    if (!owner) return;
    const std::uint32_t m = tokmask;
    np = static_cast<std::uint32_t>(__builtin_popcount(m));
    for (std::uint32_t i = threadIdx.x; i < T * k; i += blockDim.x)
      if ((i == threadIdx.x ? idpre : ids[i]) == e) rows_s[__builtin_popcount(m & ((1u << (i / k)) - 1u))] = i;
  }
  if (T > 1) __syncthreads();
  if (j >= f) return;
  for (std::uint32_t lp = 0; lp < np; ++lp) {
    const std::uint32_t row = T == 1 ? row1 : rows_s[lp];
    const std::uint32_t tok = shared ? row - T * k : row / k;
    const std::int8_t* xt = xq + static_cast<std::size_t>(tok) * H;
    const float* st_ = xs + static_cast<std::size_t>(tok) * nblk;
    float g = 0.0f, u = 0.0f;
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      const std::uint32_t c = st * kWave * 16 + lane * 16;
      // the first row's pieces were loaded at the start (lp = 0 is the pair's own token, or token 0 shared)
      const int4 xv = lp == 0 ? x0[st] : *reinterpret_cast<const int4*>(xt + c);
      const float sx = lp == 0 ? s0[st] : st_[c / 32];
      g += sw[0][st] * (sx * static_cast<float>(Dot16(w[0][st], xv)));
      u += sw[1][st] * (sx * static_cast<float>(Dot16(w[1][st], xv)));
    }
    if constexpr (kTopKPer > 0) HALO_PHASE(3, 3);
    g = halo::GroupSum(g);
    u = halo::GroupSum(u);
    if (lane == 0) h[static_cast<std::size_t>(row) * hstride + j] = halo::Silu(g) * u;
  }
  if constexpr (kTopKPer > 0) HALO_PHASE(3, 4);
}

#define HALO_MOE_GATE_UP(S)                                                                                        \
  extern "C" __global__ void __launch_bounds__(256) halo_moe_gate_up_q8_s##S(                                     \
      const std::int8_t* gq, const std::uint16_t* gd, const std::int8_t* uq, const std::uint16_t* ud,             \
      const std::int8_t* sgq, const std::uint16_t* sgd, const std::int8_t* suq, const std::uint16_t* sud,         \
      const std::int8_t* xq, const float* xs, const std::uint32_t* ids, float* h, std::uint32_t T,                \
      std::uint32_t ff, std::uint32_t sff, std::uint32_t k, std::uint32_t hstride) {                              \
    MoeGateUp<S>(gq, gd, uq, ud, sgq, sgd, suq, sud, xq, xs, ids, h, T, ff, sff, k, hstride);                      \
  }
HALO_MOE_GATE_UP(1)
HALO_MOE_GATE_UP(2)
HALO_MOE_GATE_UP(4)
#undef HALO_MOE_GATE_UP

// The gate/up launch with the routing of its one token folded in: logits [E] (E <= 512 for _e512, <= 1024
// otherwise) -> ids / weights [k] (written by block (0, 0), read by the down launch), then as above with T = 1.
// grid (k + 1, ceil(max(ff, sff) / 4)), block 256.
#define HALO_MOE_GATE_UP_TOPK(S, NAME, PER)                                                                        \
  extern "C" __global__ void __launch_bounds__(256) NAME(                                                          \
      const std::int8_t* gq, const std::uint16_t* gd, const std::int8_t* uq, const std::uint16_t* ud,             \
      const std::int8_t* sgq, const std::uint16_t* sgd, const std::int8_t* suq, const std::uint16_t* sud,         \
      const std::int8_t* xq, const float* xs, const float* logits, std::uint32_t* ids, float* weights, float* h,  \
      std::uint32_t E, std::uint32_t ff, std::uint32_t sff, std::uint32_t k, std::uint32_t hstride) {             \
    MoeGateUp<S, PER>(gq, gd, uq, ud, sgq, sgd, suq, sud, xq, xs, nullptr, h, 1, ff, sff, k, hstride, logits, E,  \
                      ids, weights);                                                                               \
  }
HALO_MOE_GATE_UP_TOPK(1, halo_moe_gate_up_topk_q8_s1, 16)
HALO_MOE_GATE_UP_TOPK(2, halo_moe_gate_up_topk_q8_s2, 16)
HALO_MOE_GATE_UP_TOPK(4, halo_moe_gate_up_topk_q8_s4, 16)
HALO_MOE_GATE_UP_TOPK(1, halo_moe_gate_up_topk_q8_s1_e512, 8)
HALO_MOE_GATE_UP_TOPK(2, halo_moe_gate_up_topk_q8_s2_e512, 8)
HALO_MOE_GATE_UP_TOPK(4, halo_moe_gate_up_topk_q8_s4_e512, 8)
#undef HALO_MOE_GATE_UP_TOPK

// grid (ceil(H / R), T), block 64 * (k + 1) (<= 1024), R = 8 (halo_moe_down_q8) or 16 (_r16): wave s < k streams
// R rows of expert ids[t][s]'s down matrix (R / 2 KB contiguous; two rows per pass of 32 lanes x 16 bytes), wave k
// the shared expert's; each wave quantizes its h row per 32 values (amax / 127, round
// half to even; a 32-value block is two adjacent lanes) and the block combines in slot order through LDS:
//   out[t][r] = sum over s < k, in order, of weights[t][s] * (W_d[ids[t][s]][r] . q8(h[t * k + s])),
//               then + sigmoid(sgl[t]) * (W_sd[r] . q8(h[T * k + t])).
// Down [E][H][ff] repacked (row stride ff), shared down [H][sff]; ff, sff <= 512.
template <int kDownRows>
__device__ __forceinline__ void MoeDown(
    const std::int8_t* __restrict__ dq, const std::uint16_t* __restrict__ dd, const std::int8_t* __restrict__ sdq,
    const std::uint16_t* __restrict__ sdd, const float* __restrict__ h, const std::uint32_t* __restrict__ ids,
    const float* __restrict__ weights, const float* __restrict__ sgl, float* __restrict__ out, std::uint32_t T,
    std::uint32_t H, std::uint32_t ff, std::uint32_t sff, std::uint32_t k, std::uint32_t hstride) {
  __shared__ float part[33][kDownRows];
  __shared__ float wslot[33];
  // (the wave index through readfirstlane: the compiler then keeps it, and the expert id load, scalar)
  const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave,
                      sub = lane / 32, l = lane % 32;
  const std::uint32_t t = blockIdx.y, r0 = blockIdx.x * kDownRows;
  const bool shared = wave == k;
  HALO_PHASE(5, 0);
  // the combine weights are loaded now (unconditionally, from clamped addresses: a load under a branch would wait
  // at the join for its round trip before anything else is issued) and put in LDS after the dot products
  const float wv = weights[t * k + min(threadIdx.x, k - 1)];
  const float sgv = *(sgl != nullptr ? sgl + t : weights + t * k);
  if (wave < k || (shared && sdq != nullptr)) {
    const std::uint32_t f = shared ? sff : ff;
    const std::uint32_t hrow = shared ? T * k + t : t * k + wave;
    const std::uint32_t c = l * 16;
    const bool in = c < f;
    // loads from a clamped address, then a select: a load under a branch would cost a vmcnt(0) wait
    const std::uint32_t cc = in ? c : 0;
    // h: lane (sub, l) loads and quantizes values c + 8 sub .. + 7 of the 16 its dot products cover (a 32-value
    // block spans lanes 2i, 2i + 1 of both halves); the halves then swap their codes. Loads are unconditional, and
    // issued before the expert id is even read: loads complete in order, so h is in registers, and quantized,
    // while the weight rows stream in.
    const float4* hp = reinterpret_cast<const float4*>(h + static_cast<std::size_t>(hrow) * hstride + cc + 8 * sub);
    const float4 ha = hp[0], hb = hp[1];
    __builtin_amdgcn_sched_barrier(0);
    const std::size_t e = shared ? 0 : ids[t * k + wave];
    const std::int8_t* base = shared ? sdq : dq + e * H * f;
    const std::uint16_t* dbase = shared ? sdd : dd + e * H * (f / 32);
    int4 q[kDownRows / 2];
    float sw[kDownRows / 2];
#pragma unroll
    for (int p = 0; p < kDownRows / 2; ++p) {
      const std::uint32_t r = min(r0 + 2 * p + sub, H - 1);
      const int4 qv = __builtin_bit_cast(
          int4, __builtin_nontemporal_load(reinterpret_cast<const halo::V4i*>(base + static_cast<std::size_t>(r) * f + cc)));
      const float sv = F16(dbase[static_cast<std::size_t>(r) * (f / 32) + cc / 32]);
      q[p] = in ? qv : make_int4(0, 0, 0, 0);
      sw[p] = in ? sv : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);
    HALO_PHASE(5, 1);
    float hv[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      hv[i] = in ? hv[i] : 0.0f;
      amax = fmaxf(amax, fabsf(hv[i]));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    amax = fmaxf(amax, halo::Dpp<0xB1>(amax));
    const float scale = amax / 127.0f;
    int own[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      std::uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int qv = scale > 0.0f ? static_cast<int>(rintf(hv[4 * i + b] / scale)) : 0;
        word |= (static_cast<std::uint32_t>(qv) & 0xFFu) << (8 * b);
      }
      own[i] = static_cast<int>(word);
    }
    const int other0 = __shfl_xor(own[0], 32), other1 = __shfl_xor(own[1], 32);
    const int4 hq = sub == 0 ? make_int4(own[0], own[1], other0, other1) : make_int4(other0, other1, own[0], own[1]);
#pragma unroll
    for (int p = 0; p < kDownRows / 2; ++p) {
      const float v = halo::GroupSum<32>(sw[p] * (scale * static_cast<float>(Dot16(q[p], hq))));
      if (l == 0) part[wave][2 * p + sub] = v;
    }
  }
  HALO_PHASE(5, 2);
  if (threadIdx.x < k) wslot[threadIdx.x] = wv;
  if (threadIdx.x == k) wslot[k] = sdq != nullptr ? halo::Sigmoid(sgv) : 0.0f;
  __syncthreads();
  HALO_PHASE(5, 3);
  if (threadIdx.x < kDownRows && r0 + threadIdx.x < H) {
    float acc = 0.0f;
    for (std::uint32_t s = 0; s < k; ++s) acc += wslot[s] * part[s][threadIdx.x];
    if (sdq != nullptr) acc += wslot[k] * part[k][threadIdx.x];
    out[static_cast<std::size_t>(t) * H + r0 + threadIdx.x] = acc;
  }
  HALO_PHASE(5, 4);
}
// 8 rows per block at one token (more blocks in flight); 16 for token batches, which halves the h rows each block
// reads and quantizes again.
#define HALO_MOE_DOWN(NAME, R)                                                                                     \
  extern "C" __global__ void __launch_bounds__(1024) NAME(                                                        \
      const std::int8_t* __restrict__ dq, const std::uint16_t* __restrict__ dd, const std::int8_t* __restrict__ sdq, \
      const std::uint16_t* __restrict__ sdd, const float* __restrict__ h, const std::uint32_t* __restrict__ ids,   \
      const float* __restrict__ weights, const float* __restrict__ sgl, float* __restrict__ out, std::uint32_t T,  \
      std::uint32_t H, std::uint32_t ff, std::uint32_t sff, std::uint32_t k, std::uint32_t hstride) {             \
    MoeDown<R>(dq, dd, sdq, sdd, h, ids, weights, sgl, out, T, H, ff, sff, k, hstride);                            \
  }
HALO_MOE_DOWN(halo_moe_down_q8, 8)
HALO_MOE_DOWN(halo_moe_down_q8_r16, 16)
#undef HALO_MOE_DOWN

// Reference-named router top-k (src/kernels/core.hip:1110-1120): one token per block (grid 1 or T), the first
// wave computes softmax/top-k of `n` logits; ids/weights receive k entries.
extern "C" __global__ void __launch_bounds__(64)
    halo_router_topk(const float* logits, std::uint32_t* ids, float* weights, std::uint32_t n, std::uint32_t k) {
  __shared__ std::uint32_t scratch[64];
  __shared__ float wscratch[64];
  __shared__ TopKScratch sc;
  WaveTopK<16>(logits, n, k, ids, weights, scratch, wscratch, sc);
}
extern "C" __global__ void __launch_bounds__(64)
    halo_router_topk_rows(const float* logits, std::uint32_t* ids, float* weights, std::uint32_t n, std::uint32_t k) {
  __shared__ std::uint32_t scratch[64];
  __shared__ float wscratch[64];
  __shared__ TopKScratch sc;
  const std::size_t t = blockIdx.x;
  WaveTopK<16>(logits + t * n, n, k, ids + t * k, weights + t * k, scratch, wscratch, sc);
}
