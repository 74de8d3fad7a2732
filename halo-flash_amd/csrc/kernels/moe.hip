// MoE decode layer for T <= 16 tokens (gfx950, wave64): router, softmax/top-k with the session union of experts,
// grouped gate/up + SwiGLU over the active experts, and the down projection with the routed combine.
//
// Reference semantics: ReferenceModel::Moe (src/model/reference.cpp:530-578), cpu::RouteTopK
// (src/model/cpu_ops.cpp:187-207), GPU RouterTopk (src/kernels/core.hip:1053-1108), session-union bucketing
// halo_moe_bucket_b (src/kernels/batch_decode.hip:417-446).
//
// Launches (all take device buffers only, so one captured graph replays for any routing):
//   1. halo_moe_router     logits[t][e] = W_r[e] . x[t] (fp32), shared-gate logit, x quantized per 32 (int8).
//   2. halo_moe_route      one wave per token: softmax, top-k (ties -> lower id), renormalized weights; then the
//                          union U of experts over tokens (ascending id) with each expert's (token, slot) pairs.
//   3. halo_moe_gate_up_q8 block (active expert u, 32 ff rows): gate and up rows streamed once for all of the
//                          expert's pairs, h = SiLU(g) * u, quantized per 32 into hq[pair]. The shared expert is
//                          the extra u = maxU, with pairs T*k + t.
//   4. halo_moe_down_q8    a wave owns 2 output rows for every token: sum over slots in slot order of
//                          w[t][s] * (W_d[e][r] . h[pair]), then + sigmoid(shared gate) * (W_sd[r] . h_shared).
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

namespace {
// Softmax over E logits and top-k of the probabilities for one token, one wave. Returns (in lane 0's registers
// and written to ids/weights) the k ids in descending probability, ties to the lower id, and the weights
// renormalized by max(sum, 2^-14) (src/model/cpu_ops.cpp:187-207; sum accumulated in slot order).
constexpr int kMaxPerLane = 16;  // E <= 1024

__device__ void WaveTopK(const float* logits, std::uint32_t E, std::uint32_t k, std::uint32_t* ids, float* weights,
                         std::uint32_t* lds_ids) {
  const std::uint32_t lane = threadIdx.x % kWave;
  float p[kMaxPerLane];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const std::uint32_t e = lane + kWave * i;
    p[i] = e < E ? logits[e] : -INFINITY;
    mx = fmaxf(mx, p[i]);
  }
  mx = halo::GroupMax(mx);
  float den = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const std::uint32_t e = lane + kWave * i;
    p[i] = e < E ? expf(p[i] - mx) : 0.0f;
    den += p[i];
  }
  den = halo::GroupSum(den);
  std::uint32_t taken = 0;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const std::uint32_t e = lane + kWave * i;
    p[i] = e < E ? p[i] / den : -1.0f;
  }
  float sum = 0.0f;
  for (std::uint32_t s = 0; s < k; ++s) {
    float v = -2.0f;
    std::uint32_t at = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i)
      if (!((taken >> i) & 1u) && p[i] > v) {  // ascending i: the first maximum has the lowest id in this lane
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
    sum += v;  // every lane holds the same v: slot-order sum
    if (lane == 0) {
      ids[s] = at;
      weights[s] = v;
      lds_ids[s] = at;
    }
  }
  sum = fmaxf(sum, 6.103515625e-5f);
  if (lane == 0)
    for (std::uint32_t s = 0; s < k; ++s) weights[s] = weights[s] / sum;
}
}  // namespace

// One block of 1024 threads. logits [T][E] -> ids [T][k], weights [T][k]; the union of experts:
//   route[0] = U, expert[u] (ascending id), pair_begin[u] (U + 1 entries; pairs of expert u are
//   [pair_begin[u], pair_begin[u+1]) in ascending token order), pair_token[p], pair_of[t][s] = p.
extern "C" __global__ void __launch_bounds__(1024)
    halo_moe_route(const float* __restrict__ logits, std::uint32_t* __restrict__ ids, float* __restrict__ weights,
                   std::uint32_t* __restrict__ route, std::uint32_t* __restrict__ expert,
                   std::uint32_t* __restrict__ pair_begin, std::uint32_t* __restrict__ pair_token,
                   std::uint32_t* __restrict__ pair_of, std::uint32_t T, std::uint32_t E, std::uint32_t k) {
  __shared__ std::uint32_t sel[kMoeMaxT * 32];
  __shared__ std::uint32_t ubeg[1024];
  __shared__ std::uint32_t wtot[2][16];
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (wave < T)
    WaveTopK(logits + static_cast<std::size_t>(wave) * E, E, k, ids + wave * k, weights + wave * k, sel + wave * k);
  __syncthreads();
  // per expert: number of pairs; exclusive scans of (active, count) over experts
  const std::uint32_t e = threadIdx.x;
  std::uint32_t cnt = 0;
  if (e < E)
    for (std::uint32_t i = 0; i < T * k; ++i) cnt += sel[i] == e;
  std::uint32_t a = cnt > 0, c = cnt;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {  // inclusive wave scan
    const std::uint32_t ao = __shfl_up(a, o, kWave), co = __shfl_up(c, o, kWave);
    if (lane >= static_cast<std::uint32_t>(o)) {
      a += ao;
      c += co;
    }
  }
  if (lane == kWave - 1) {
    wtot[0][wave] = a;
    wtot[1][wave] = c;
  }
  __syncthreads();
  std::uint32_t abase = 0, cbase = 0;
  for (std::uint32_t w = 0; w < wave; ++w) {
    abase += wtot[0][w];
    cbase += wtot[1][w];
  }
  const std::uint32_t aex = abase + a - (cnt > 0), cex = cbase + c - cnt;
  if (e < E) {
    ubeg[e] = cex;
    if (cnt > 0) {
      expert[aex] = e;
      pair_begin[aex] = cex;
    }
  }
  if (threadIdx.x == blockDim.x - 1) {
    std::uint32_t U = 0;
    for (std::uint32_t w = 0; w < blockDim.x / kWave; ++w) U += wtot[0][w];
    route[0] = U;
    pair_begin[U] = T * k;
  }
  __syncthreads();
  if (threadIdx.x < T * k) {
    const std::uint32_t t = threadIdx.x / k, ex = sel[threadIdx.x];
    std::uint32_t pos = 0;
    for (std::uint32_t i = 0; i < t * k; ++i) pos += sel[i] == ex;  // earlier tokens routed to the same expert
    const std::uint32_t p = ubeg[ex] + pos;
    pair_token[p] = t;
    pair_of[threadIdx.x] = p;
  }
}

namespace {
constexpr int kGuRowsPerWave = 4;  // 4 ff rows of gate and 4 of up
constexpr int kGuMaxSteps = 4;     // H <= 4096 (1024 columns per step with 64 lanes x 16 bytes)
}  // namespace

// grid (maxU + 1, ceil(max(ff, sff) / 32)), block 512 (8 waves x 4 ff rows = 32). Gate/up [E][ff][H] repacked
// Q8_0 (row stride qstride = H); shared gate/up [sff][H]. hq [T * (k + 1)][max ff] int8, hs [.][max ff / 32].
extern "C" __global__ void __launch_bounds__(512) halo_moe_gate_up_q8(
    const std::int8_t* __restrict__ gq, const std::uint16_t* __restrict__ gd, const std::int8_t* __restrict__ uq,
    const std::uint16_t* __restrict__ ud, const std::int8_t* __restrict__ sgq, const std::uint16_t* __restrict__ sgd,
    const std::int8_t* __restrict__ suq, const std::uint16_t* __restrict__ sud, const std::int8_t* __restrict__ xq,
    const float* __restrict__ xs, const std::uint32_t* __restrict__ route, const std::uint32_t* __restrict__ expert,
    const std::uint32_t* __restrict__ pair_begin, const std::uint32_t* __restrict__ pair_token,
    std::int8_t* __restrict__ hq, float* __restrict__ hs, std::uint32_t T, std::uint32_t H, std::uint32_t ff,
    std::uint32_t sff, std::uint32_t k, std::uint32_t maxU, std::uint32_t hstride) {
  const std::uint32_t ux = blockIdx.x, jb = blockIdx.y;
  const bool shared = ux == maxU;
  std::uint32_t pb, pe, f;
  const std::int8_t *q0, *q1;
  const std::uint16_t *d0, *d1;
  const std::uint32_t nblk = H / 32;
  if (shared) {
    if (sgq == nullptr) return;
    pb = T * k;
    pe = T * k + T;
    f = sff;
    q0 = sgq;
    d0 = sgd;
    q1 = suq;
    d1 = sud;
  } else {
    if (ux >= route[0]) return;
    const std::size_t e = expert[ux];
    pb = pair_begin[ux];
    pe = pair_begin[ux + 1];
    f = ff;
    q0 = gq + e * ff * H;
    d0 = gd + e * ff * nblk;
    q1 = uq + e * ff * H;
    d1 = ud + e * ff * nblk;
  }
  if (jb * 32 >= f) return;
  __shared__ float hbuf[kMoeMaxT][32];
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const std::uint32_t j0 = jb * 32 + wave * kGuRowsPerWave;
  const std::uint32_t steps = H / (kWave * 16);
  // weights: rows j0..j0+3 of gate (r < 4) and up (r >= 4), all column steps, loaded once
  int4 w[2 * kGuRowsPerWave][kGuMaxSteps];
  float sw[2 * kGuRowsPerWave][kGuMaxSteps];
#pragma unroll
  for (int r = 0; r < 2 * kGuRowsPerWave; ++r) {
    const std::int8_t* base = (r < kGuRowsPerWave ? q0 : q1) + static_cast<std::size_t>(j0 + r % kGuRowsPerWave) * H;
    const std::uint16_t* dbase =
        (r < kGuRowsPerWave ? d0 : d1) + static_cast<std::size_t>(j0 + r % kGuRowsPerWave) * nblk;
#pragma unroll
    for (int st = 0; st < kGuMaxSteps; ++st)
      if (st < static_cast<int>(steps)) {
        const std::uint32_t c = st * kWave * 16 + lane * 16;
        w[r][st] = __builtin_bit_cast(int4, __builtin_nontemporal_load(reinterpret_cast<const halo::V4i*>(base + c)));
        sw[r][st] = F16(dbase[c / 32]);
      }
  }
  for (std::uint32_t p = pb; p < pe; ++p) {
    const std::uint32_t t = shared ? p - T * k : pair_token[p];
    const std::int8_t* xt = xq + static_cast<std::size_t>(t) * H;
    const float* st_ = xs + static_cast<std::size_t>(t) * nblk;
    float acc[2 * kGuRowsPerWave];
#pragma unroll
    for (int r = 0; r < 2 * kGuRowsPerWave; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int st = 0; st < kGuMaxSteps; ++st)
      if (st < static_cast<int>(steps)) {
        const std::uint32_t c = st * kWave * 16 + lane * 16;
        const int4 xv = *reinterpret_cast<const int4*>(xt + c);
        const float sx = st_[c / 32];
#pragma unroll
        for (int r = 0; r < 2 * kGuRowsPerWave; ++r) acc[r] += sw[r][st] * (sx * static_cast<float>(Dot16(w[r][st], xv)));
      }
#pragma unroll
    for (int r = 0; r < 2 * kGuRowsPerWave; ++r) acc[r] = halo::GroupSum(acc[r]);
    if (lane < kGuRowsPerWave) {
      float g = acc[0], u = acc[kGuRowsPerWave];
#pragma unroll
      for (int r = 1; r < kGuRowsPerWave; ++r)
        if (static_cast<int>(lane) == r) {
          g = acc[r];
          u = acc[kGuRowsPerWave + r];
        }
      hbuf[p - pb][wave * kGuRowsPerWave + lane] = halo::Silu(g) * u;
    }
  }
  __syncthreads();
  // quantize h per 32 values: one half wave per pair
  const std::uint32_t hw = threadIdx.x / 32, hl = threadIdx.x % 32;
  for (std::uint32_t lp = hw; lp < pe - pb; lp += blockDim.x / 32) {
    const float v = hbuf[lp][hl];
    const float amax = halo::GroupMax<32>(fabsf(v));
    const float scale = amax / 127.0f;
    const int q = scale > 0.0f ? static_cast<int>(rintf(v / scale)) : 0;
    const std::uint32_t p = pb + lp;
    hq[static_cast<std::size_t>(p) * hstride + jb * 32 + hl] = static_cast<std::int8_t>(q);
    if (hl == 0) hs[static_cast<std::size_t>(p) * (hstride / 32) + jb] = scale;
  }
}

// grid ceil(H / 8), block 256 (4 waves x 2 rows; a row is 32 lanes x 16 bytes, ff <= 512 per step). Down
// [E][H][ff] repacked (qstride ff), shared down [H][sff]. out [T][H].
extern "C" __global__ void __launch_bounds__(256) halo_moe_down_q8(
    const std::int8_t* __restrict__ dq, const std::uint16_t* __restrict__ dd, const std::int8_t* __restrict__ sdq,
    const std::uint16_t* __restrict__ sdd, const std::int8_t* __restrict__ hq, const float* __restrict__ hs,
    const std::uint32_t* __restrict__ ids, const float* __restrict__ weights, const std::uint32_t* __restrict__ pair_of,
    const float* __restrict__ sgl, float* __restrict__ out, std::uint32_t T, std::uint32_t H, std::uint32_t ff,
    std::uint32_t sff, std::uint32_t k, std::uint32_t hstride) {
  constexpr int LPR = 32;
  const std::uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, sub = lane / LPR, l = lane % LPR;
  const std::uint32_t r = (blockIdx.x * (blockDim.x / kWave) + wave) * 2 + sub;
  const bool live = r < H;
  const std::uint32_t rr = live ? r : H - 1;
  for (std::uint32_t t = 0; t < T; ++t) {
    float acc = 0.0f;
    for (std::uint32_t s0 = 0; s0 <= k; s0 += 4) {
      // up to 4 slots' loads in flight; slot k is the shared expert
      float part[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const std::uint32_t s = s0 + i;
        part[i] = 0.0f;
        if (s > k) continue;
        const bool sh = s == k;
        if (sh && sdq == nullptr) continue;
        const std::uint32_t f = sh ? sff : ff;
        const std::size_t e = sh ? 0 : ids[t * k + s];
        const std::uint32_t p = sh ? T * k + t : pair_of[t * k + s];
        const std::int8_t* row = (sh ? sdq : dq + e * H * f) + static_cast<std::size_t>(rr) * f;
        const std::uint16_t* drow = (sh ? sdd : dd + e * H * (f / 32)) + static_cast<std::size_t>(rr) * (f / 32);
        float a = 0.0f;
        for (std::uint32_t c = l * 16; c < f; c += LPR * 16) {
          const int4 q = __builtin_bit_cast(int4, __builtin_nontemporal_load(reinterpret_cast<const halo::V4i*>(row + c)));
          const int4 hv = *reinterpret_cast<const int4*>(hq + static_cast<std::size_t>(p) * hstride + c);
          a += F16(drow[c / 32]) * (hs[static_cast<std::size_t>(p) * (hstride / 32) + c / 32] *
                                    static_cast<float>(Dot16(q, hv)));
        }
        part[i] = a;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const std::uint32_t s = s0 + i;
        if (s > k) break;
        const float v = halo::GroupSum<LPR>(part[i]);
        if (s < k)
          acc += weights[t * k + s] * v;
        else if (sdq != nullptr)
          acc += halo::Sigmoid(sgl[t]) * v;
      }
    }
    if (live && l == 0) out[static_cast<std::size_t>(t) * H + r] = acc;
  }
}

// Reference-named router top-k (src/kernels/core.hip:1110-1120): one token per block (grid 1 or T), the first
// wave computes softmax/top-k of `n` logits; ids/weights receive k entries.
extern "C" __global__ void __launch_bounds__(64)
    halo_router_topk(const float* logits, std::uint32_t* ids, float* weights, std::uint32_t n, std::uint32_t k) {
  __shared__ std::uint32_t scratch[64];
  WaveTopK(logits, n, k, ids, weights, scratch);
}
extern "C" __global__ void __launch_bounds__(64)
    halo_router_topk_rows(const float* logits, std::uint32_t* ids, float* weights, std::uint32_t n, std::uint32_t k) {
  __shared__ std::uint32_t scratch[64];
  const std::size_t t = blockIdx.x;
  WaveTopK(logits + t * n, n, k, ids + t * k, weights + t * k, scratch);
}
