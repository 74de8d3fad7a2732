// Shared device helpers for the gfx950 (CDNA4, wave64) code object.
//
// Kernel ABI (reference src/rt/device.hpp:8-11): every kernel is extern "C" __global__; pointer parameters are
// device buffers, every other parameter is a by-value scalar of at most 8 bytes. Kernels are looked up by name.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

// Phase timing (diagnostic builds only, `make timing`): HALO_PHASE(k, i) records the device wall clock (wall_clock64,
// 100 MHz) at point i (< 8) of block blockIdx.x + gridDim.x blockIdx.y (< 4096) of kernel family k (0: the DeltaNet
// decode step, 1: the decode attention partials, 2: the RMSNorm-prologue projections, 3: the MoE gate/up launch with
// the routing, 4: the MoE router with the FFN norm, 5: MoE down + combine) into the code object's
// halo_phase_timing[k], read back with halo_read_global. In the product build it is empty.
#ifdef HALO_PHASE_TIMING
extern "C" __device__ unsigned long long halo_phase_timing[6][4096][8];
#define HALO_PHASE(k, i)                                                                                   \
  do {                                                                                                     \
    const unsigned b_ = blockIdx.x + gridDim.x * blockIdx.y;                                             \
    if (threadIdx.x == 0 && b_ < 4096) halo_phase_timing[k][b_][i] = wall_clock64();                     \
  } while (0)
#else
#define HALO_PHASE(k, i) \
  do {               \
  } while (0)
#endif

namespace halo {

constexpr int kWave = 64;

typedef int V4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float F16(std::uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ std::uint16_t ToF16Bits(float f) {
  return __builtin_bit_cast(std::uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ float Bf16(std::uint16_t h) { return __uint_as_float(static_cast<std::uint32_t>(h) << 16); }
__device__ __forceinline__ std::uint16_t ToBf16Bits(float v) {
  const std::uint32_t u = __float_as_uint(v);
  return static_cast<std::uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// Cross-lane data movement within 16-lane rows uses DPP (a VALU operand modifier, a few cycles) instead of the
// LDS permute unit; the four row results are combined with v_readlane. Control: quad_perm [1,0,3,2] = 0xB1,
// quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int kCtrl>
__device__ __forceinline__ float Dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}
template <int kCtrl>
__device__ __forceinline__ int DppI(int v) {
  return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xF, 0xF, false);
}
__device__ __forceinline__ float ReadLane(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Sum / max over groups of `kWidth` consecutive lanes (kWidth in {16, 32, 64}); every lane of the group gets the
// result. Each group must be entirely active (whole rows of 16 for widths 16 and 32 use only their own lanes).
template <int kWidth = kWave>
__device__ __forceinline__ float GroupSum(float v) {
  static_assert(kWidth == 16 || kWidth == 32 || kWidth == 64, "group width");
  v += Dpp<0xB1>(v);
  v += Dpp<0x4E>(v);
  v += Dpp<0x141>(v);
  v += Dpp<0x140>(v);
  if constexpr (kWidth == 16) {
    return v;
  } else if constexpr (kWidth == 32) {
    const float lo = ReadLane(v, 0) + ReadLane(v, 16), hi = ReadLane(v, 32) + ReadLane(v, 48);
    return (threadIdx.x & 32) ? hi : lo;
  } else {
    return (ReadLane(v, 0) + ReadLane(v, 16)) + (ReadLane(v, 32) + ReadLane(v, 48));
  }
}
template <int kWidth = kWave>
__device__ __forceinline__ float GroupMax(float v) {
  static_assert(kWidth == 16 || kWidth == 32 || kWidth == 64, "group width");
  v = fmaxf(v, Dpp<0xB1>(v));
  v = fmaxf(v, Dpp<0x4E>(v));
  v = fmaxf(v, Dpp<0x141>(v));
  v = fmaxf(v, Dpp<0x140>(v));
  if constexpr (kWidth == 16) {
    return v;
  } else if constexpr (kWidth == 32) {
    const float lo = fmaxf(ReadLane(v, 0), ReadLane(v, 16)), hi = fmaxf(ReadLane(v, 32), ReadLane(v, 48));
    return (threadIdx.x & 32) ? hi : lo;
  } else {
    return fmaxf(fmaxf(ReadLane(v, 0), ReadLane(v, 16)), fmaxf(ReadLane(v, 32), ReadLane(v, 48)));
  }
}
template <int kWidth = kWave>
__device__ __forceinline__ int GroupSumI(int v) {
  static_assert(kWidth == 64, "group width");
  v += DppI<0xB1>(v);
  v += DppI<0x4E>(v);
  v += DppI<0x141>(v);
  v += DppI<0x140>(v);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

// Sum / max over groups of 8 consecutive lanes (two DPP quad swaps, then the half-row mirror that pairs quad 0 with
// quad 1 of each 8). Both lanes of every pair add the same two operands, so all 8 lanes hold identical bits.
__device__ __forceinline__ float Group8Sum(float v) {
  v += Dpp<0xB1>(v);
  v += Dpp<0x4E>(v);
  return v + Dpp<0x141>(v);
}
__device__ __forceinline__ float Group8Max(float v) {
  v = fmaxf(v, Dpp<0xB1>(v));
  v = fmaxf(v, Dpp<0x4E>(v));
  return fmaxf(v, Dpp<0x141>(v));
}

// Q8_0 quantization of a 32-value block spread over 8 consecutive lanes, 4 values per lane (lane 8g + i holds values
// 4i .. 4i + 3 of block g): scale = amax / 127 (IEEE divide), code = rint(v / scale) (round half to even; 0 when the
// block is all zero). Returns the lane's 4 codes packed little-endian into one word; every lane of the 8 gets scale.
__device__ __forceinline__ std::uint32_t QuantQuad(const float4& v, float& scale) {
  const float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  scale = Group8Max(m) / 127.0f;
  const float e[4] = {v.x, v.y, v.z, v.w};
  std::uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = scale > 0.0f ? static_cast<int>(rintf(e[i] / scale)) : 0;
    word |= (static_cast<std::uint32_t>(q) & 0xFFu) << (8 * i);
  }
  return word;
}

// Block-wide reductions; `scratch` holds one float per wave. Every thread of the block must call them.
__device__ __forceinline__ float BlockSum(float v, float* scratch) {
  v = GroupSum(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, waves = (blockDim.x + kWave - 1) / kWave;
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float r = 0.0f;
  for (int w = 0; w < waves; ++w) r += scratch[w];
  return r;
}
__device__ __forceinline__ float BlockMax(float v, float* scratch) {
  v = GroupMax(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, waves = (blockDim.x + kWave - 1) / kWave;
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float r = -INFINITY;
  for (int w = 0; w < waves; ++w) r = fmaxf(r, scratch[w]);
  return r;
}

__device__ __forceinline__ float Sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float Silu(float x) { return x * Sigmoid(x); }
__device__ __forceinline__ float Softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Signed int8 x4 dot product accumulate: v_dot4_i32_i8.
__device__ __forceinline__ int Dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// 16 int8 x 16 int8 -> int32 (exact; |sum| <= 16 * 127 * 128).
__device__ __forceinline__ int Dot16(const int4& a, const int4& b) {
  int i = Dot4(a.x, b.x, 0);
  i = Dot4(a.y, b.y, i);
  i = Dot4(a.z, b.z, i);
  return Dot4(a.w, b.w, i);
}

// Counter-based hash (splitmix64 finalizer) for seeded synthetic tensors.
__device__ __forceinline__ std::uint64_t Mix64(std::uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
// Uniform in (0, 1] from the top 24 bits.
__device__ __forceinline__ float Unit(std::uint64_t h) {
  return (static_cast<float>(h >> 40) + 1.0f) * (1.0f / 16777216.0f);
}
// Standard normal from two hashes (Box-Muller).
__device__ __forceinline__ float Normal(std::uint64_t key) {
  const std::uint64_t a = Mix64(key), b = Mix64(key ^ 0xD1B54A32D192ED03ull);
  const float u1 = Unit(a), u2 = Unit(b);
  return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

}  // namespace halo

// ---- canonical row prologue: residual add, RMS norm and Q8 quantization of one activation row -----------------
// Every kernel that normalizes or quantizes a row in its prologue uses this decomposition, so all of them produce
// the same bits (sums of squares are explicit fused multiply-adds: left to contraction, the choice of which
// product of p1 + p2 gets fused differs between kernels, and so do the last bits): 256 threads, thread t holds the 8-value chunks c = t + 256 k (k < KC, c < n / 8) of the row;
// the sum of squares runs over a thread's chunks in order, then GroupSum, then the four wave sums in order.
// A 32-value Q8 block is the 4 chunks of 4 consecutive lanes (a DPP quad).
namespace halo {

// Block barrier for LDS traffic only: waits for this wave's LDS operations, then s_barrier. Unlike __syncthreads()
// (whose workgroup release fence also waits for every outstanding global load and store), loads issued ahead into
// registers stay in flight across it. Only for exchanges through LDS; the "memory" clobber keeps the compiler from
// moving memory accesses across it.
__device__ __forceinline__ void LdsSync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int KC>
struct Row8 {
  float v[KC][8];
};

// v = x (+ delta) for the chunks of this thread; chunks past n are zero. The loads are unconditional (a chunk past n
// reloads the last one and is then zeroed): a load under a branch costs a vmcnt(0) wait at the join.
template <int KC>
__device__ __forceinline__ void LoadRow8(const float* __restrict__ x, const float* __restrict__ delta, std::uint32_t n,
                                         Row8<KC>& r) {
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const std::uint32_t c = threadIdx.x + 256u * k, cc = min(c, n / 8 - 1);
    const bool in = c < n / 8;
    const float4 a = reinterpret_cast<const float4*>(x)[2 * cc], b = reinterpret_cast<const float4*>(x)[2 * cc + 1];
    r.v[k][0] = a.x, r.v[k][1] = a.y, r.v[k][2] = a.z, r.v[k][3] = a.w;
    r.v[k][4] = b.x, r.v[k][5] = b.y, r.v[k][6] = b.z, r.v[k][7] = b.w;
    {  // delta (or, without one, x again: a cache hit) is loaded either way and added times 1 or 0, so the load is
       // not moved under a branch; v + delta * 1 is v + delta exactly, v + x * 0 is v
      const float* dsrc = delta != nullptr ? delta : x;
      const float on = delta != nullptr ? 1.0f : 0.0f;
      const float4 e = reinterpret_cast<const float4*>(dsrc)[2 * cc],
                   f = reinterpret_cast<const float4*>(dsrc)[2 * cc + 1];
      r.v[k][0] += e.x * on, r.v[k][1] += e.y * on, r.v[k][2] += e.z * on, r.v[k][3] += e.w * on;
      r.v[k][4] += f.x * on, r.v[k][5] += f.y * on, r.v[k][6] += f.z * on, r.v[k][7] += f.w * on;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[k][e] = in ? r.v[k][e] : 0.0f;
  }
}

template <int KC>
__device__ __forceinline__ void StoreRow8(float* __restrict__ y, std::uint32_t n, const Row8<KC>& r) {
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const std::uint32_t c = threadIdx.x + 256u * k;
    if (c < n / 8) {
      reinterpret_cast<float4*>(y)[2 * c] = make_float4(r.v[k][0], r.v[k][1], r.v[k][2], r.v[k][3]);
      reinterpret_cast<float4*>(y)[2 * c + 1] = make_float4(r.v[k][4], r.v[k][5], r.v[k][6], r.v[k][7]);
    }
  }
}

// In place: v = v * (1 / sqrt(mean(v^2) + eps)) * w. Block of exactly 256 threads; red holds 4 floats.
template <int KC>
__device__ __forceinline__ void RmsNormRow8(Row8<KC>& r, const float* __restrict__ w, std::uint32_t n, float eps,
                                            float* red) {
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < KC; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(r.v[k][e], r.v[k][e], ss);
  ss = GroupSum(ss);
  __syncthreads();
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  ss = ((red[0] + red[1]) + red[2]) + red[3];
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const std::uint32_t c = threadIdx.x + 256u * k;
    if (c < n / 8) {
      if (w != nullptr) {  // kernel-uniform; a null w means unit weights
        const float4 a = reinterpret_cast<const float4*>(w)[2 * c], b = reinterpret_cast<const float4*>(w)[2 * c + 1];
        const float wv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) r.v[k][e] = r.v[k][e] * scale * wv[e];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) r.v[k][e] = r.v[k][e] * scale;
      }
    }
  }
}

// In place, per 128-value head (16 chunks = one 16-lane DPP row): v = RMSNorm(v) * w * sigmoid(z), the DeltaNet
// output norm (w [128] shared by heads, z [n] the gate row). Block of exactly 256 threads.
template <int KC>
__device__ __forceinline__ void GatedNormRow8(Row8<KC>& r, const float* __restrict__ z, const float* __restrict__ w,
                                              std::uint32_t n, float eps) {
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const std::uint32_t c = threadIdx.x + 256u * k;
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(r.v[k][e], r.v[k][e], ss);
    ss = GroupSum<16>(ss);
    if (c < n / 8) {
      const float scale = 1.0f / sqrtf(ss / 128.0f + eps);
      const float4 wa = reinterpret_cast<const float4*>(w)[2 * (c % 16)],
                   wb = reinterpret_cast<const float4*>(w)[2 * (c % 16) + 1];
      const float4 za = reinterpret_cast<const float4*>(z)[2 * c], zb = reinterpret_cast<const float4*>(z)[2 * c + 1];
      const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
      const float zv[8] = {za.x, za.y, za.z, za.w, zb.x, zb.y, zb.z, zb.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) r.v[k][e] = r.v[k][e] * scale * wv[e] * Sigmoid(zv[e]);
    }
  }
}

// RmsNormRow8 / GatedNormRow8 with the weights (and gate) already in registers, in the same chunk layout (w8: the
// 8 weights of this thread's position in its head). Same arithmetic, same bits.
template <int KC>
__device__ __forceinline__ void RmsNormRow8W(Row8<KC>& r, const Row8<KC>& w, std::uint32_t n, float eps, float* red) {
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < KC; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(r.v[k][e], r.v[k][e], ss);
  ss = GroupSum(ss);
  __syncthreads();
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  ss = ((red[0] + red[1]) + red[2]) + red[3];
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
#pragma unroll
  for (int k = 0; k < KC; ++k)
    if (threadIdx.x + 256u * k < n / 8)
#pragma unroll
      for (int e = 0; e < 8; ++e) r.v[k][e] = r.v[k][e] * scale * w.v[k][e];
}
template <int KC>
__device__ __forceinline__ void GatedNormRow8W(Row8<KC>& r, const Row8<KC>& z, const float (&w8)[8], std::uint32_t n,
                                               float eps) {
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const std::uint32_t c = threadIdx.x + 256u * k;
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(r.v[k][e], r.v[k][e], ss);
    ss = GroupSum<16>(ss);
    if (c < n / 8) {
      const float scale = 1.0f / sqrtf(ss / 128.0f + eps);
#pragma unroll
      for (int e = 0; e < 8; ++e) r.v[k][e] = r.v[k][e] * scale * w8[e] * Sigmoid(z.v[k][e]);
    }
  }
}

// Q8 quantization of the row (amax / 127, round half to even): xq [n] int8, xs [n / 32].
template <int KC>
__device__ __forceinline__ void QuantRow8(const Row8<KC>& r, std::uint32_t n, std::int8_t* xq, float* xs) {
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const std::uint32_t c = threadIdx.x + 256u * k;
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(r.v[k][e]));
    amax = fmaxf(amax, Dpp<0xB1>(amax));
    amax = fmaxf(amax, Dpp<0x4E>(amax));
    if (c < n / 8) {
      const float scale = amax / 127.0f;
      std::uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int q = scale > 0.0f ? static_cast<int>(rintf(r.v[k][e] / scale)) : 0;
        const std::uint32_t b = static_cast<std::uint32_t>(q) & 0xFFu;
        if (e < 4)
          lo |= b << (8 * e);
        else
          hi |= b << (8 * (e - 4));
      }
      reinterpret_cast<uint2*>(xq)[c] = make_uint2(lo, hi);
      if (threadIdx.x % 4 == 0) xs[c / 4] = scale;
    }
  }
}

}  // namespace halo

// ---- last-arriving block -------------------------------------------------------------------------------------
// Every block of a group of n calls this once (all threads). Returns true, in every thread, in exactly one block:
// the last to arrive, which then sees every global store the group made before arriving (agent-scope release by
// each block, acquire by the last; this writes back / invalidates the per-XCD L2 lines involved). The last block
// returns the counter to zero for the next launch. flag is one LDS word.
namespace halo {
__device__ __forceinline__ bool LastBlock(std::uint32_t* counter, std::uint32_t n, std::uint32_t* flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) *flag = atomicAdd(counter, 1u) == n - 1 ? 1u : 0u;
  __syncthreads();
  const bool last = *flag != 0u;
  if (last) {
    __threadfence();
    if (threadIdx.x == 0) atomicExch(counter, 0u);
  }
  return last;
}

// ---- attention head prologue (one wave per 256-dim head; lane l holds dims l + 64 i, i < 4) ------------------
// NEOX rotary angles of the dims this lane holds among the first `rot` (rot <= 128: dims l and l + 64) at
// position pos: freq = theta^(-2 j' / rot) with j' = j mod rot / 2. Not inlined: the precise powf / cosf / sinf are
// long, and a caller that needs the angles of a few positions keeps one copy of them.
struct RopeCS {
  float c[2], s[2];
};
__device__ __noinline__ RopeCS RopeAngles(std::uint32_t pos, std::uint32_t rot, float theta) {
  RopeCS r{{1.0f, 1.0f}, {0.0f, 0.0f}};
  const std::uint32_t lane = threadIdx.x % kWave, half = rot / 2;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const std::uint32_t j = lane + 64 * i;
    if (j < rot) {
      const std::uint32_t jj = j < half ? j : j - half;
      const float freq = powf(theta, -2.0f * static_cast<float>(jj) / static_cast<float>(rot));
      const float ang = static_cast<float>(pos) * freq;
      r.c[i] = cosf(ang);
      r.s[i] = sinf(ang);
    }
  }
  return r;
}
// x (this lane's 4 dims of one head, w the matching norm weights) -> RMSNorm(x) * w, then the NEOX rotation of the first rot dims: pairs
// (j, j + rot / 2), y_j c - y_{j + rot/2} s and y_j s + y_{j + rot/2} c. The whole wave calls it.
__device__ __forceinline__ void NormRopeHead(const float (&x)[4], const float (&w)[4], const RopeCS& cs,
                                             std::uint32_t rot, float eps, float (&out)[4]) {
  constexpr std::uint32_t d = 256;
  const std::uint32_t lane = threadIdx.x % kWave;
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss += x[i] * x[i];
  ss = GroupSum(ss);
  const float sc = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
  float y[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) y[i] = x[i] * sc * w[i];
  const std::uint32_t half = rot / 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[i] = y[i];
    const std::uint32_t j = lane + 64 * i;
    if (i < 2 && j < rot) {
      const std::uint32_t pj = j < half ? j + half : j - half;  // partner: element j + half or j - half
      float partner = 0.0f;
#pragma unroll
      for (int i2 = 0; i2 < 4; ++i2) {
        const float cand = __shfl(y[i2], pj % 64, kWave);
        if (static_cast<std::uint32_t>(i2) == pj / 64) partner = cand;
      }
      out[i] = j < half ? y[i] * cs.c[i] - partner * cs.s[i] : partner * cs.s[i] + y[i] * cs.c[i];
    }
  }
}

}  // namespace halo

namespace halo {
// fp32 operands on fp16 matrix cores: x enters as the pair hi = fp16(x), lo = fp16(x - hi) (|x - hi - lo| <= 2^-22 |x|
// for normal values) and each product as hi * hi + hi * lo + lo * hi on v_mfma_f32_16x16x32_f16 (products of halves
// are exact in the fp32 accumulator; the dropped lo * lo term is below 2^-22 of the product). Three fp16 MFMAs take
// 3/16 of the fp32 MFMA issue time of the same products. Operands must lie within the fp16 range (|x| < 65504).
typedef float V4F __attribute__((ext_vector_type(4)));
typedef _Float16 H8 __attribute__((ext_vector_type(8)));
typedef _Float16 H4 __attribute__((ext_vector_type(4)));

// hi / lo halves of s * a and s * b, packed two to a register (a in the low half): hi = fp16(s x), lo = fp16(s x -
// hi), one v_fma_mix per value and half (the product and the difference are formed exactly inside the mixed-precision
// FMA, so the result equals the convert / subtract / convert sequence bit for bit).
__device__ __forceinline__ void SplitPair(float a, float b, float s, std::uint32_t& hi, std::uint32_t& lo) {
  asm("v_fma_mixlo_f16 %0, %2, %4, 0\n\t"
      "v_fma_mixhi_f16 %0, %3, %4, 0\n\t"
      "v_fma_mixlo_f16 %1, %2, %4, -%0 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %1, %3, %4, -%0 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
      : "=&v"(hi), "=&v"(lo)
      : "v"(a), "v"(b), "v"(s));
}

// s: a power of two applied first (exact), so that the lo halves of the operand's typical values stay normal fp16
// numbers: a subnormal lo keeps only an absolute precision of 2^-25.
__device__ __forceinline__ void SplitHalves(const float (&x)[8], H8& hi, H8& lo, float s = 1.0f) {
  std::uint32_t h[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) SplitPair(x[2 * e], x[2 * e + 1], s, h[e], l[e]);
  hi = __builtin_bit_cast(H8, h);
  lo = __builtin_bit_cast(H8, l);
}
__device__ __forceinline__ void SplitHalves4(const float (&x)[4], H4& hi, H4& lo, float s = 1.0f) {
  std::uint32_t h[2], l[2];
  SplitPair(x[0], x[1], s, h[0], l[0]);
  SplitPair(x[2], x[3], s, h[1], l[1]);
  hi = __builtin_bit_cast(H4, h);
  lo = __builtin_bit_cast(H4, l);
}

// The power-of-two operand scale for a group of values of absolute maximum amax: `base` (the scale that keeps small
// values' lo halves normal) while amax * base stays below the fp16 maximum 65504, else 2^(15 - e) with amax < 2^e, so
// every scaled value lies below 2^15. Groups within the base range keep the same scale (and bits) as a fixed one.
__device__ __forceinline__ float SplitScale(float amax, float base) {
  if (amax * base < 65504.0f) return base;
  int e = 0;
  (void)frexpf(amax, &e);
  return ldexpf(1.0f, 15 - e);
}

__device__ __forceinline__ V4F Mfma3(const H8& ah, const H8& al, const H8& bh, const H8& bl, V4F c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, c, 0, 0, 0);
}

// Global -> LDS loads that bypass registers (wave-uniform LDS base in M0; lane l's element lands at base + 16 l or
// base + 4 l) and a wait on the vector-memory counter by count (loads complete in issue order).
__device__ __forceinline__ void DmaRow16(const void* sbase, std::uint32_t voff, std::uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void DmaDword(const void* addr, std::uint32_t lds) {
  asm volatile("global_load_lds_dword %0, off" ::"v"(addr), "{m0}"(lds) : "memory");
}
template <int N>
__device__ __forceinline__ void WaitVmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
}  // namespace halo
