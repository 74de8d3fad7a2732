// Shared device helpers for the gfx950 (CDNA4, wave64) code object.
//
// Kernel ABI (reference src/rt/device.hpp:8-11): every kernel is extern "C" __global__; pointer parameters are
// device buffers, every other parameter is a by-value scalar of at most 8 bytes. Kernels are looked up by name.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

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
