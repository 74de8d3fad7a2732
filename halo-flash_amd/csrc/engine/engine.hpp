// Internal C++ side of halo_engine: kernel-id cache, argument packing and shared launch helpers.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <utility>
#include <string>
#include <type_traits>
#include <unordered_map>

#include "halo_ops.h"
#include "halo_rt.h"

struct halo_engine {
  halo_device* dev = nullptr;
  std::unordered_map<std::string, halo_kernel_id> ids;
  // Arrival counters for kernels whose last block finishes the work of the others (zeroed at create; every such
  // kernel returns its counters to zero). Kernels on the device's one stream never overlap, so slots are reused.
  halo_buffer sync{};
};

namespace halo::engine {

inline void SetErr(char* err, std::size_t errlen, const char* fmt, ...) {
  if (err == nullptr || errlen == 0) return;
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(err, errlen, fmt, ap);
  va_end(ap);
}

// Refuses null required device pointers of an operator: the kernels dereference them unconditionally, and a null
// read faults the GPU. `ptrs` pairs each required argument's name with its value.
inline int RequirePtrs(char* err, std::size_t errlen, const char* op,
                       std::initializer_list<std::pair<const char*, const void*>> ptrs) {
  for (const auto& np : ptrs)
    if (np.second == nullptr) return SetErr(err, errlen, "%s: %s is null", op, np.first), -1;
  return 0;
}

// Kernel argument builders (the reference's Arg::Buf / Arg::Val, src/rt/device.hpp:35-59).
inline halo_arg Ptr(const void* p) {
  halo_arg a{};
  a.kind = HALO_ARG_BUFFER;
  a.buffer.device = const_cast<void*>(p);
  a.buffer.bytes = 0;
  return a;
}
template <typename T>
inline halo_arg Val(T v) {
  static_assert(sizeof(T) <= 8 && std::is_trivially_copyable_v<T>);
  halo_arg a{};
  a.kind = HALO_ARG_SCALAR;
  a.size = sizeof(T);
  std::memcpy(a.bytes, &v, sizeof(T));
  return a;
}
inline halo_arg U32(std::uint32_t v) { return Val(v); }

inline halo_dim3 D3(std::uint32_t x, std::uint32_t y = 1, std::uint32_t z = 1) { return halo_dim3{x, y, z}; }

// Counter slots of halo_engine::sync.
constexpr std::uint32_t kSyncSlots = 1024;
constexpr std::uint32_t kSyncMoeRouter = 0;   // one
constexpr std::uint32_t kSyncProjTail = 1;    // one
constexpr std::uint32_t kSyncGdnHeads = 64;   // sessions * value heads (<= 960)
inline std::uint32_t* SyncCounters(halo_engine* eng, std::uint32_t slot) {
  return static_cast<std::uint32_t*>(eng->sync.device) + slot;
}

inline std::uint32_t CeilDiv(std::uint64_t a, std::uint64_t b) { return static_cast<std::uint32_t>((a + b - 1) / b); }

// Launch by name through the device layer.
template <std::size_t N>
inline int Launch(halo_engine* eng, const char* name, halo_dim3 grid, halo_dim3 block, const halo_arg (&args)[N],
                  char* err, std::size_t errlen) {
  return halo_engine_launch(eng, name, grid, block, args, N, err, errlen);
}

// The MoE prefill workspace (halo_op_moe_prefill): router logits [T][E], shared gate logit [T], x codes / scales,
// routing ids / weights [T][k], group counts and starts, the tile table, each sorted pair's token, pos[t k + s] (the
// sorted position of token t's slot s; the shared expert's pair of token t sits at T k + t), h [G][F] fp32 and its
// codes / scales, the down outputs y [G][H].
struct MoePrefillViews {
  float *logits, *sgl, *xs, *weights, *h, *hs, *y;
  std::int8_t *xq, *hq;
  std::uint32_t *ids, *count, *start, *tiles, *ntiles, *token, *pos;
  std::uint32_t max_tiles;
  std::size_t bytes;
};
int MoePrefillLayout(const halo_moe_weights* w, std::uint32_t T, void* ws, MoePrefillViews* v, char* err,
                     std::size_t errlen);

}  // namespace halo::engine

// The engine a model was created on (model.cpp; used by the GGUF loader).
struct halo_model;
halo_engine* halo_model_engine_of(const halo_model* m);
