// MoE decode without allocation: halo_op_moe_decode with its workspace in a fixed device array of this library, for
// callers that may not allocate device memory (code under stream capture, serving loops that forbid hipMalloc).
//
// The workspace (routing logits and tables, quantized x, h) lives in `scratch`, a file-scope __device__ array of
// kScratchBytes. Its device address is looked up once per device with hipGetSymbolAddress, with that device
// current, and kept in a per-device table; only that address ever reaches a kernel. Every call on a device shares
// the device's one array: two calls that overlap on one device (two streams, two threads) race on it. The MoE
// launches write every workspace byte they read before reading it, so nothing needs clearing between calls.
#include <hip/hip_runtime.h>

#include <array>
#include <mutex>

#include "engine.hpp"

namespace {

// 512 KiB: the C2 layer (512 experts top-10, hidden 2048, ff 512) at 16 tokens needs 422 KiB.
constexpr std::size_t kScratchBytes = std::size_t{512} << 10;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
std::array<void*, kMaxDevices> g_ptr{};  // scratch's device address per device, null until looked up

// Device `ordinal`'s scratch address, looked up on the first call on that device with that device made current
// (the calling thread's current device is restored afterwards).
void* ScratchOfDevice(int ordinal, char* err, std::size_t errlen) {
  if (ordinal < 0 || ordinal >= kMaxDevices)
    return halo::engine::SetErr(err, errlen, "moe noalloc: device %d out of range", ordinal), nullptr;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_ptr[ordinal] == nullptr) {
    int prev = -1;
    hipError_t e = hipGetDevice(&prev);
    if (e != hipSuccess) return halo::engine::SetErr(err, errlen, "hipGetDevice: %s", hipGetErrorString(e)), nullptr;
    if (prev != ordinal && (e = hipSetDevice(ordinal)) != hipSuccess)
      return halo::engine::SetErr(err, errlen, "hipSetDevice(%d): %s", ordinal, hipGetErrorString(e)), nullptr;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (prev != ordinal) (void)hipSetDevice(prev);
    if (e != hipSuccess || p == nullptr)
      return halo::engine::SetErr(err, errlen, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e)), nullptr;
    g_ptr[ordinal] = p;
  }
  return g_ptr[ordinal];
}

}  // namespace

extern "C" {

int halo_op_moe_decode_noalloc(halo_engine* eng, const halo_moe_weights* w, const float* x, float* out,
                               uint32_t tokens, char* err, size_t errlen) {
  if (w == nullptr || x == nullptr || out == nullptr)
    return halo::engine::SetErr(err, errlen, "moe noalloc: null weights, input or output"), -1;
  const std::size_t need = halo_op_moe_workspace_bytes(w, tokens);
  if (need == 0) {
    halo_moe_views v;  // reports why the layer is refused
    if (halo_op_moe_views(w, tokens, nullptr, &v, err, errlen) != 0) return -1;
    return halo::engine::SetErr(err, errlen, "moe noalloc: unsupported layer"), -1;
  }
  if (need > kScratchBytes)
    return halo::engine::SetErr(err, errlen,
                                "moe noalloc: %u tokens need %zu workspace bytes, more than the %zu-byte fixed scratch",
                                tokens, need, kScratchBytes),
           -1;
  if (eng == nullptr || eng->dev == nullptr) return halo::engine::SetErr(err, errlen, "moe noalloc: null engine"), -1;
  void* ws = ScratchOfDevice(halo_device_ordinal(eng->dev), err, errlen);
  if (ws == nullptr) return -1;
  return halo_op_moe_decode(eng, w, x, out, tokens, ws, kScratchBytes, err, errlen);
}

}  // extern "C"
