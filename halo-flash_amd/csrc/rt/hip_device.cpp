// HIP implementation of the device C ABI (include/halo_rt.h) for MI355X (gfx950).
//
// Mirrors the reference's HipDevice (src/rt/hip_device.cpp): one non-blocking stream per device, code objects
// loaded with hipModuleLoadData, kernels resolved by name with hipModuleGetFunction, kernargs packed in declaration
// order (pointer = buffer address + offset, scalar = its bytes) and launched with hipModuleLaunchKernel, stream
// capture into an instantiated hipGraphExec.
#include "halo_rt.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <thread>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

struct halo_device {
  hipStream_t stream = nullptr;
  hipModule_t module = nullptr;
  std::vector<std::uint8_t> image;
  std::vector<hipFunction_t> functions;
  std::vector<std::string> names;
  bool capturing = false;
  std::size_t captured = 0;          // launches recorded since BeginCapture
  std::vector<void*> deferred_free;  // Free() calls made while capturing, released at EndCapture
  std::vector<std::pair<void*, std::size_t>> deferred_ranges;  // ReleaseRange() calls made while capturing
  int ordinal = 0;                                               // the HIP device this stream belongs to
  // per-launch event timing of eager launches (halo_profile_begin / _end)
  bool profiling = false;
  struct Timed {
    halo_kernel_id k;
    hipEvent_t a, b;
  };
  std::vector<Timed> timed;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  // page mapping (halo_page_bytes ... halo_unmap_page): 0 when the device has no virtual memory management
  std::size_t page_bytes = 0;
  hipMemAllocationProp prop{};
  // A mapping change is followed by kVmmSettle before the next launch or copy: the reference measured its GPU's
  // address translation lagging hipMemMap / hipMemUnmap by tens of microseconds with no HIP synchronization ordering
  // it (src/rt/hip_device.cpp:349-356); the same bounded wait here keeps a kernel from touching a page too early.
  std::chrono::steady_clock::time_point vmm_changed{};
  bool vmm_pending = false;
};

namespace {

void SetErr(char* err, std::size_t errlen, const char* fmt, ...) {
  if (err == nullptr || errlen == 0) return;
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(err, errlen, fmt, ap);
  va_end(ap);
}

bool Ok(hipError_t e, const char* what, char* err, std::size_t errlen) {
  if (e == hipSuccess) return true;
  SetErr(err, errlen, "%s: %s", what, hipGetErrorString(e));
  return false;
}

bool NotCapturing(halo_device* dev, const char* what, char* err, std::size_t errlen) {
  if (dev == nullptr) {
    SetErr(err, errlen, "%s: null device", what);
    return false;
  }
  if (!dev->capturing) return true;
  SetErr(err, errlen, "%s is not capturable", what);
  return false;
}

constexpr std::size_t kPageTarget = std::size_t{2} << 20;  // mapping granularity (the reference's 2 MB pages)
constexpr auto kVmmSettle = std::chrono::microseconds(1000);

void VmmStamp(halo_device* dev) {
  dev->vmm_changed = std::chrono::steady_clock::now();
  dev->vmm_pending = true;
}
// Waits out the settle interval after the last mapping change (before GPU work that may touch mapped pages).
void VmmSettle(halo_device* dev) {
  if (!dev->vmm_pending) return;
  dev->vmm_pending = false;
  const auto until = dev->vmm_changed + kVmmSettle;
  const auto now = std::chrono::steady_clock::now();
  if (now < until) std::this_thread::sleep_for(until - now);
}

bool InRange(const halo_buffer* b, std::size_t offset, std::size_t bytes, char* err, std::size_t errlen) {
  if (b == nullptr || b->device == nullptr) {
    SetErr(err, errlen, "null buffer");
    return false;
  }
  if (offset > b->bytes || bytes > b->bytes - offset) {
    SetErr(err, errlen, "range [%zu, %zu) outside a buffer of %zu bytes", offset, offset + bytes, b->bytes);
    return false;
  }
  return true;
}

}  // namespace

extern "C" {

int halo_device_create(int backend, halo_device** out, char* err, size_t errlen) {
  if (out == nullptr) return SetErr(err, errlen, "null out"), -1;
  *out = nullptr;
  if (backend != HALO_BACKEND_HIP) return SetErr(err, errlen, "unsupported backend %d", backend), -1;
  int n = 0;
  if (!Ok(hipGetDeviceCount(&n), "hipGetDeviceCount", err, errlen)) return -1;
  if (n == 0) return SetErr(err, errlen, "no HIP device"), -1;
  auto* dev = new halo_device();
  if (!Ok(hipSetDevice(0), "hipSetDevice", err, errlen) ||
      !Ok(hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking), "hipStreamCreate", err, errlen) ||
      !Ok(hipEventCreate(&dev->t0), "hipEventCreate", err, errlen) ||
      !Ok(hipEventCreate(&dev->t1), "hipEventCreate", err, errlen)) {
    halo_device_destroy(dev);
    return -1;
  }
  // page mapping where the device supports it (reference src/rt/hip_device.cpp:52-66)
  int vmm = 0;
  dev->prop.type = hipMemAllocationTypePinned;
  dev->prop.location.type = hipMemLocationTypeDevice;
  dev->prop.location.id = 0;
  std::size_t gran = 0;
  if (hipDeviceGetAttribute(&vmm, hipDeviceAttributeVirtualMemoryManagementSupported, 0) == hipSuccess && vmm &&
      hipMemGetAllocationGranularity(&gran, &dev->prop, hipMemAllocationGranularityMinimum) == hipSuccess &&
      gran > 0)
    dev->page_bytes = (kPageTarget + gran - 1) / gran * gran;
  (void)hipGetLastError();
  *out = dev;
  return 0;
}

int halo_device_ordinal(const halo_device* dev) { return dev ? dev->ordinal : -1; }

void halo_device_destroy(halo_device* dev) {
  if (dev == nullptr) return;
  if (dev->stream) (void)hipStreamSynchronize(dev->stream);
  if (dev->module) (void)hipModuleUnload(dev->module);
  if (dev->t0) (void)hipEventDestroy(dev->t0);
  if (dev->t1) (void)hipEventDestroy(dev->t1);
  if (dev->stream) (void)hipStreamDestroy(dev->stream);
  delete dev;
}

int halo_alloc(halo_device* dev, size_t bytes, halo_buffer* out, char* err, size_t errlen) {
  if (dev == nullptr || out == nullptr) return SetErr(err, errlen, "null argument"), -1;
  *out = halo_buffer{};
  if (!NotCapturing(dev, "Alloc", err, errlen)) return -1;
  void* p = nullptr;
  if (!Ok(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc", err, errlen)) return -1;
  out->device = p;
  out->bytes = bytes;
  return 0;
}

void halo_free(halo_device* dev, halo_buffer* buf) {
  if (buf == nullptr || buf->device == nullptr) return;
  // hipFree is not capturable (it would invalidate the capture): a free requested mid-capture is deferred.
  if (dev != nullptr && dev->capturing)
    dev->deferred_free.push_back(buf->device);
  else
    (void)hipFree(buf->device);
  *buf = halo_buffer{};
}

int halo_upload(halo_device* dev, const halo_buffer* dst, size_t offset, const void* src, size_t bytes, char* err,
                size_t errlen) {
  if (!NotCapturing(dev, "Upload", err, errlen) || !InRange(dst, offset, bytes, err, errlen)) return -1;
  VmmSettle(dev);
  if (bytes == 0) return 0;
  if (!Ok(hipMemcpyAsync(static_cast<char*>(dst->device) + offset, src, bytes, hipMemcpyHostToDevice, dev->stream),
          "hipMemcpyAsync(HtoD)", err, errlen))
    return -1;
  return Ok(hipStreamSynchronize(dev->stream), "hipStreamSynchronize", err, errlen) ? 0 : -1;
}

int halo_upload_async(halo_device* dev, const halo_buffer* dst, size_t offset, const void* src, size_t bytes,
                      char* err, size_t errlen) {
  if (!NotCapturing(dev, "UploadAsync", err, errlen) || !InRange(dst, offset, bytes, err, errlen)) return -1;
  VmmSettle(dev);
  if (bytes == 0) return 0;
  return Ok(hipMemcpyAsync(static_cast<char*>(dst->device) + offset, src, bytes, hipMemcpyHostToDevice,
                           dev->stream),
            "hipMemcpyAsync(HtoD)", err, errlen)
             ? 0
             : -1;
}

int halo_download(halo_device* dev, const halo_buffer* src, size_t offset, void* dst, size_t bytes, char* err,
                  size_t errlen) {
  if (!NotCapturing(dev, "Download", err, errlen) || !InRange(src, offset, bytes, err, errlen)) return -1;
  VmmSettle(dev);
  if (bytes == 0) return Ok(hipStreamSynchronize(dev->stream), "hipStreamSynchronize", err, errlen) ? 0 : -1;
  if (!Ok(hipMemcpyAsync(dst, static_cast<const char*>(src->device) + offset, bytes, hipMemcpyDeviceToHost,
                         dev->stream),
          "hipMemcpyAsync(DtoH)", err, errlen))
    return -1;
  return Ok(hipStreamSynchronize(dev->stream), "hipStreamSynchronize", err, errlen) ? 0 : -1;
}

int halo_fill(halo_device* dev, const halo_buffer* dst, uint8_t value, char* err, size_t errlen) {
  // Memset nodes are kept out of captured graphs: fills run eagerly only.
  if (!NotCapturing(dev, "Fill", err, errlen) || !InRange(dst, 0, dst ? dst->bytes : 0, err, errlen)) return -1;
  VmmSettle(dev);
  return Ok(hipMemsetAsync(dst->device, value, dst->bytes, dev->stream), "hipMemsetAsync", err, errlen) ? 0 : -1;
}

void* halo_alloc_host(halo_device* dev, size_t bytes, char* err, size_t errlen) {
  (void)dev;
  void* p = nullptr;
  if (!Ok(hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc", err, errlen)) return nullptr;
  return p;
}

void halo_free_host(halo_device* dev, void* p) {
  (void)dev;
  if (p) (void)hipHostFree(p);
}

size_t halo_available_bytes(halo_device* dev) {
  (void)dev;
  std::size_t free_b = 0, total = 0;
  if (hipMemGetInfo(&free_b, &total) != hipSuccess) return SIZE_MAX;
  return free_b;
}

int halo_code_object_mach(const uint8_t* code, size_t bytes) {
  // ELF64 little-endian header: magic, class 2, data 1; e_machine (offset 18) EM_AMDGPU = 224; e_flags at 48
  if (code == nullptr || bytes < 64 || std::memcmp(code, "\x7f" "ELF", 4) != 0 || code[4] != 2 || code[5] != 1)
    return -1;
  const unsigned machine = code[18] | (code[19] << 8);
  if (machine != 224) return -1;
  return code[48];
}

int halo_load_module(halo_device* dev, const uint8_t* code, size_t bytes, char* err, size_t errlen) {
  if (dev == nullptr || code == nullptr || bytes == 0) return SetErr(err, errlen, "empty code object"), -1;
  if (dev->module) return SetErr(err, errlen, "a module is already loaded"), -1;
  dev->image.assign(code, code + bytes);
  return Ok(hipModuleLoadData(&dev->module, dev->image.data()), "hipModuleLoadData", err, errlen) ? 0 : -1;
}

halo_kernel_id halo_kernel(halo_device* dev, const char* name, char* err, size_t errlen) {
  if (dev == nullptr || dev->module == nullptr) return SetErr(err, errlen, "no module loaded"), -1;
  for (std::size_t i = 0; i < dev->names.size(); ++i)
    if (dev->names[i] == name) return static_cast<halo_kernel_id>(i);
  hipFunction_t f = nullptr;
  if (!Ok(hipModuleGetFunction(&f, dev->module, name), name, err, errlen)) return -1;
  dev->functions.push_back(f);
  dev->names.emplace_back(name);
  return static_cast<halo_kernel_id>(dev->functions.size() - 1);
}

int halo_launch(halo_device* dev, halo_kernel_id kernel, halo_dim3 grid, halo_dim3 block, const halo_arg* args,
                size_t nargs, char* err, size_t errlen) {
  if (dev == nullptr || kernel < 0 || static_cast<std::size_t>(kernel) >= dev->functions.size())
    return SetErr(err, errlen, "bad kernel id %d", kernel), -1;
  if (grid.x == 0 || grid.y == 0 || grid.z == 0 || block.x == 0 || block.y == 0 || block.z == 0 ||
      block.x * block.y * block.z > 1024)
    return SetErr(err, errlen, "bad launch shape (%u,%u,%u)x(%u,%u,%u) for %s", grid.x, grid.y, grid.z, block.x,
                  block.y, block.z, dev->names[kernel].c_str()),
           -1;
  std::uint64_t storage[32];
  void* params[32];
  if (nargs > 32) return SetErr(err, errlen, "too many kernel arguments"), -1;
  if (nargs > 0 && args == nullptr) return SetErr(err, errlen, "null argument list"), -1;
  VmmSettle(dev);
  for (std::size_t i = 0; i < nargs; ++i) {
    storage[i] = 0;
    if (args[i].kind == HALO_ARG_BUFFER) {
      if (args[i].buffer.device == nullptr && args[i].offset != 0)
        return SetErr(err, errlen, "argument %zu of %s: offset %zu into a null buffer", i, dev->names[kernel].c_str(),
                      args[i].offset),
               -1;
      void* p = args[i].buffer.device ? static_cast<char*>(args[i].buffer.device) + args[i].offset : nullptr;
      std::memcpy(&storage[i], &p, sizeof(p));
    } else {
      if (args[i].size == 0 || args[i].size > 8) return SetErr(err, errlen, "bad scalar size"), -1;
      std::memcpy(&storage[i], args[i].bytes, args[i].size);
    }
    params[i] = &storage[i];
  }
  if (dev->capturing) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(dev->stream, &st) == hipSuccess && st != hipStreamCaptureStatusActive)
      return SetErr(err, errlen, "capture is no longer active (status %d) before launch %zu (%s)", static_cast<int>(st),
                    dev->captured, dev->names[kernel].c_str()),
             -1;
  }
  const bool timing = dev->profiling && !dev->capturing;
  halo_device::Timed tm{kernel, nullptr, nullptr};
  if (timing) {
    (void)hipEventCreate(&tm.a);
    (void)hipEventCreate(&tm.b);
    (void)hipEventRecord(tm.a, dev->stream);
  }
  if (!Ok(hipModuleLaunchKernel(dev->functions[kernel], grid.x, grid.y, grid.z, block.x, block.y, block.z, 0,
                                dev->stream, params, nullptr),
          "hipModuleLaunchKernel", err, errlen)) {
    std::string m = err ? std::string(err) : std::string();
    SetErr(err, errlen, "%s (launching %s, launch %zu of the capture)", m.c_str(), dev->names[kernel].c_str(),
           dev->captured);
    return -1;
  }
  if (dev->capturing) ++dev->captured;
  if (timing) {
    (void)hipEventRecord(tm.b, dev->stream);
    dev->timed.push_back(tm);
  }
  return 0;
}

int halo_synchronize(halo_device* dev, char* err, size_t errlen) {
  if (!NotCapturing(dev, "Synchronize", err, errlen)) return -1;
  return Ok(hipStreamSynchronize(dev->stream), "hipStreamSynchronize", err, errlen) ? 0 : -1;
}

int halo_begin_capture(halo_device* dev, char* err, size_t errlen) {
  if (dev->capturing) return SetErr(err, errlen, "already capturing"), -1;
  // Drain all device work first (allocations and copies the runtime may still be completing on other queues), so
  // that nothing outside the capturing stream is pending when capture starts.
  if (!Ok(hipDeviceSynchronize(), "hipDeviceSynchronize", err, errlen)) return -1;
  dev->captured = 0;
  if (!Ok(hipStreamBeginCapture(dev->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture", err, errlen))
    return -1;
  dev->capturing = true;
  return 0;
}

int halo_end_capture(halo_device* dev, halo_graph* out, char* err, size_t errlen) {
  if (!dev->capturing) return SetErr(err, errlen, "not capturing"), -1;
  dev->capturing = false;
  hipGraph_t g = nullptr;
  const hipError_t end = hipStreamEndCapture(dev->stream, &g);
  for (void* p : dev->deferred_free) (void)hipFree(p);
  dev->deferred_free.clear();
  for (const auto& r : dev->deferred_ranges) (void)hipMemAddressFree(r.first, r.second);
  dev->deferred_ranges.clear();
  if (!Ok(end, "hipStreamEndCapture", err, errlen)) return -1;
  hipGraphExec_t exec = nullptr;
  const bool ok = Ok(hipGraphInstantiate(&exec, g, nullptr, nullptr, 0), "hipGraphInstantiate", err, errlen);
  (void)hipGraphDestroy(g);
  if (!ok) return -1;
  out->exec = exec;
  return 0;
}

int halo_launch_graph(halo_device* dev, const halo_graph* graph, char* err, size_t errlen) {
  if (dev == nullptr || graph == nullptr || graph->exec == nullptr) return SetErr(err, errlen, "null graph"), -1;
  VmmSettle(dev);
  return Ok(hipGraphLaunch(static_cast<hipGraphExec_t>(graph->exec), dev->stream), "hipGraphLaunch", err, errlen)
             ? 0
             : -1;
}

void halo_free_graph(halo_device* dev, halo_graph* graph) {
  (void)dev;
  if (graph && graph->exec) (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph->exec));
  if (graph) graph->exec = nullptr;
}

// ---- page mapping (reference rt::Device PageBytes ... UnmapPage, src/rt/device.hpp:101-112;
// src/rt/hip_device.cpp:127-198) ----
size_t halo_page_bytes(halo_device* dev) { return dev ? dev->page_bytes : 0; }

int halo_reserve_range(halo_device* dev, size_t bytes, halo_buffer* out, char* err, size_t errlen) {
  if (dev == nullptr || out == nullptr) return SetErr(err, errlen, "null argument"), -1;
  *out = halo_buffer{};
  if (dev->page_bytes == 0) return SetErr(err, errlen, "page mapping: not supported by this device"), -1;
  const std::size_t n = std::max<std::size_t>((bytes + dev->page_bytes - 1) / dev->page_bytes, 1) * dev->page_bytes;
  void* p = nullptr;
  if (!Ok(hipMemAddressReserve(&p, n, 0, nullptr, 0), "hipMemAddressReserve", err, errlen)) return -1;
  out->device = p;
  out->bytes = n;
  return 0;
}

void halo_release_range(halo_device* dev, halo_buffer* range) {
  if (range == nullptr || range->device == nullptr) return;
  if (dev != nullptr && dev->capturing) {
    // no stream drain is possible mid-capture (it would invalidate the capture): the release waits for EndCapture
    dev->deferred_ranges.emplace_back(range->device, range->bytes);
    *range = halo_buffer{};
    return;
  }
  if (dev != nullptr) (void)hipStreamSynchronize(dev->stream);  // queued work may still address the range
  (void)hipMemAddressFree(range->device, range->bytes);
  if (dev != nullptr) VmmStamp(dev);
  *range = halo_buffer{};
}

int halo_create_page(halo_device* dev, void** page, char* err, size_t errlen) {
  if (dev == nullptr || page == nullptr) return SetErr(err, errlen, "null argument"), -1;
  *page = nullptr;
  if (dev->page_bytes == 0) return SetErr(err, errlen, "page mapping: not supported by this device"), -1;
  hipMemGenericAllocationHandle_t h{};
  if (!Ok(hipMemCreate(&h, dev->page_bytes, &dev->prop, 0), "hipMemCreate", err, errlen)) return -1;
  *page = reinterpret_cast<void*>(h);
  return 0;
}

void halo_release_page(halo_device* dev, void* page) {
  (void)dev;
  if (page != nullptr) (void)hipMemRelease(reinterpret_cast<hipMemGenericAllocationHandle_t>(page));
}

int halo_map_page(halo_device* dev, const halo_buffer* range, size_t offset, void* page, char* err, size_t errlen) {
  if (dev == nullptr || range == nullptr || range->device == nullptr || page == nullptr)
    return SetErr(err, errlen, "null argument"), -1;
  if (!NotCapturing(dev, "MapPage", err, errlen)) return -1;
  if (dev->page_bytes == 0 || offset % dev->page_bytes != 0 || offset + dev->page_bytes > range->bytes)
    return SetErr(err, errlen, "map: offset %zu is not a page of a %zu-byte range", offset, range->bytes), -1;
  void* at = static_cast<char*>(range->device) + offset;
  hipMemAccessDesc acc{};
  acc.location = dev->prop.location;
  acc.flags = hipMemAccessFlagsProtReadWrite;
  if (!Ok(hipMemMap(at, dev->page_bytes, 0, reinterpret_cast<hipMemGenericAllocationHandle_t>(page), 0), "hipMemMap",
          err, errlen))
    return -1;
  const bool ok = Ok(hipMemSetAccess(at, dev->page_bytes, &acc, 1), "hipMemSetAccess", err, errlen);
  if (!ok) (void)hipMemUnmap(at, dev->page_bytes);  // a failed map leaves the range as it was
  VmmStamp(dev);
  return ok ? 0 : -1;
}

int halo_unmap_page(halo_device* dev, const halo_buffer* range, size_t offset, char* err, size_t errlen) {
  if (dev == nullptr || range == nullptr || range->device == nullptr) return SetErr(err, errlen, "null argument"), -1;
  if (!NotCapturing(dev, "UnmapPage", err, errlen)) return -1;
  if (dev->page_bytes == 0 || offset % dev->page_bytes != 0 || offset + dev->page_bytes > range->bytes)
    return SetErr(err, errlen, "unmap: offset %zu is not a page of a %zu-byte range", offset, range->bytes), -1;
  // work queued on the stream may still read the page: drain it first
  const bool ok = Ok(hipStreamSynchronize(dev->stream), "hipStreamSynchronize", err, errlen) &&
                  Ok(hipMemUnmap(static_cast<char*>(range->device) + offset, dev->page_bytes), "hipMemUnmap", err,
                     errlen);
  VmmStamp(dev);
  return ok ? 0 : -1;
}

// ---- module-scope variables (reference rt::Device ReadGlobal / WriteGlobal, src/rt/device.hpp:122-126;
// src/rt/hip_device.cpp:231-249) ----
namespace {
int Global(halo_device* dev, const char* name, size_t bytes, void** p, char* err, size_t errlen) {
  if (dev == nullptr || dev->module == nullptr || name == nullptr) return SetErr(err, errlen, "no module loaded"), -1;
  hipDeviceptr_t dp = nullptr;
  std::size_t size = 0;
  if (!Ok(hipModuleGetGlobal(&dp, &size, dev->module, name), name, err, errlen)) return -1;
  if (bytes > size) return SetErr(err, errlen, "%s has %zu bytes, %zu requested", name, size, bytes), -1;
  *p = reinterpret_cast<void*>(dp);
  return 0;
}
}  // namespace

int halo_read_global(halo_device* dev, const char* name, void* dst, size_t bytes, char* err, size_t errlen) {
  void* p = nullptr;
  if (!NotCapturing(dev, "ReadGlobal", err, errlen) || Global(dev, name, bytes, &p, err, errlen) != 0) return -1;
  VmmSettle(dev);
  return Ok(hipMemcpyAsync(dst, p, bytes, hipMemcpyDeviceToHost, dev->stream), "hipMemcpyAsync(DtoH)", err,
            errlen) &&
                 Ok(hipStreamSynchronize(dev->stream), "hipStreamSynchronize", err, errlen)
             ? 0
             : -1;
}

int halo_write_global(halo_device* dev, const char* name, const void* src, size_t bytes, char* err, size_t errlen) {
  void* p = nullptr;
  if (!NotCapturing(dev, "WriteGlobal", err, errlen) || Global(dev, name, bytes, &p, err, errlen) != 0) return -1;
  VmmSettle(dev);
  return Ok(hipMemcpyAsync(p, src, bytes, hipMemcpyHostToDevice, dev->stream), "hipMemcpyAsync(HtoD)", err,
            errlen) &&
                 Ok(hipStreamSynchronize(dev->stream), "hipStreamSynchronize", err, errlen)
             ? 0
             : -1;
}

int halo_timer_start(halo_device* dev, char* err, size_t errlen) {
  return Ok(hipEventRecord(dev->t0, dev->stream), "hipEventRecord", err, errlen) ? 0 : -1;
}

int halo_timer_stop(halo_device* dev, float* ms, char* err, size_t errlen) {
  if (!Ok(hipEventRecord(dev->t1, dev->stream), "hipEventRecord", err, errlen) ||
      !Ok(hipEventSynchronize(dev->t1), "hipEventSynchronize", err, errlen))
    return -1;
  return Ok(hipEventElapsedTime(ms, dev->t0, dev->t1), "hipEventElapsedTime", err, errlen) ? 0 : -1;
}

int halo_wall_clock_khz(halo_device* dev, int* khz, char* err, size_t errlen) {
  if (dev == nullptr || khz == nullptr) return SetErr(err, errlen, "null argument"), -1;
  return Ok(hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev->ordinal), "hipDeviceGetAttribute", err,
            errlen)
             ? 0
             : -1;
}

void* halo_device_stream(halo_device* dev) { return dev ? static_cast<void*>(dev->stream) : nullptr; }

int halo_profile_begin(halo_device* dev, char* err, size_t errlen) {
  if (dev == nullptr) return SetErr(err, errlen, "null device"), -1;
  dev->profiling = true;
  return 0;
}

int halo_profile_end(halo_device* dev, char* report, size_t len, char* err, size_t errlen) {
  if (dev == nullptr) return SetErr(err, errlen, "null device"), -1;
  dev->profiling = false;
  if (!Ok(hipStreamSynchronize(dev->stream), "hipStreamSynchronize", err, errlen)) return -1;
  std::vector<double> total(dev->functions.size(), 0.0);
  std::vector<std::size_t> count(dev->functions.size(), 0);
  for (const auto& t : dev->timed) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, t.a, t.b) == hipSuccess) {
      total[t.k] += ms;
      ++count[t.k];
    }
    (void)hipEventDestroy(t.a);
    (void)hipEventDestroy(t.b);
  }
  dev->timed.clear();
  std::string out;
  for (std::size_t i = 0; i < total.size(); ++i)
    if (count[i]) {
      char line[256];
      std::snprintf(line, sizeof line, "%s %zu %.3f\n", dev->names[i].c_str(), count[i], total[i] * 1e3);
      out += line;
    }
  if (report && len) {
    std::snprintf(report, len, "%s", out.c_str());
  }
  return 0;
}

}  // extern "C"
