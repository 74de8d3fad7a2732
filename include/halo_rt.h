/* halo-flash MI355X device layer: the C ABI the reference's engine reaches the GPU through.
 *
 * Each entry point replaces one member of the reference's device interface `halo::rt::Device`
 * (src/rt/device.hpp:77-137), implemented for ROCm/HIP on gfx950 in halo-flash_amd/csrc/rt/hip_device.cpp.
 * Plain C: pointers, sizes, PODs. Functions return 0 on success and -1 on failure with a NUL-terminated message
 * in err (truncated to errlen; err may be NULL), the convention of the reference's include/halo_variant.h:12-13.
 *
 * The kernels are a gfx950 code object embedded in the library (halo_core_code_object), loaded with
 * halo_load_module and looked up by their extern "C" names: the reference's names and parameter lists for the
 * hot-path subset (src/kernels/core.hip, src/kernels/batch_decode.hip) plus new MI355X kernels; halo_kernels.h
 * lists them.
 *
 * Threading (reference src/rt/hip_device.cpp:50, 282): one non-blocking stream per device, stream capture in
 * thread-local mode. A device is used by one thread at a time. */
#ifndef HALO_RT_H_
#define HALO_RT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct halo_device halo_device;

/* Device memory: `device` is the address kernels see (reference rt::Buffer, src/rt/device.hpp:28-33). */
typedef struct halo_buffer {
  void* device;
  size_t bytes;
  void* handle;
} halo_buffer;

/* A kernel argument: a buffer (+ byte offset) or a by-value scalar of at most 8 bytes
 * (reference rt::Arg, src/rt/device.hpp:35-59). */
enum { HALO_ARG_BUFFER = 0, HALO_ARG_SCALAR = 1 };
typedef struct halo_arg {
  uint8_t kind;
  uint8_t size;   /* scalar bytes (1, 2, 4 or 8) */
  uint8_t pad[6];
  halo_buffer buffer;
  size_t offset;  /* buffer byte offset */
  uint8_t bytes[8];
} halo_arg;

typedef struct halo_dim3 {
  uint32_t x, y, z;
} halo_dim3;

/* A replayable launch sequence recorded by stream capture (reference rt::Graph, src/rt/device.hpp:68-75). */
typedef struct halo_graph {
  void* exec;
} halo_graph;

typedef int32_t halo_kernel_id; /* -1 on error (reference rt::KernelId) */

enum { HALO_BACKEND_HIP = 0 };

/* Device::Create (src/rt/device.hpp:80). Uses HIP device 0 and one non-blocking stream. */
int halo_device_create(int backend, halo_device** out, char* err, size_t errlen);
void halo_device_destroy(halo_device* dev);
/* The HIP device ordinal the device's stream belongs to (no counterpart in the reference, whose Device hides it);
 * -1 for a null device. Code that resolves per-device addresses (hipGetSymbolAddress) selects this device first. */
int halo_device_ordinal(const halo_device* dev);

/* Device::Alloc / Free (src/rt/device.hpp:83-84). */
int halo_alloc(halo_device* dev, size_t bytes, halo_buffer* out, char* err, size_t errlen);
void halo_free(halo_device* dev, halo_buffer* buf);

/* Device::Upload / Download / UploadAsync / Fill (src/rt/device.hpp:85-95). Upload and Download are ordered on the
 * device stream and complete before returning; UploadAsync's source must stay unchanged until the next
 * halo_synchronize or halo_download. */
int halo_upload(halo_device* dev, const halo_buffer* dst, size_t offset, const void* src, size_t bytes, char* err,
                size_t errlen);
int halo_upload_async(halo_device* dev, const halo_buffer* dst, size_t offset, const void* src, size_t bytes,
                      char* err, size_t errlen);
int halo_download(halo_device* dev, const halo_buffer* src, size_t offset, void* dst, size_t bytes, char* err,
                  size_t errlen);
int halo_fill(halo_device* dev, const halo_buffer* dst, uint8_t value, char* err, size_t errlen);

/* Device::AllocHost / FreeHost (src/rt/device.hpp:96-99): pinned host memory. */
void* halo_alloc_host(halo_device* dev, size_t bytes, char* err, size_t errlen);
void halo_free_host(halo_device* dev, void* p);

/* Device::AvailableBytes (src/rt/device.hpp:114-118). */
size_t halo_available_bytes(halo_device* dev);

/* Physical pages mapped into reserved virtual ranges, for paged KV caches (Device::PageBytes / ReserveRange /
 * ReleaseRange / CreatePage / ReleasePage / MapPage / UnmapPage, src/rt/device.hpp:101-112). halo_page_bytes is
 * the mapping granularity (2 MiB rounded to the device's granule), 0 when the device cannot map pages (callers
 * then allocate whole ranges with halo_alloc). A reserved range has device addresses but no memory until pages are
 * mapped into it; one page may be mapped into several ranges (offsets multiples of halo_page_bytes) and is read
 * and written through any of them. Unmapping and releasing a range drain the device stream first; the first launch
 * or copy after a mapping change waits out a 1 ms settle interval (as the reference's HIP backend does). Not
 * capturable: map / unmap refuse during capture, and a range released during capture is freed at halo_end_capture.
 * A map whose access grant fails is undone (the range is left unmapped at that offset). */
size_t halo_page_bytes(halo_device* dev);
int halo_reserve_range(halo_device* dev, size_t bytes, halo_buffer* out, char* err, size_t errlen);
void halo_release_range(halo_device* dev, halo_buffer* range);
int halo_create_page(halo_device* dev, void** page, char* err, size_t errlen);
void halo_release_page(halo_device* dev, void* page);
int halo_map_page(halo_device* dev, const halo_buffer* range, size_t offset, void* page, char* err, size_t errlen);
int halo_unmap_page(halo_device* dev, const halo_buffer* range, size_t offset, char* err, size_t errlen);

/* Device::ReadGlobal / WriteGlobal (src/rt/device.hpp:122-126): copies a module-scope __device__ variable of the
 * loaded code object to or from the host (bytes <= the variable's size). Not capturable. */
int halo_read_global(halo_device* dev, const char* name, void* dst, size_t bytes, char* err, size_t errlen);
int halo_write_global(halo_device* dev, const char* name, const void* src, size_t bytes, char* err, size_t errlen);

/* kernels::CoreHsaco() (reference CMakeLists.txt:143-179): the embedded gfx950 code object. */
const uint8_t* halo_core_code_object(size_t* bytes);
/* The processor a code object targets: EF_AMDGPU_MACH of an AMDGPU ELF64 object (e_flags & 0xff; gfx950 is
 * HALO_MACH_GFX950), -1 when the bytes are not one. Lets a loader that is handed another target's code object (the
 * reference engine passes its gfx1151 CoreHsaco) load the embedded one instead. No counterpart in the reference. */
enum { HALO_MACH_GFX950 = 0x4f };
int halo_code_object_mach(const uint8_t* code, size_t bytes);

/* Device::LoadModule / Kernel (src/rt/device.hpp:120-121). */
int halo_load_module(halo_device* dev, const uint8_t* code, size_t bytes, char* err, size_t errlen);
halo_kernel_id halo_kernel(halo_device* dev, const char* name, char* err, size_t errlen);

/* Device::Launch / Synchronize (src/rt/device.hpp:128-130): kernargs in declaration order. */
int halo_launch(halo_device* dev, halo_kernel_id kernel, halo_dim3 grid, halo_dim3 block, const halo_arg* args,
                size_t nargs, char* err, size_t errlen);
int halo_synchronize(halo_device* dev, char* err, size_t errlen);

/* Device::BeginCapture / EndCapture / LaunchGraph / FreeGraph (src/rt/device.hpp:132-136). Uploads, downloads,
 * fills and synchronize fail while capturing. */
int halo_begin_capture(halo_device* dev, char* err, size_t errlen);
int halo_end_capture(halo_device* dev, halo_graph* out, char* err, size_t errlen);
int halo_launch_graph(halo_device* dev, const halo_graph* graph, char* err, size_t errlen);
void halo_free_graph(halo_device* dev, halo_graph* graph);

/* Stream-ordered timing (no counterpart in rt::Device; the reference times with a timestamp kernel,
 * src/engine/flash_next_gpu.cpp:160-210). halo_timer_start records an event on the device stream;
 * halo_timer_stop records another, waits for it and returns the elapsed milliseconds. */
int halo_timer_start(halo_device* dev, char* err, size_t errlen);
int halo_timer_stop(halo_device* dev, float* ms, char* err, size_t errlen);
/* Frequency of the device's constant wall clock (the counter kernels read with wall_clock64, e.g. halo_clock_stamp),
 * in kHz. No counterpart in the reference. */
int halo_wall_clock_khz(halo_device* dev, int* khz, char* err, size_t errlen);

/* The raw HIP stream (hipStream_t) of the device, for callers that interoperate with other HIP code. */
void* halo_device_stream(halo_device* dev);

/* Per-launch timing of eager launches (the reference's StartKernelTiming / StopKernelTiming,
 * src/engine/flash_next_gpu.cpp:160-210): between begin and end every non-captured launch is bracketed by events;
 * end synchronizes and writes one line per kernel, "name launches total_microseconds", into report. */
int halo_profile_begin(halo_device* dev, char* err, size_t errlen);
int halo_profile_end(halo_device* dev, char* report, size_t len, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif

#endif /* HALO_RT_H_ */
