// The reference-side device adapter: an rt::Device (reference src/rt/device.hpp:77-137) that forwards every member
// to this library's C ABI (include/halo_rt.h). A maintainer adds this file to the reference as
// src/rt/amd_device.cpp, gives Device::Create (src/rt/device.cpp) a branch that calls CreateAmdDevice, and links
// -lhalo_flash_amd. FlashNextGpu::Init's LoadModule(kernels::CoreHsaco()) (src/engine/flash_next_gpu.cpp:273) needs no
// edit: handed a code object for another target, LoadModule loads halo_core_code_object() instead. tests/test_integration_adapter.py compiles it against the reference's
// device.hpp.
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "rt/device.hpp"

extern "C" {
#include "halo_rt.h"
}

namespace halo::rt {
namespace {

constexpr std::size_t kErr = 512;

bool Check(int rc, const char* err, std::string* error) {
  if (rc != 0 && error != nullptr) *error = err;
  return rc == 0;
}
halo_buffer Raw(const Buffer& b) { return halo_buffer{b.device, b.bytes, b.handle}; }
Buffer Wrap(const halo_buffer& b) { return Buffer{b.device, b.bytes, b.handle}; }

class AmdDevice final : public Device {
 public:
  explicit AmdDevice(halo_device* d) : d_(d) {}
  ~AmdDevice() override { halo_device_destroy(d_); }

  Backend backend() const noexcept override { return Backend::kHip; }

  Buffer Alloc(std::size_t bytes, std::string* error) override {
    halo_buffer b{};
    char e[kErr];
    return Check(halo_alloc(d_, bytes, &b, e, kErr), e, error) ? Wrap(b) : Buffer{};
  }
  void Free(Buffer& buffer) noexcept override {
    halo_buffer b = Raw(buffer);
    halo_free(d_, &b);
    buffer = {};
  }
  bool Upload(const Buffer& dst, std::size_t off, const void* src, std::size_t n, std::string* error) override {
    const halo_buffer b = Raw(dst);
    char e[kErr];
    return Check(halo_upload(d_, &b, off, src, n, e, kErr), e, error);
  }
  bool UploadAsync(const Buffer& dst, std::size_t off, const void* src, std::size_t n, std::string* error) override {
    const halo_buffer b = Raw(dst);
    char e[kErr];
    return Check(halo_upload_async(d_, &b, off, src, n, e, kErr), e, error);
  }
  bool Download(const Buffer& src, std::size_t off, void* dst, std::size_t n, std::string* error) override {
    const halo_buffer b = Raw(src);
    char e[kErr];
    return Check(halo_download(d_, &b, off, dst, n, e, kErr), e, error);
  }
  bool Fill(const Buffer& dst, std::uint8_t v, std::string* error) override {
    const halo_buffer b = Raw(dst);
    char e[kErr];
    return Check(halo_fill(d_, &b, v, e, kErr), e, error);
  }
  void* AllocHost(std::size_t bytes, std::string* error) override {
    char e[kErr];
    void* p = halo_alloc_host(d_, bytes, e, kErr);
    if (p == nullptr && error != nullptr) *error = e;
    return p;
  }
  void FreeHost(void* p) noexcept override { halo_free_host(d_, p); }

  // page mapping (P6 KV paging)
  std::size_t PageBytes() const noexcept override { return halo_page_bytes(d_); }
  Buffer ReserveRange(std::size_t bytes, std::string* error) override {
    halo_buffer b{};
    char e[kErr];
    return Check(halo_reserve_range(d_, bytes, &b, e, kErr), e, error) ? Wrap(b) : Buffer{};
  }
  void ReleaseRange(Buffer& range) noexcept override {
    halo_buffer b = Raw(range);
    halo_release_range(d_, &b);
    range = {};
  }
  void* CreatePage(std::string* error) override {
    void* page = nullptr;
    char e[kErr];
    return Check(halo_create_page(d_, &page, e, kErr), e, error) ? page : nullptr;
  }
  void ReleasePage(void* page) noexcept override { halo_release_page(d_, page); }
  bool MapPage(const Buffer& range, std::size_t offset, void* page, std::string* error) override {
    const halo_buffer b = Raw(range);
    char e[kErr];
    return Check(halo_map_page(d_, &b, offset, page, e, kErr), e, error);
  }
  bool UnmapPage(const Buffer& range, std::size_t offset, std::string* error) override {
    const halo_buffer b = Raw(range);
    char e[kErr];
    return Check(halo_unmap_page(d_, &b, offset, e, kErr), e, error);
  }
  std::size_t AvailableBytes() const override { return halo_available_bytes(d_); }

  bool LoadModule(std::span<const std::uint8_t> code, std::string* error) override {
    char e[kErr];
    const std::uint8_t* data = code.data();
    std::size_t bytes = code.size();
    // another target's code object (the engine's gfx1151 CoreHsaco): the library's own gfx950 object, which holds
    // the same kernel names and parameter lists, is loaded instead
    if (halo_code_object_mach(data, bytes) != HALO_MACH_GFX950) data = halo_core_code_object(&bytes);
    return Check(halo_load_module(d_, data, bytes, e, kErr), e, error);
  }
  KernelId Kernel(std::string_view name, std::string* error) override {
    char e[kErr];
    const KernelId id = halo_kernel(d_, std::string(name).c_str(), e, kErr);
    if (id < 0 && error != nullptr) *error = e;
    return id;
  }
  bool ReadGlobal(std::string_view name, void* dst, std::size_t bytes, std::string* error) override {
    char e[kErr];
    return Check(halo_read_global(d_, std::string(name).c_str(), dst, bytes, e, kErr), e, error);
  }
  bool WriteGlobal(std::string_view name, const void* src, std::size_t bytes, std::string* error) override {
    char e[kErr];
    return Check(halo_write_global(d_, std::string(name).c_str(), src, bytes, e, kErr), e, error);
  }
  bool Launch(KernelId k, Dim3 grid, Dim3 block, std::span<const Arg> args, std::string* error) override {
    std::vector<halo_arg> a(args.size());
    for (std::size_t i = 0; i < args.size(); ++i) {
      a[i].kind = args[i].kind == Arg::Kind::kBuffer ? HALO_ARG_BUFFER : HALO_ARG_SCALAR;
      a[i].size = args[i].size;
      a[i].buffer = Raw(args[i].buffer);
      a[i].offset = args[i].offset;
      std::memcpy(a[i].bytes, args[i].bytes, sizeof a[i].bytes);
    }
    char e[kErr];
    return Check(halo_launch(d_, k, halo_dim3{grid.x, grid.y, grid.z}, halo_dim3{block.x, block.y, block.z},
                             a.data(), a.size(), e, kErr),
                 e, error);
  }
  bool Synchronize(std::string* error) override {
    char e[kErr];
    return Check(halo_synchronize(d_, e, kErr), e, error);
  }
  bool BeginCapture(std::string* error) override {
    char e[kErr];
    return Check(halo_begin_capture(d_, e, kErr), e, error);
  }
  bool EndCapture(Graph* out, std::string* error) override {
    halo_graph g{};
    char e[kErr];
    if (!Check(halo_end_capture(d_, &g, e, kErr), e, error)) return false;
    out->exec = g.exec;
    return true;
  }
  bool LaunchGraph(const Graph& graph, std::string* error) override {
    const halo_graph g{graph.exec};
    char e[kErr];
    return Check(halo_launch_graph(d_, &g, e, kErr), e, error);
  }
  void FreeGraph(Graph& graph) noexcept override {
    halo_graph g{graph.exec};
    halo_free_graph(d_, &g);
    graph = {};
  }

 private:
  halo_device* d_;
};

}  // namespace

std::unique_ptr<Device> CreateAmdDevice(std::string* error) {
  halo_device* d = nullptr;
  char e[kErr];
  if (halo_device_create(HALO_BACKEND_HIP, &d, e, kErr) != 0) {
    if (error != nullptr) *error = e;
    return nullptr;
  }
  return std::make_unique<AmdDevice>(d);
}

}  // namespace halo::rt
