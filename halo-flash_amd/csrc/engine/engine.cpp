// halo_engine: code-object load, kernel lookup and the Q8_0 projection dispatch.
//
// Reference: FlashNextGpu::Init (src/engine/flash_next_gpu.cpp:256-327) loads the code object and repacks Q8_0
// weights; FlashNextGpu::MatVec (212-254) picks the GEMV variant and grid per matrix.
#include "engine.hpp"

#include <elf.h>

#include <vector>

using namespace halo::engine;

namespace {

// Names of every kernel in an AMDGPU code object: the symbols with a ".kd" (kernel descriptor) suffix.
std::vector<std::string> KernelNames(const std::uint8_t* code, std::size_t bytes) {
  std::vector<std::string> out;
  if (bytes < sizeof(Elf64_Ehdr)) return out;
  Elf64_Ehdr eh;
  std::memcpy(&eh, code, sizeof eh);
  if (std::memcmp(eh.e_ident, ELFMAG, SELFMAG) != 0 || eh.e_shoff == 0) return out;
  for (unsigned i = 0; i < eh.e_shnum; ++i) {
    Elf64_Shdr sh;
    std::memcpy(&sh, code + eh.e_shoff + i * sizeof(Elf64_Shdr), sizeof sh);
    if (sh.sh_type != SHT_SYMTAB && sh.sh_type != SHT_DYNSYM) continue;
    Elf64_Shdr strh;
    std::memcpy(&strh, code + eh.e_shoff + sh.sh_link * sizeof(Elf64_Shdr), sizeof strh);
    const char* strtab = reinterpret_cast<const char*>(code + strh.sh_offset);
    for (std::size_t off = 0; off + sizeof(Elf64_Sym) <= sh.sh_size; off += sizeof(Elf64_Sym)) {
      Elf64_Sym sym;
      std::memcpy(&sym, code + sh.sh_offset + off, sizeof sym);
      std::string name(strtab + sym.st_name);
      if (name.size() > 3 && name.compare(name.size() - 3, 3, ".kd") == 0) {
        name.resize(name.size() - 3);
        bool seen = false;
        for (const auto& n : out) seen = seen || n == name;
        if (!seen) out.push_back(name);
      }
    }
  }
  return out;
}

}  // namespace

extern "C" {

int halo_engine_create(halo_device* dev, halo_engine** out, char* err, size_t errlen) {
  if (dev == nullptr || out == nullptr) return SetErr(err, errlen, "null argument"), -1;
  *out = nullptr;
  std::size_t bytes = 0;
  const std::uint8_t* code = halo_core_code_object(&bytes);
  if (halo_load_module(dev, code, bytes, err, errlen) != 0) return -1;
  auto* eng = new halo_engine();
  eng->dev = dev;
  // Resolve every kernel now: lookups are not allowed while a graph is being captured.
  for (const auto& name : KernelNames(code, bytes)) {
    const halo_kernel_id id = halo_kernel(dev, name.c_str(), err, errlen);
    if (id < 0) {
      delete eng;
      return -1;
    }
    eng->ids.emplace(name, id);
  }
  if (eng->ids.empty()) {
    delete eng;
    return SetErr(err, errlen, "the code object lists no kernels"), -1;
  }
  if (halo_alloc(dev, kSyncSlots * sizeof(std::uint32_t), &eng->sync, err, errlen) != 0 ||
      halo_fill(dev, &eng->sync, 0, err, errlen) != 0 || halo_synchronize(dev, err, errlen) != 0) {
    if (eng->sync.device != nullptr) halo_free(dev, &eng->sync);
    delete eng;
    return -1;
  }
  *out = eng;
  return 0;
}

void halo_engine_destroy(halo_engine* eng) {
  if (eng == nullptr) return;
  if (eng->sync.device != nullptr) {
    (void)halo_synchronize(eng->dev, nullptr, 0);
    halo_free(eng->dev, &eng->sync);
  }
  delete eng;
}

halo_device* halo_engine_device(halo_engine* eng) { return eng ? eng->dev : nullptr; }

int halo_engine_launch(halo_engine* eng, const char* kernel, halo_dim3 grid, halo_dim3 block, const halo_arg* args,
                       size_t nargs, char* err, size_t errlen) {
  if (eng == nullptr) return SetErr(err, errlen, "null engine"), -1;
  auto it = eng->ids.find(kernel);
  halo_kernel_id id;
  if (it == eng->ids.end()) {
    id = halo_kernel(eng->dev, kernel, err, errlen);
    if (id < 0) return -1;
    eng->ids.emplace(kernel, id);
  } else {
    id = it->second;
  }
  return halo_launch(eng->dev, id, grid, block, args, nargs, err, errlen);
}

int halo_op_repack_q8_0(halo_engine* eng, const void* raw, int8_t* qs, uint16_t* d, uint32_t rows, uint32_t cols,
                        uint32_t qstride, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "repack_q8_0", {{"raw", raw}, {"qs", qs}, {"d", d}}) != 0) return -1;
  if (cols % 32 != 0 || qstride < cols || qstride % 16 != 0)
    return SetErr(err, errlen, "repack: cols %u must be a multiple of 32, qstride %u >= cols and a multiple of 16",
                  cols, qstride),
           -1;
  const std::uint64_t blocks = static_cast<std::uint64_t>(rows) * (cols / 32);
  const std::uint32_t grid = static_cast<std::uint32_t>(std::min<std::uint64_t>(CeilDiv(blocks, 256), 8192));
  const halo_arg a[] = {Ptr(raw), Ptr(qs), Ptr(d), U32(rows), U32(cols), U32(qstride)};
  return Launch(eng, "halo_repack_q8_0", D3(grid ? grid : 1), D3(256), a, err, errlen);
}

int halo_op_quantize_q8(halo_engine* eng, const float* x, int8_t* xq, float* xs, uint32_t tokens, uint32_t cols,
                        char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "quantize_q8", {{"x", x}, {"xq", xq}, {"xs", xs}}) != 0) return -1;
  if (cols % 32 != 0 || tokens == 0) return SetErr(err, errlen, "quantize: cols %% 32 != 0 or no tokens"), -1;
  const halo_arg a[] = {Ptr(x), Ptr(xq), Ptr(xs), U32(cols)};
  return Launch(eng, "halo_quantize_q8_rows", D3(tokens), D3(256), a, err, errlen);
}

int halo_op_quantize_q8_pair(halo_engine* eng, const float* x0, int8_t* xq0, float* xs0, uint32_t cols0,
                             const float* x1, int8_t* xq1, float* xs1, uint32_t cols1, uint32_t tokens, char* err,
                             size_t errlen) {
  if (RequirePtrs(err, errlen, "quantize_q8_pair",
                  {{"x0", x0}, {"xq0", xq0}, {"xs0", xs0}, {"x1", x1}, {"xq1", xq1}, {"xs1", xs1}}) != 0)
    return -1;
  if (cols0 % 32 != 0 || cols1 % 32 != 0 || tokens == 0)
    return SetErr(err, errlen, "quantize pair: cols %% 32 != 0 or no tokens"), -1;
  const halo_arg a[] = {Ptr(x0), Ptr(xq0), Ptr(xs0), U32(cols0), Ptr(x1), Ptr(xq1), Ptr(xs1), U32(cols1), U32(tokens)};
  return Launch(eng, "halo_quantize_q8_rows2", D3(2 * tokens), D3(256), a, err, errlen);
}

static int CheckMatrix(const halo_q8_matrix* w, char* err, size_t errlen) {
  if (w == nullptr || w->qs == nullptr || w->d == nullptr) return SetErr(err, errlen, "null matrix"), -1;
  if (w->rows == 0 || w->cols == 0 || w->cols % 32 != 0 || w->qstride < w->cols || w->qstride % 16 != 0)
    return SetErr(err, errlen, "bad Q8_0 matrix %ux%u qstride %u", w->rows, w->cols, w->qstride), -1;
  return 0;
}

int halo_op_matvec_q8a8_tiled(halo_engine* eng, const halo_q8_matrix* w, const int8_t* xq, const float* xs,
                              float* y, uint32_t m, uint32_t ystride, uint32_t lpr, uint32_t rpl, uint32_t waves,
                              char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "matvec_q8a8_tiled", {{"xq", xq}, {"xs", xs}, {"y", y}}) != 0) return -1;
  if (CheckMatrix(w, err, errlen) != 0) return -1;
  if (!(m == 1 || m == 2 || m == 4 || m == 8)) return SetErr(err, errlen, "tiled GEMV takes m in {1,2,4,8}"), -1;
  if (!(lpr == 16 || lpr == 32 || lpr == 64) || !(rpl == 1 || rpl == 2 || rpl == 4) || waves < 1 || waves > 4)
    return SetErr(err, errlen, "bad tiling lpr=%u r=%u waves=%u", lpr, rpl, waves), -1;
  if (m > 1 && ystride < w->rows) return SetErr(err, errlen, "ystride %u < rows %u", ystride, w->rows), -1;
  char name[64];
  std::snprintf(name, sizeof name, "halo_gemv_q8a8_l%u_r%u_b%u", lpr, rpl, m);
  const std::uint32_t rows_per_block = waves * rpl * (64 / lpr);
  const halo_arg a[] = {Ptr(w->qs), Ptr(w->d), Ptr(xq), Ptr(xs), Ptr(y),
                        U32(w->rows), U32(w->cols), U32(w->qstride), U32(m > 1 ? ystride : w->rows)};
  return Launch(eng, name, D3(CeilDiv(w->rows, rows_per_block)), D3(64 * waves), a, err, errlen);
}

int halo_op_matvec_q8a8(halo_engine* eng, const halo_q8_matrix* w, const int8_t* xq, const float* xs, float* y,
                        uint32_t m, uint32_t ystride, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "matvec_q8a8", {{"xq", xq}, {"xs", xs}, {"y", y}}) != 0) return -1;
  if (CheckMatrix(w, err, errlen) != 0) return -1;
  if (m == 0) return SetErr(err, errlen, "m == 0"), -1;
  if (m > 1 && ystride < w->rows) return SetErr(err, errlen, "ystride %u < rows %u", ystride, w->rows), -1;
  if (m >= 64 && w->rows >= 128 && w->cols % 64 == 0 &&
      static_cast<std::uint64_t>(w->rows) * w->qstride < (std::uint64_t{1} << 32)) {
    // prefill-sized M: 128 x 128 tiles staged through LDS, one 32x32x32 MFMA per Q8_0 block and tile
    const halo_arg a[] = {Ptr(w->qs), Ptr(w->d), Ptr(xq), Ptr(xs), Ptr(y), U32(w->rows), U32(w->cols),
                          U32(w->qstride), U32(m), U32(ystride)};
    return Launch(eng, "halo_gemm_q8a8_mfma32", D3(CeilDiv(w->rows, 128), CeilDiv(m, 128)), D3(512), a, err, errlen);
  }
  if (m >= 9 && m <= 16 && ystride == w->rows && w->qstride == w->cols &&
      (w->cols == 1024 || w->cols == 2048 || w->cols == 4096)) {
    // 9-16 token rows: the grouped projection's int8 matrix-core kernel (the weights streamed once, 16-byte loads)
    halo_proj_input in{};
    in.xq = xq;
    in.xs = xs;
    in.mode = HALO_PROJ_Q;
    return halo_op_proj_q8(eng, w, &y, 1, &in, m, err, errlen);
  }
  if (m >= 16) {
    // int8 MFMA tiles: 16 rows x 16 (or 64) tokens per block, one MFMA per Q8_0 block
    const std::uint32_t ys = m > 1 ? ystride : w->rows;
    const bool wide = m >= 64;
    const halo_arg a[] = {Ptr(w->qs), Ptr(w->d), Ptr(xq), Ptr(xs), Ptr(y), U32(w->rows), U32(w->cols),
                          U32(w->qstride), U32(m), U32(ys)};
    return Launch(eng, wide ? "halo_gemm_q8a8_mfma_t4" : "halo_gemm_q8a8_mfma_t1",
                  D3(CeilDiv(w->rows, 16), CeilDiv(m, wide ? 64 : 16)), D3(256), a, err, errlen);
  }
  // Up to 8 tokens, a dense output and rows of at most 2048 columns (4096 from 3 tokens up): the grouped projection
  // kernel in its quantized-input mode (one task of rows per wave, activations staged in LDS once per block). Wider
  // rows at 1-2 tokens measure faster on the per-group GEMV below, whose 64 lanes per row read the activations
  // straight from the caches; from 3 tokens on its per-lane activation loads cost more than the LDS staging
  // (2048 x 4096 at 4 tokens: 7.4 -> 5.2 us).
  if (m <= 8 && (m == 1 || ystride == w->rows) && w->qstride == w->cols &&
      (w->cols <= 2048 || (m >= 3 && w->cols <= 4096))) {
    halo_proj_input in{};
    in.xq = xq;
    in.xs = xs;
    in.mode = HALO_PROJ_Q;
    return halo_op_proj_q8(eng, w, &y, 1, &in, m, err, errlen);
  }
  if (m == 1 && (w->cols == 2048 || w->cols == 4096)) {
    // one token over 2048 / 4096 columns: one row per wave, the activation row staged in LDS once per 4-wave block
    // (bitwise the per-group GEMV's y; the 4096 x 4096 C0 GEMV 4.78 -> 4.69 us)
    const halo_arg a[] = {Ptr(w->qs), Ptr(w->d), Ptr(xq), Ptr(xs), Ptr(y),
                          U32(w->rows), U32(w->cols), U32(w->qstride), U32(w->rows)};
    return Launch(eng, "halo_gemv_q8a8s_l64_r1_b1", D3(CeilDiv(w->rows, 4)), D3(256), a, err, errlen);
  }
  // Otherwise the per-group GEMV: a row is covered by as many lanes as its 16-byte pieces allow (up to a wave);
  // more activation columns reuse each weight load over more rows per lane group.
  const std::uint32_t lpr = w->cols >= 1024 ? 64 : (w->cols >= 512 ? 32 : 16);
  std::uint32_t done = 0;
  while (done < m) {
    const std::uint32_t left = m - done;
    const std::uint32_t nb = left >= 8 ? 8 : (left >= 4 ? 4 : (left >= 2 ? 2 : 1));
    const std::uint32_t rpl = nb >= 4 ? 2 : 1;
    const std::size_t nblk = w->cols / 32;
    if (halo_op_matvec_q8a8_tiled(eng, w, xq + static_cast<std::size_t>(done) * w->cols, xs + done * nblk,
                                  y + static_cast<std::size_t>(done) * (m > 1 ? ystride : 0), nb,
                                  m > 1 ? ystride : w->rows, lpr, rpl, 4, err, errlen) != 0)
      return -1;
    done += nb;
  }
  return 0;
}

int halo_op_matvec_q8_f32x(halo_engine* eng, const halo_q8_matrix* w, const float* x, float* y, char* err,
                           size_t errlen) {
  if (RequirePtrs(err, errlen, "matvec_q8_f32x", {{"x", x}, {"y", y}}) != 0) return -1;
  if (CheckMatrix(w, err, errlen) != 0) return -1;
  const bool r4 = w->rows >= 2048;
  const halo_arg a[] = {Ptr(w->qs), Ptr(w->d), Ptr(x), Ptr(y), U32(w->rows), U32(w->cols), U32(w->qstride)};
  return Launch(eng, r4 ? "halo_gemv_q8r_r4" : "halo_gemv_q8r_r2", D3(CeilDiv(w->rows, r4 ? 32 : 16)), D3(256), a,
                err, errlen);
}

int halo_op_q8_half_dots(halo_engine* eng, const halo_q8_matrix* w, const int8_t* xq, int32_t* isum, char* err,
                         size_t errlen) {
  if (RequirePtrs(err, errlen, "q8_half_dots", {{"xq", xq}, {"isum", isum}}) != 0) return -1;
  if (CheckMatrix(w, err, errlen) != 0) return -1;
  const std::uint64_t n = static_cast<std::uint64_t>(w->rows) * (w->cols / 16);
  const halo_arg a[] = {Ptr(w->qs), Ptr(xq), Ptr(isum), U32(w->rows), U32(w->cols), U32(w->qstride)};
  return Launch(eng, "halo_q8_half_dots", D3(static_cast<std::uint32_t>(std::min<std::uint64_t>(CeilDiv(n, 256), 8192))),
                D3(256), a, err, errlen);
}

int halo_op_synth_q8(halo_engine* eng, int8_t* qs, uint16_t* d, uint32_t rows, uint32_t cols, uint32_t qstride,
                     uint64_t seed, float sigma, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "synth_q8", {{"qs", qs}, {"d", d}}) != 0) return -1;
  if (cols % 32 != 0 || qstride < cols || qstride % 16 != 0) return SetErr(err, errlen, "synth: bad shape"), -1;
  const std::uint64_t n = static_cast<std::uint64_t>(rows) * (cols / 16);
  const halo_arg a[] = {Ptr(qs), Ptr(d), U32(rows), U32(cols), U32(qstride), Val(seed), Val(sigma)};
  return Launch(eng, "halo_synth_q8", D3(static_cast<std::uint32_t>(std::min<std::uint64_t>(CeilDiv(n, 256), 65536))),
                D3(256), a, err, errlen);
}

int halo_op_synth_f32(halo_engine* eng, float* x, uint64_t n, uint64_t seed, float sigma, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "synth_f32", {{"x", x}}) != 0) return -1;
  const halo_arg a[] = {Ptr(x), Val(n), Val(seed), Val(sigma)};
  return Launch(eng, "halo_synth_f32", D3(static_cast<std::uint32_t>(std::min<std::uint64_t>(CeilDiv(n, 256), 65536))),
                D3(256), a, err, errlen);
}

}  // extern "C"
