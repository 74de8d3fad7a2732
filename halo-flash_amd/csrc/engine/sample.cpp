// Device sampling dispatch: four launches (prep, weights, collect over 4096-token slices; final per row).
#include "engine.hpp"
#include "halo_sample.h"
#include "kernels/sample_layout.h"

using namespace halo::engine;

size_t halo_op_sample_workspace_bytes(uint32_t rows, uint32_t vocab) {
  return halo::sample::MakeLayout(rows, vocab).bytes;
}

int halo_op_sample(halo_engine* eng, const float* logits, uint32_t rows, uint64_t row_stride, uint32_t vocab,
                   const HaloSampleParams* params, const HaloPenalty* penalties, uint32_t pen_stride,
                   HaloSampleOut* out, void* ws, size_t ws_bytes, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "sample", {{"logits", logits}, {"params", params}, {"out", out}, {"ws", ws}}) != 0) return -1;
  if (rows == 0 || rows > 65535 || vocab == 0 || vocab > HALO_SAMPLE_MAX_VOCAB)
    return SetErr(err, errlen, "sample: rows %u (1..65535), vocab %u (1..%u)", rows, vocab, HALO_SAMPLE_MAX_VOCAB),
           -1;
  if (row_stride < vocab) return SetErr(err, errlen, "sample: row stride %llu < vocab %u",
                                        static_cast<unsigned long long>(row_stride), vocab), -1;
  if (logits == nullptr || params == nullptr || out == nullptr || (penalties == nullptr && pen_stride != 0))
    return SetErr(err, errlen, "sample: null buffer"), -1;
  if (ws == nullptr || ws_bytes < halo_op_sample_workspace_bytes(rows, vocab))
    return SetErr(err, errlen, "sample: workspace %zu < %zu bytes", ws_bytes,
                  halo_op_sample_workspace_bytes(rows, vocab)), -1;
  const std::uint32_t nb = halo::sample::Blocks(vocab);
  const halo_arg a1[] = {Ptr(logits), Val(row_stride), Ptr(params), Ptr(penalties), U32(pen_stride), U32(vocab),
                         U32(rows), Ptr(ws)};
  const halo_arg a2[] = {Ptr(params), U32(pen_stride), U32(vocab), U32(rows), Ptr(ws)};
  const halo_arg a4[] = {Ptr(params), U32(pen_stride), U32(vocab), U32(rows), Ptr(ws), Ptr(out)};
  if (Launch(eng, "halo_sample_prep", D3(nb, rows), D3(1024), a1, err, errlen) != 0) return -1;
  if (Launch(eng, "halo_sample_weights", D3(nb, rows), D3(1024), a2, err, errlen) != 0) return -1;
  if (Launch(eng, "halo_sample_collect", D3(nb, rows), D3(1024), a2, err, errlen) != 0) return -1;
  return Launch(eng, "halo_sample_final", D3(rows), D3(1024), a4, err, errlen);
}
