// Device sampling dispatch: one block of halo_sample_rows per row.
#include "engine.hpp"
#include "halo_sample.h"

using namespace halo::engine;

size_t halo_op_sample_workspace_bytes(uint32_t rows, uint32_t vocab) {
  return static_cast<size_t>(rows) * vocab * 16;
}

int halo_op_sample(halo_engine* eng, const float* logits, uint32_t rows, uint64_t row_stride, uint32_t vocab,
                   const HaloSampleParams* params, const HaloPenalty* penalties, uint32_t pen_stride,
                   HaloSampleOut* out, void* ws, size_t ws_bytes, char* err, size_t errlen) {
  if (rows == 0 || vocab == 0 || vocab > HALO_SAMPLE_MAX_VOCAB)
    return SetErr(err, errlen, "sample: rows %u, vocab %u (1..%u)", rows, vocab, HALO_SAMPLE_MAX_VOCAB), -1;
  if (row_stride < vocab) return SetErr(err, errlen, "sample: row stride %llu < vocab %u",
                                        static_cast<unsigned long long>(row_stride), vocab), -1;
  if (logits == nullptr || params == nullptr || out == nullptr || (penalties == nullptr && pen_stride != 0))
    return SetErr(err, errlen, "sample: null buffer"), -1;
  if (ws == nullptr || ws_bytes < halo_op_sample_workspace_bytes(rows, vocab))
    return SetErr(err, errlen, "sample: workspace %zu < %zu bytes", ws_bytes,
                  halo_op_sample_workspace_bytes(rows, vocab)), -1;
  char* w = static_cast<char*>(ws);
  const halo_arg a[] = {Ptr(logits), Val(row_stride), Ptr(params), Ptr(penalties), U32(pen_stride), U32(vocab),
                        Ptr(w), Ptr(w + static_cast<size_t>(rows) * vocab * 8), Ptr(out)};
  return Launch(eng, "halo_sample_rows", D3(rows), D3(1024), a, err, errlen);
}
