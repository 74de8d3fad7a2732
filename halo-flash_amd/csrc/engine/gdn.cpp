// Gated DeltaNet dispatch (the recurrence launches of FlashNextGpu::Linear, src/engine/flash_next_gpu.cpp:510-579,
// and of LinearChunk, src/engine/prefill_chunk.cpp:520).
#include "engine.hpp"

using namespace halo::engine;

extern "C" {

int halo_op_gdn_decode(halo_engine* eng, float* state, const float* q, const float* k, const float* v,
                       const float* g, const float* beta, float* o, uint32_t S, uint32_t Hv, uint32_t Hk,
                       uint32_t d, char* err, size_t errlen) {
  if (d != 128) return SetErr(err, errlen, "gdn: head dim %u unsupported (128)", d), -1;
  if (S == 0 || Hv == 0 || Hk == 0 || Hv % Hk != 0)
    return SetErr(err, errlen, "gdn: %u sessions, %u value heads, %u key heads", S, Hv, Hk), -1;
  const halo_arg a[] = {Ptr(state), Ptr(q), Ptr(k), Ptr(v), Ptr(g), Ptr(beta), Ptr(o), U32(S), U32(Hv), U32(Hk)};
  return Launch(eng, "halo_gdn_decode_d128", D3(S * Hv * 4), D3(256), a, err, errlen);
}

}  // extern "C"
