// Gated DeltaNet dispatch (the recurrence launches of FlashNextGpu::Linear, src/engine/flash_next_gpu.cpp:510-579,
// and of LinearChunk, src/engine/prefill_chunk.cpp:520).
#include "engine.hpp"

using namespace halo::engine;

extern "C" {

int halo_op_gdn_decode(halo_engine* eng, float* state, const float* q, const float* k, const float* v,
                       const float* g, const float* beta, float* o, uint32_t S, uint32_t Hv, uint32_t Hk,
                       uint32_t d, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "gdn_decode", {{"state", state}, {"q", q}, {"k", k}, {"v", v}, {"g", g}, {"beta", beta}, {"o", o}}) != 0) return -1;
  if (d != 128) return SetErr(err, errlen, "gdn: head dim %u unsupported (128)", d), -1;
  if (S == 0 || Hv == 0 || Hk == 0 || Hv % Hk != 0)
    return SetErr(err, errlen, "gdn: %u sessions, %u value heads, %u key heads", S, Hv, Hk), -1;
  const halo_arg a[] = {Ptr(state), Ptr(q), Ptr(k), Ptr(v), Ptr(g), Ptr(beta), Ptr(o), U32(S), U32(Hv), U32(Hk)};
  return Launch(eng, "halo_gdn_decode_d128", D3(S * Hv * 4), D3(256), a, err, errlen);
}

uint32_t halo_gdn_chunk_table(const uint32_t* seqlens, uint32_t n_seq, uint32_t* chunks, uint32_t* seqs) {
  std::uint32_t n = 0, tok = 0;
  for (std::uint32_t s = 0; s < n_seq; ++s) {
    const std::uint32_t nc = (seqlens[s] + 63) / 64;
    if (seqs) {
      seqs[2 * s] = n;
      seqs[2 * s + 1] = nc;
    }
    for (std::uint32_t c = 0; c < nc; ++c, ++n)
      if (chunks) {
        chunks[3 * n] = tok + 64 * c;
        chunks[3 * n + 1] = std::min<std::uint32_t>(64, seqlens[s] - 64 * c);
        chunks[3 * n + 2] = s;
      }
    tok += seqlens[s];
  }
  return n;
}

size_t halo_op_gdn_prefill_workspace_bytes(uint32_t n_chunks, uint32_t Hv) {
  return static_cast<std::size_t>(n_chunks) * Hv * (4 * 64 * 128 + 64) * sizeof(float);
}

namespace {
int GdnPrefill(halo_engine* eng, bool f32, const void* q, const void* k, const void* v, const float* g,
               const float* beta, const uint32_t* chunks, const uint32_t* seqs, uint32_t n_chunks, uint32_t n_seq,
               float* state, float* o, uint32_t Hv, uint32_t Hk, uint32_t d, void* ws, size_t ws_bytes, char* err,
               size_t errlen) {
  if (d != 128) return SetErr(err, errlen, "gdn prefill: head dim %u unsupported (128)", d), -1;
  if (n_chunks == 0 || n_seq == 0 || Hv == 0 || Hk == 0 || Hv % Hk != 0)
    return SetErr(err, errlen, "gdn prefill: empty batch or bad heads"), -1;
  const std::size_t need = halo_op_gdn_prefill_workspace_bytes(n_chunks, Hv);
  if (ws == nullptr || ws_bytes < need) return SetErr(err, errlen, "gdn prefill: workspace %zu < %zu", ws_bytes, need), -1;
  float* wy = static_cast<float*>(ws);
  float* Gc = wy + static_cast<std::size_t>(n_chunks) * Hv * 4 * 64 * 128;
  {
    const halo_arg a[] = {Ptr(q), Ptr(k), Ptr(v), Ptr(g), Ptr(beta), Ptr(chunks), Ptr(wy), Ptr(Gc), U32(Hv), U32(Hk)};
    if (Launch(eng, f32 ? "halo_gdn_wy_prep_f32" : "halo_gdn_wy_prep", D3(n_chunks, Hv), D3(512), a, err, errlen) != 0)
      return -1;
  }
  const halo_arg a[] = {Ptr(k), Ptr(wy), Ptr(Gc), Ptr(chunks), Ptr(seqs), Ptr(state), Ptr(o), U32(Hv), U32(Hk)};
  // 32 value columns per block, or 16 when even then the blocks fit the 256 CUs once (one long prompt): the scan is
  // chunk-serial, so idle CUs are better spent splitting each block's work
  const bool n16 = static_cast<std::uint64_t>(n_seq) * Hv * 8 <= 256;
  const char* name = f32 ? (n16 ? "halo_gdn_wy_scan_f32_n16" : "halo_gdn_wy_scan_f32")
                         : (n16 ? "halo_gdn_wy_scan_n16" : "halo_gdn_wy_scan");
  return Launch(eng, name, D3(n_seq * Hv * (n16 ? 8 : 4)), D3(512), a, err, errlen);
}
}  // namespace

int halo_op_gdn_prefill(halo_engine* eng, const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                        const float* beta, const uint32_t* chunks, const uint32_t* seqs, uint32_t n_chunks,
                        uint32_t n_seq, float* state, float* o, uint32_t Hv, uint32_t Hk, uint32_t d, void* ws,
                        size_t ws_bytes, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "gdn_prefill", {{"q", q}, {"k", k}, {"v", v}, {"g", g}, {"beta", beta}, {"chunks", chunks}, {"seqs", seqs}, {"state", state}, {"o", o}, {"ws", ws}}) != 0) return -1;
  return GdnPrefill(eng, false, q, k, v, g, beta, chunks, seqs, n_chunks, n_seq, state, o, Hv, Hk, d, ws, ws_bytes,
                    err, errlen);
}

int halo_op_gdn_prefill_f32(halo_engine* eng, const float* q, const float* k, const float* v, const float* g,
                            const float* beta, const uint32_t* chunks, const uint32_t* seqs, uint32_t n_chunks,
                            uint32_t n_seq, float* state, float* o, uint32_t Hv, uint32_t Hk, uint32_t d, void* ws,
                            size_t ws_bytes, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "gdn_prefill_f32", {{"q", q}, {"k", k}, {"v", v}, {"g", g}, {"beta", beta}, {"chunks", chunks}, {"seqs", seqs}, {"state", state}, {"o", o}, {"ws", ws}}) != 0) return -1;
  return GdnPrefill(eng, true, q, k, v, g, beta, chunks, seqs, n_chunks, n_seq, state, o, Hv, Hk, d, ws, ws_bytes,
                    err, errlen);
}

}  // extern "C"
