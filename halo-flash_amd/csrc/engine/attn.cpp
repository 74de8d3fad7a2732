// Decode attention dispatch (FlashNextGpu::Attention, src/engine/flash_next_gpu.cpp:581-680, and the batched
// per-entry attention of StepBatch): paged KV, prefix read once per step for all sessions.
#include <algorithm>
#include <vector>

#include "engine.hpp"

using namespace halo::engine;

namespace {

constexpr std::uint32_t kChunk = 32;

int Check(const halo_paged_kv* kv, std::uint32_t Hq, char* err, std::size_t errlen) {
  if (kv == nullptr || kv->k_pool == nullptr || kv->v_pool == nullptr || kv->pages == nullptr || kv->nkv == nullptr)
    return SetErr(err, errlen, "attn: missing kv buffers"), -1;
  if (kv->head_dim != 256) return SetErr(err, errlen, "attn: head dim %u unsupported (256)", kv->head_dim), -1;
  if (kv->kv_heads == 0 || Hq % kv->kv_heads != 0 || kv->sessions == 0 || kv->sessions * (Hq / kv->kv_heads) > 32)
    return SetErr(err, errlen, "attn: %u sessions x %u q heads / %u kv heads unsupported", kv->sessions, Hq,
                  kv->kv_heads),
           -1;
  if (kv->prefix % 64 != 0 || kv->prefix > kv->max_context || kv->max_context > kv->max_pages * 16 ||
      CeilDiv(kv->max_context, kChunk) > 1024)
    return SetErr(err, errlen, "attn: prefix %u must be a multiple of 64 within max_context %u <= 16 * %u pages (<= 32K)",
                  kv->prefix, kv->max_context, kv->max_pages),
           -1;
  return 0;
}

void Chunks(const halo_paged_kv* kv, std::uint32_t* prefix_chunks, std::uint32_t* suffix_chunks) {
  *prefix_chunks = kv->prefix / kChunk;
  *suffix_chunks = std::max<std::uint32_t>(1, CeilDiv(kv->max_context - kv->prefix, kChunk));
}

}  // namespace

extern "C" {

size_t halo_op_attn_decode_workspace_bytes(const halo_paged_kv* kv, uint32_t Hq) {
  if (Check(kv, Hq, nullptr, 0) != 0) return 0;
  std::uint32_t pc, sc;
  Chunks(kv, &pc, &sc);
  const std::size_t items = static_cast<std::size_t>(kv->kv_heads) * (pc + kv->sessions * sc);
  const std::size_t slots = kv->sessions * (Hq / kv->kv_heads);
  return items * slots * (2 + kv->head_dim) * sizeof(float);
}

int halo_op_attn_decode_q8(halo_engine* eng, const halo_paged_kv* kv, const float* q, const float* gate, float* o,
                           int8_t* oq, float* os, uint32_t Hq, void* ws, size_t ws_bytes, char* err,
                           size_t errlen) {
  if (RequirePtrs(err, errlen, "attn_decode_q8", {{"kv", kv}, {"q", q}, {"ws", ws}}) != 0) return -1;
  if (Check(kv, Hq, err, errlen) != 0) return -1;
  const std::size_t need = halo_op_attn_decode_workspace_bytes(kv, Hq);
  if (ws == nullptr || ws_bytes < need) return SetErr(err, errlen, "attn: workspace %zu < %zu", ws_bytes, need), -1;
  std::uint32_t pc, sc;
  Chunks(kv, &pc, &sc);
  const std::uint32_t S = kv->sessions, Hkv = kv->kv_heads;
  const std::size_t items = static_cast<std::size_t>(Hkv) * (pc + S * sc);
  const std::size_t slots = S * (Hq / Hkv);
  float* pm = static_cast<float*>(ws);
  float* pl = pm + items * slots;
  float* pacc = pl + items * slots;
  {
    const halo_arg a[] = {Ptr(q), Ptr(kv->k_pool), Ptr(kv->v_pool), Ptr(kv->pages), Ptr(kv->nkv), Ptr(pm), Ptr(pl),
                          Ptr(pacc), U32(S), U32(Hq), U32(Hkv), U32(kv->prefix), U32(kv->max_pages), U32(pc), U32(sc)};
    // the same arithmetic per query as the fused step launch of this batch size (halo_op_attn_decode_step_q8)
    const char* name = slots <= 8 ? "halo_attn_decode_partial" : "halo_attn_decode_partial_mma";
    if (Launch(eng, name, D3(static_cast<std::uint32_t>(items)), D3(256), a, err, errlen) != 0) return -1;
  }
  const halo_arg a[] = {Ptr(pm), Ptr(pl), Ptr(pacc), Ptr(gate), Ptr(o), Ptr(oq), Ptr(os), U32(S), U32(Hq), U32(Hkv),
                        U32(pc), U32(sc)};
  // small batches split each head into 8 dim slices instead of 4: twice the blocks, twice the loads in flight
  const bool eighths = S * Hq * 4 < 256;
  return Launch(eng, eighths ? "halo_attn_decode_combine8" : "halo_attn_decode_combine", D3(S * Hq * (eighths ? 8 : 4)),
                D3(256), a, err, errlen);
}

int halo_op_attn_decode_step_q8(halo_engine* eng, const halo_paged_kv* kv, const float* qg, const float* k,
                                const float* v, const float* q_norm, const float* k_norm, uint32_t rot, float theta,
                                float eps, float* o, int8_t* oq, float* os, uint32_t Hq, void* ws, size_t ws_bytes,
                                char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "attn_decode_step_q8",
                  {{"kv", kv}, {"qg", qg}, {"k", k}, {"v", v}, {"q_norm", q_norm}, {"k_norm", k_norm}, {"ws", ws}}) != 0)
    return -1;
  if (Check(kv, Hq, err, errlen) != 0) return -1;
  if (rot == 0 || rot % 2 != 0 || rot > 128)
    return SetErr(err, errlen, "attn decode step: rotary dims %u must be even and <= 128", rot), -1;
  if (o == nullptr && oq == nullptr) return SetErr(err, errlen, "attn decode step: no output"), -1;
  if ((oq == nullptr) != (os == nullptr)) return SetErr(err, errlen, "attn decode step: oq and os go together"), -1;
  const std::size_t need = halo_op_attn_decode_workspace_bytes(kv, Hq);
  if (ws_bytes < need) return SetErr(err, errlen, "attn: workspace %zu < %zu", ws_bytes, need), -1;
  std::uint32_t pc, sc;
  Chunks(kv, &pc, &sc);
  const std::uint32_t S = kv->sessions, Hkv = kv->kv_heads;
  const std::size_t items = static_cast<std::size_t>(Hkv) * (pc + S * sc);
  const std::size_t slots = S * (Hq / Hkv);
  float* pm = static_cast<float*>(ws);
  float* pl = pm + items * slots;
  float* pacc = pl + items * slots;
  {
    const halo_arg a[] = {Ptr(qg), Ptr(k), Ptr(v), Ptr(q_norm), Ptr(k_norm), Ptr(kv->k_pool), Ptr(kv->v_pool),
                          Ptr(kv->pages), Ptr(kv->nkv), Ptr(pm), Ptr(pl), Ptr(pacc), U32(S), U32(Hq), U32(Hkv),
                          U32(kv->prefix), U32(kv->max_pages), U32(pc), U32(sc), U32(rot), Val(theta), Val(eps)};
    const char* name = slots <= 8 ? "halo_attn_decode_partial_qk2" : "halo_attn_decode_partial_qk";
    if (Launch(eng, name, D3(static_cast<std::uint32_t>(items)), D3(256), a, err, errlen) != 0)
      return -1;
  }
  const halo_arg a[] = {Ptr(pm), Ptr(pl), Ptr(pacc), Ptr(qg + 256), Ptr(o), Ptr(oq), Ptr(os), U32(S), U32(Hq),
                        U32(Hkv), U32(pc), U32(sc)};
  const bool eighths = S * Hq * 4 < 256;
  return Launch(eng, eighths ? "halo_attn_decode_combine8_qg" : "halo_attn_decode_combine_qg",
                D3(S * Hq * (eighths ? 8 : 4)), D3(256), a, err, errlen);
}

int halo_op_attn_decode(halo_engine* eng, const halo_paged_kv* kv, const float* q, const float* gate, float* o,
                        uint32_t Hq, void* ws, size_t ws_bytes, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "attn_decode", {{"kv", kv}, {"q", q}, {"o", o}, {"ws", ws}}) != 0) return -1;
  return halo_op_attn_decode_q8(eng, kv, q, gate, o, nullptr, nullptr, Hq, ws, ws_bytes, err, errlen);
}

size_t halo_op_attn_prefill_workspace_bytes(const halo_prefill_segment* segs, uint32_t nseg) {
  if (segs == nullptr) return 0;
  std::size_t tiles = 0;
  for (std::uint32_t i = 0; i < nseg; ++i) tiles += CeilDiv(segs[i].length, 8);
  return std::max<std::size_t>(tiles, 1) * 4 * sizeof(std::uint32_t);
}

int halo_op_attn_prefill(halo_engine* eng, const halo_paged_kv* kv, const halo_prefill_segment* segs, uint32_t nseg,
                         const float* q, const float* gate, float* o, int8_t* oq, float* os, uint32_t Hq, void* ws,
                         size_t ws_bytes, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "attn_prefill", {{"kv", kv}, {"segs", segs}, {"q", q}, {"ws", ws}}) != 0) return -1;
  if (kv == nullptr || kv->k_pool == nullptr || kv->v_pool == nullptr || kv->pages == nullptr)
    return SetErr(err, errlen, "attn prefill: missing kv buffers"), -1;
  if (kv->head_dim != 256 || kv->kv_heads == 0 || Hq != 8 * kv->kv_heads)
    return SetErr(err, errlen, "attn prefill: head dim 256 and 8 q heads per kv head (got %u / %u)", Hq, kv->kv_heads),
           -1;
  if (segs == nullptr || nseg == 0 || q == nullptr || gate == nullptr || (o == nullptr && oq == nullptr) ||
      ((oq == nullptr) != (os == nullptr)))
    return SetErr(err, errlen, "attn prefill: missing arguments"), -1;
  std::vector<std::uint32_t> tiles;
  for (std::uint32_t i = 0; i < nseg; ++i) {
    const halo_prefill_segment& g = segs[i];
    if (g.session >= kv->sessions || g.length == 0 || g.start + g.length > kv->max_context)
      return SetErr(err, errlen, "attn prefill: segment %u (session %u, %u + %u) out of range", i, g.session, g.start,
                    g.length),
             -1;
    for (std::uint32_t k = 0; k < g.length; k += 8)
      tiles.insert(tiles.end(), {g.first + k, std::min<std::uint32_t>(8, g.length - k), g.session, g.start + k});
  }
  const std::size_t need = tiles.size() * sizeof(std::uint32_t);
  if (ws == nullptr || ws_bytes < need) return SetErr(err, errlen, "attn prefill: workspace %zu < %zu", ws_bytes, need), -1;
  halo_buffer b{ws, need, nullptr};
  if (halo_upload(halo_engine_device(eng), &b, 0, tiles.data(), need, err, errlen) != 0) return -1;
  const halo_arg a[] = {Ptr(q), Ptr(gate), Ptr(kv->k_pool), Ptr(kv->v_pool), Ptr(kv->pages), Ptr(ws), Ptr(o), Ptr(oq),
                        Ptr(os), U32(Hq), U32(kv->kv_heads), U32(kv->max_pages)};
  return Launch(eng, "halo_attn_prefill", D3(static_cast<std::uint32_t>(tiles.size() / 4), kv->kv_heads), D3(256), a,
                err, errlen);
}

int halo_op_kv_append(halo_engine* eng, const halo_paged_kv* kv, const float* k, const float* v, char* err,
                      size_t errlen) {
  if (RequirePtrs(err, errlen, "kv_append", {{"kv", kv}, {"k", k}, {"v", v}}) != 0) return -1;
  if (kv == nullptr || kv->head_dim != 256) return SetErr(err, errlen, "kv append: head dim 256 only"), -1;
  const halo_arg a[] = {Ptr(k), Ptr(v), Ptr(kv->k_pool), Ptr(kv->v_pool), Ptr(kv->pages), Ptr(kv->nkv),
                        U32(kv->kv_heads), U32(kv->max_pages)};
  return Launch(eng, "halo_kv_append", D3(kv->sessions * kv->kv_heads), D3(64), a, err, errlen);
}

}  // extern "C"
