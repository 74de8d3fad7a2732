// MoE decode dispatch (FlashNextGpu::Moe, src/engine/flash_next_gpu.cpp:697-845, and the session-union path of
// StepBatch, src/engine/batch_decode.cpp): four launches over device-resident routing (three at one token: the
// routing folded into the gate/up launch), no host round trip.
// Workspace: logits, shared logit, quantized x, ids/weights, h in fp32 (rows t*k+s routed, T*k+t shared).
#include "engine.hpp"

using namespace halo::engine;

namespace {

constexpr std::uint32_t kMaxTokens = 16;

std::size_t Align(std::size_t v) { return (v + 255) / 256 * 256; }

int Check(const halo_moe_weights* w, std::uint32_t T, char* err, std::size_t errlen) {
  if (w == nullptr || w->router == nullptr || w->gate.qs == nullptr || w->up.qs == nullptr || w->down.qs == nullptr)
    return SetErr(err, errlen, "moe: missing tensors"), -1;
  if (T == 0 || T > kMaxTokens) return SetErr(err, errlen, "moe decode takes 1..%u tokens, got %u", kMaxTokens, T), -1;
  const std::uint32_t H = w->hidden, F = w->ff, SF = w->shared_ff;
  if (w->n_experts == 0 || w->n_experts > 1024 || w->n_used == 0 || w->n_used > 15 || w->n_used > w->n_experts)
    return SetErr(err, errlen, "moe: %u experts / %u used unsupported", w->n_experts, w->n_used), -1;
  if (H % 1024 != 0 || H > 4096 || H % 32 != 0) return SetErr(err, errlen, "moe: hidden %u must be 1024..4096 step 1024", H), -1;
  if (F % 32 != 0 || F == 0 || F > 512) return SetErr(err, errlen, "moe: expert ff %u must be a multiple of 32, <= 512", F), -1;
  const bool shared = w->shared_gate_proj.qs != nullptr;
  if (shared && (SF % 32 != 0 || SF == 0 || SF > 512 || w->shared_up.qs == nullptr || w->shared_down.qs == nullptr))
    return SetErr(err, errlen, "moe: shared ff %u must be a multiple of 32, <= 512", SF), -1;
  auto dense = [](const halo_q8_matrix& m, std::uint32_t rows, std::uint32_t cols) {
    return m.rows == rows && m.cols == cols && m.qstride == cols;
  };
  if (!dense(w->gate, w->n_experts * F, H) || !dense(w->up, w->n_experts * F, H) ||
      !dense(w->down, w->n_experts * H, F))
    return SetErr(err, errlen, "moe: expert tensors must be stacked [E*ff][H] / [E*H][ff] with qstride == cols"), -1;
  if (shared && (!dense(w->shared_gate_proj, SF, H) || !dense(w->shared_up, SF, H) || !dense(w->shared_down, H, SF)))
    return SetErr(err, errlen, "moe: shared expert tensors must be [sff][H] / [H][sff] with qstride == cols"), -1;
  return 0;
}

}  // namespace

extern "C" {

int halo_op_moe_views(const halo_moe_weights* w, uint32_t T, void* ws, halo_moe_views* v, char* err, size_t errlen) {
  if (Check(w, T, err, errlen) != 0) return -1;
  const std::uint32_t E = w->n_experts, k = w->n_used, H = w->hidden;
  const std::uint32_t hstride = std::max(w->ff, w->shared_ff ? w->shared_ff : w->ff);
  const std::uintptr_t base = reinterpret_cast<std::uintptr_t>(ws);
  std::size_t o = 0;
  auto take = [&](std::size_t bytes) {
    const std::uintptr_t r = base + o;
    o += Align(bytes);
    return reinterpret_cast<char*>(r);
  };
  v->logits = reinterpret_cast<float*>(take(sizeof(float) * T * E));
  v->shared_logit = reinterpret_cast<float*>(take(sizeof(float) * T));
  v->xq = reinterpret_cast<int8_t*>(take(static_cast<std::size_t>(T) * H));
  v->xs = reinterpret_cast<float*>(take(sizeof(float) * T * (H / 32)));
  v->ids = reinterpret_cast<uint32_t*>(take(sizeof(uint32_t) * T * k));
  v->weights = reinterpret_cast<float*>(take(sizeof(float) * T * k));
  v->h = reinterpret_cast<float*>(take(sizeof(float) * T * (k + 1) * hstride));
  v->hstride = hstride;
  v->bytes = o;
  return 0;
}

size_t halo_op_moe_workspace_bytes(const halo_moe_weights* w, uint32_t T) {
  halo_moe_views v;
  if (halo_op_moe_views(w, T, nullptr, &v, nullptr, 0) != 0) return 0;
  return v.bytes;
}

}  // extern "C"

namespace {
// The MoE decode launches after the router stage; `in` (mode N) selects the router with the norm prologue.
int MoeDecode(halo_engine* eng, const halo_moe_weights* w, const float* x, const halo_proj_input* in, float* out,
              uint32_t T, void* ws, size_t ws_bytes, char* err, size_t errlen) {
  halo_moe_views v;
  if (halo_op_moe_views(w, T, ws, &v, err, errlen) != 0) return -1;
  if (ws == nullptr || ws_bytes < v.bytes)
    return SetErr(err, errlen, "moe: workspace of %zu bytes < %zu", ws_bytes, v.bytes), -1;
  const std::uint32_t E = w->n_experts, k = w->n_used, H = w->hidden, F = w->ff;
  const bool shared = w->shared_gate_proj.qs != nullptr;
  const std::uint32_t SF = shared ? w->shared_ff : 0;
  if (in != nullptr) {
    // 1. FFN norm + router logits + shared gate logit + x quantized, one launch
    if (T == 0 || T > 4 || (H != 2048 && H != 4096) || T * H > 8192 || in->x == nullptr || in->delta == nullptr ||
        in->norm_w == nullptr || in->res_out == nullptr || in->res_out == in->x)
      return SetErr(err, errlen, "moe: fused norm needs T <= 4, hidden 2048 / 4096, T * hidden <= 8192, x, delta, "
                                 "norm weights and a separate residual output"), -1;
    const halo_arg a[] = {Ptr(w->router), Ptr(shared ? w->shared_gate : nullptr), Ptr(in->x), Ptr(in->delta),
                          Ptr(in->norm_w), Ptr(in->res_out), Ptr(v.logits), Ptr(v.shared_logit), Ptr(v.xq),
                          Ptr(v.xs), U32(E), U32(T), Val(in->eps)};
    const char* rname = T == 1 ? (H == 2048 ? "halo_moe_router_n1_h2048" : "halo_moe_router_n1_h4096")
                               : (H == 2048 ? "halo_moe_router_n_h2048" : "halo_moe_router_n_h4096");
    if (Launch(eng, rname, D3(CeilDiv(E + 1, 4)), D3(256), a, err, errlen) != 0)
      return -1;
  } else {
    // 1. router logits + shared gate logit + x quantized
    const std::uint32_t qblocks = CeilDiv(static_cast<std::uint64_t>(T) * (H / 32), 8);
    const halo_arg a[] = {Ptr(w->router), Ptr(shared ? w->shared_gate : nullptr), Ptr(x), Ptr(v.logits),
                          Ptr(v.shared_logit), Ptr(v.xq), Ptr(v.xs), U32(E), U32(H), U32(T)};
    if (Launch(eng, "halo_moe_router", D3(E + 1 + qblocks), D3(256), a, err, errlen) != 0) return -1;
  }
  if (H != 1024 && H != 2048 && H != 4096) return SetErr(err, errlen, "moe: hidden %u has no gate/up instance", H), -1;
  if (T == 1) {
    // 2 + 3. one token: the routing runs in every routed gate/up block (cheaper than a launch of its own)
    const halo_arg a[] = {Ptr(w->gate.qs), Ptr(w->gate.d), Ptr(w->up.qs), Ptr(w->up.d),
                          Ptr(shared ? w->shared_gate_proj.qs : nullptr), Ptr(shared ? w->shared_gate_proj.d : nullptr),
                          Ptr(shared ? w->shared_up.qs : nullptr), Ptr(shared ? w->shared_up.d : nullptr),
                          Ptr(v.xq), Ptr(v.xs), Ptr(v.logits), Ptr(v.ids), Ptr(v.weights), Ptr(v.h), U32(E), U32(F),
                          U32(SF), U32(k), U32(v.hstride)};
    char name[48];
    std::snprintf(name, sizeof name, "halo_moe_gate_up_topk_q8_s%u%s", H / 1024, E <= 512 ? "_e512" : "");
    if (Launch(eng, name, D3(k + 1, v.hstride / 4), D3(256), a, err, errlen) != 0) return -1;
  } else {
    // 2. softmax / top-k, one wave per token
    const halo_arg t[] = {Ptr(v.logits), Ptr(v.ids), Ptr(v.weights), U32(E), U32(k)};
    const bool wave = E <= 1024 && k <= 64;
    if (Launch(eng, !wave ? "halo_moe_topk" : E <= 512 ? "halo_moe_topk_w512" : "halo_moe_topk_w1024", D3(T),
               D3(wave ? 64 : CeilDiv(E, 64) * 64), t, err, errlen) != 0)
      return -1;
    // 3. gate/up over the union of experts + SwiGLU
    const halo_arg a[] = {Ptr(w->gate.qs), Ptr(w->gate.d), Ptr(w->up.qs), Ptr(w->up.d),
                          Ptr(shared ? w->shared_gate_proj.qs : nullptr), Ptr(shared ? w->shared_gate_proj.d : nullptr),
                          Ptr(shared ? w->shared_up.qs : nullptr), Ptr(shared ? w->shared_up.d : nullptr),
                          Ptr(v.xq), Ptr(v.xs), Ptr(v.ids), Ptr(v.h), U32(T), U32(F), U32(SF), U32(k),
                          U32(v.hstride)};
    const char* name = H == 1024 ? "halo_moe_gate_up_q8_s1" : H == 2048 ? "halo_moe_gate_up_q8_s2" : "halo_moe_gate_up_q8_s4";
    if (Launch(eng, name, D3(T * k + 1, v.hstride / 4), D3(256), a, err, errlen) != 0) return -1;
  }
  // 4. down + routed combine + shared expert
  {
    const halo_arg a[] = {Ptr(w->down.qs), Ptr(w->down.d), Ptr(shared ? w->shared_down.qs : nullptr),
                          Ptr(shared ? w->shared_down.d : nullptr), Ptr(v.h), Ptr(v.ids), Ptr(v.weights),
                          Ptr(v.shared_logit), Ptr(out), U32(T), U32(H), U32(F), U32(SF), U32(k), U32(v.hstride)};
    // 8 output rows per block at one token, 16 for token batches (measured: T = 1 16.9 vs 17.9 us, T = 4 38.9 vs
    // 37.5 us, T = 16 112.8 vs 107.7 us)
    const std::uint32_t rows = T == 1 ? 8 : 16;
    if (Launch(eng, T == 1 ? "halo_moe_down_q8" : "halo_moe_down_q8_r16", D3(CeilDiv(H, rows), T), D3(64 * (k + 1)),
               a, err, errlen) != 0)
      return -1;
  }
  return 0;
}
}  // namespace

extern "C" {

int halo_op_moe_decode(halo_engine* eng, const halo_moe_weights* w, const float* x, float* out, uint32_t T, void* ws,
                       size_t ws_bytes, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "moe_decode", {{"x", x}, {"out", out}, {"ws", ws}}) != 0) return -1;
  return MoeDecode(eng, w, x, nullptr, out, T, ws, ws_bytes, err, errlen);
}

int halo_op_moe_decode_norm(halo_engine* eng, const halo_moe_weights* w, const halo_proj_input* in, float* out,
                            uint32_t T, void* ws, size_t ws_bytes, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "moe_decode_norm", {{"in", in}, {"out", out}, {"ws", ws}}) != 0) return -1;
  if (in == nullptr) return SetErr(err, errlen, "moe: no input"), -1;
  return MoeDecode(eng, w, nullptr, in, out, T, ws, ws_bytes, err, errlen);
}

}  // extern "C"

namespace {
// Pairs per grouped-GEMM tile: 128 once the groups average 96 pairs or more (a prefill batch of thousands of tokens:
// twice the weight reuse per staged stage outweighs the emptier last tile of each group), else 64.
std::uint32_t PrefillTile(std::uint64_t pairs, std::uint32_t E) { return pairs >= 96ull * E ? 128u : 64u; }
}  // namespace

namespace halo::engine {
int MoePrefillLayout(const halo_moe_weights* w, std::uint32_t T, void* ws, MoePrefillViews* v, char* err,
                     std::size_t errlen) {
  if (w == nullptr || w->router == nullptr || w->gate.qs == nullptr) return SetErr(err, errlen, "moe: missing tensors"), -1;
  const std::uint32_t E = w->n_experts, k = w->n_used, H = w->hidden, F = w->ff;
  const bool shared = w->shared_gate_proj.qs != nullptr;
  if (T == 0) return SetErr(err, errlen, "moe prefill: no tokens"), -1;
  if (E == 0 || E + 1 > 1024 || k == 0 || k > 16 || k > E)
    return SetErr(err, errlen, "moe prefill: %u experts / %u used unsupported", E, k), -1;
  if (H % 64 != 0 || F % 64 != 0 || F == 0) return SetErr(err, errlen, "moe prefill: hidden %u / ff %u", H, F), -1;
  if (shared && (w->shared_ff != F || w->shared_gate == nullptr))
    return SetErr(err, errlen, "moe prefill: the shared expert must have ff %u and a gate row", F), -1;
  auto dense = [](const halo_q8_matrix& m, std::uint32_t rows, std::uint32_t cols) {
    return m.rows == rows && m.cols == cols && m.qstride == cols;
  };
  if (!dense(w->gate, E * F, H) || !dense(w->up, E * F, H) || !dense(w->down, E * H, F))
    return SetErr(err, errlen, "moe prefill: expert tensors must be stacked with qstride == cols"), -1;
  const std::uint64_t P = static_cast<std::uint64_t>(T) * k, G = P + (shared ? T : 0);
  const std::uintptr_t base = reinterpret_cast<std::uintptr_t>(ws);
  std::size_t o = 0;
  auto take = [&](std::size_t bytes) {
    const std::uintptr_t r = base + o;
    o += Align(bytes);
    return reinterpret_cast<char*>(r);
  };
  v->logits = reinterpret_cast<float*>(take(sizeof(float) * T * E));
  v->sgl = reinterpret_cast<float*>(take(sizeof(float) * T));
  v->xq = reinterpret_cast<std::int8_t*>(take(static_cast<std::size_t>(T) * H));
  v->xs = reinterpret_cast<float*>(take(sizeof(float) * T * (H / 32)));
  v->ids = reinterpret_cast<std::uint32_t*>(take(sizeof(std::uint32_t) * P));
  v->weights = reinterpret_cast<float*>(take(sizeof(float) * P));
  v->count = reinterpret_cast<std::uint32_t*>(take(sizeof(std::uint32_t) * CeilDiv(P, 4096) * E));  // histograms
  v->start = reinterpret_cast<std::uint32_t*>(take(sizeof(std::uint32_t) * (E + 2)));
  v->max_tiles = static_cast<std::uint32_t>(CeilDiv(G, PrefillTile(P, E)) + E + 1);
  v->tiles = reinterpret_cast<std::uint32_t*>(take(sizeof(std::uint32_t) * 3 * v->max_tiles));
  v->ntiles = reinterpret_cast<std::uint32_t*>(take(sizeof(std::uint32_t)));
  v->token = reinterpret_cast<std::uint32_t*>(take(sizeof(std::uint32_t) * G));
  v->pos = reinterpret_cast<std::uint32_t*>(take(sizeof(std::uint32_t) * P));
  v->h = reinterpret_cast<float*>(take(sizeof(float) * G * F));
  v->hq = reinterpret_cast<std::int8_t*>(take(G * F));
  v->hs = reinterpret_cast<float*>(take(sizeof(float) * G * (F / 32)));
  v->y = reinterpret_cast<float*>(take(sizeof(float) * G * H));
  v->bytes = o;
  return 0;
}
}  // namespace halo::engine

namespace {
using PrefillViews = MoePrefillViews;
int PrefillLayout(const halo_moe_weights* w, std::uint32_t T, void* ws, PrefillViews* v, char* err,
                  std::size_t errlen) {
  return MoePrefillLayout(w, T, ws, v, err, errlen);
}
}  // namespace

extern "C" {

size_t halo_op_moe_prefill_workspace_bytes(const halo_moe_weights* w, uint32_t T) {
  PrefillViews v;
  if (PrefillLayout(w, T, nullptr, &v, nullptr, 0) != 0) return 0;
  return v.bytes;
}

int halo_op_moe_prefill(halo_engine* eng, const halo_moe_weights* w, const float* x, float* out, uint32_t T, void* ws,
                        size_t ws_bytes, char* err, size_t errlen) {
  if (RequirePtrs(err, errlen, "moe_prefill", {{"x", x}, {"out", out}, {"ws", ws}}) != 0) return -1;
  PrefillViews v;
  if (PrefillLayout(w, T, ws, &v, err, errlen) != 0) return -1;
  if (ws == nullptr || ws_bytes < v.bytes)
    return SetErr(err, errlen, "moe prefill: workspace of %zu bytes < %zu", ws_bytes, v.bytes), -1;
  if (reinterpret_cast<std::uintptr_t>(out) % 16 != 0 || reinterpret_cast<std::uintptr_t>(ws) % 16 != 0)
    return SetErr(err, errlen, "moe prefill: out and ws must be 16-byte aligned (the combine stores 16-byte rows)"), -1;
  const std::uint32_t E = w->n_experts, k = w->n_used, H = w->hidden, F = w->ff;
  const bool shared = w->shared_gate_proj.qs != nullptr;
  const std::uint32_t G = T * k + (shared ? T : 0);
  // 1. router logits [T][E] and the shared gate logit [T]
  {
    const halo_arg a[] = {Ptr(x), Ptr(w->router), Ptr(shared ? w->shared_gate : nullptr), Ptr(v.logits), Ptr(v.sgl),
                          U32(T), U32(E), U32(H), U32(E)};
    if (Launch(eng, "halo_gemm_f32_nt", D3(CeilDiv(E + 1, 64), CeilDiv(T, 64)), D3(256), a, err, errlen) != 0) return -1;
  }
  // 2. x quantized per 32
  {
    const halo_arg a[] = {Ptr(x), Ptr(v.xq), Ptr(v.xs), U32(H), U32(T)};
    if (Launch(eng, "halo_quantize_q8_rows8", D3(CeilDiv(T, 8)), D3(256), a, err, errlen) != 0) return -1;
  }
  // 3. softmax / top-k per token
  {
    const halo_arg a[] = {Ptr(v.logits), Ptr(v.ids), Ptr(v.weights), U32(E), U32(k)};
    if (Launch(eng, "halo_moe_topk", D3(T), D3(CeilDiv(E, 64) * 64), a, err, errlen) != 0) return -1;
  }
  // 4. group the pairs by expert (token order within an expert), tile table
  {
    const std::uint32_t nb = static_cast<std::uint32_t>(CeilDiv(static_cast<std::uint64_t>(T) * k, 4096));
    const std::uint32_t tile = PrefillTile(static_cast<std::uint64_t>(T) * k, E);
    const halo_arg a[] = {Ptr(v.ids), Ptr(v.count), U32(T), U32(k), U32(E)};
    if (Launch(eng, "halo_moe_group_count", D3(nb), D3(256), a, err, errlen) != 0) return -1;
    const halo_arg b[] = {Ptr(v.count), Ptr(v.start), Ptr(v.tiles), Ptr(v.ntiles), U32(E), U32(T), U32(shared ? 1 : 0),
                          U32(tile), U32(nb)};
    if (Launch(eng, "halo_moe_group_scan", D3(1), D3(1024), b, err, errlen) != 0) return -1;
    const halo_arg c[] = {Ptr(v.ids), Ptr(v.start), Ptr(v.token), Ptr(v.pos), U32(T), U32(k), U32(E)};
    if (Launch(eng, "halo_moe_group_fill", D3(E + (shared ? 1 : 0)), D3(1024), c, err, errlen) != 0) return -1;
  }
  // 5. grouped gate / up + SwiGLU -> h [G][F]
  {
    const halo_arg a[] = {Ptr(w->gate.qs), Ptr(w->gate.d), Ptr(w->up.qs), Ptr(w->up.d),
                          Ptr(shared ? w->shared_gate_proj.qs : nullptr), Ptr(shared ? w->shared_gate_proj.d : nullptr),
                          Ptr(shared ? w->shared_up.qs : nullptr), Ptr(shared ? w->shared_up.d : nullptr), Ptr(v.xq),
                          Ptr(v.xs), Ptr(v.token), Ptr(v.tiles), Ptr(v.ntiles), Ptr(v.h), U32(F), U32(H), U32(E), U32(F)};
    const bool t128 = PrefillTile(static_cast<std::uint64_t>(T) * k, E) == 128;
    if (Launch(eng, t128 ? "halo_moe_grouped_gate_up_q8_t128" : "halo_moe_grouped_gate_up_q8",
               D3(CeilDiv(F, 64), v.max_tiles), D3(t128 ? 512 : 256), a, err, errlen) != 0)
      return -1;
  }
  // 6. h quantized per 32
  {
    const halo_arg a[] = {Ptr(v.h), Ptr(v.hq), Ptr(v.hs), U32(F), U32(G)};
    if (Launch(eng, "halo_quantize_q8_rows8", D3(CeilDiv(G, 8)), D3(256), a, err, errlen) != 0) return -1;
  }
  // 7. grouped down -> y [G][H]
  {
    const halo_arg a[] = {Ptr(w->down.qs), Ptr(w->down.d), Ptr(shared ? w->shared_down.qs : nullptr),
                          Ptr(shared ? w->shared_down.d : nullptr), Ptr(v.hq), Ptr(v.hs), Ptr(v.tiles), Ptr(v.ntiles),
                          Ptr(v.y), U32(H), U32(F), U32(E)};
    const bool t128 = PrefillTile(static_cast<std::uint64_t>(T) * k, E) == 128;
    if (Launch(eng, t128 ? "halo_moe_grouped_down_q8_t128" : "halo_moe_grouped_down_q8", D3(CeilDiv(H, 128), v.max_tiles),
               D3(512), a, err, errlen) != 0)
      return -1;
  }
  // 8. slot-order combine + shared expert
  const halo_arg a[] = {Ptr(v.y), Ptr(v.pos), Ptr(v.weights), Ptr(v.sgl), Ptr(out), U32(T), U32(H), U32(k),
                        U32(shared ? 1 : 0)};
  return Launch(eng, "halo_moe_prefill_combine", D3(CeilDiv(H, 1024), T), D3(256), a, err, errlen);
}

}  // extern "C"
