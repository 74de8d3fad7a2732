// halo_model: weights, sessions and the captured decode step of the synthetic hybrid model.
//
// Reference: FlashNextGpu::Init (src/engine/flash_next_gpu.cpp:256-409) allocates weights and scratch;
// Record / Run (847-1047) record one token through every layer into a graph and replay it with per-step values in
// device memory (HaloStepParam, src/kernels/step_params.h); StepBatch (src/engine/batch_decode.cpp:629-817) runs B
// sessions per step with weights read once; ForkSession (flash_next_gpu.hpp:347-350) shares prefix pages.
#include "halo_model.h"

#include <algorithm>
#include <initializer_list>
#include <cmath>
#include <map>
#include <tuple>
#include <string>
#include <memory>
#include <utility>
#include <vector>

#include "engine.hpp"

using namespace halo::engine;

namespace {

struct Q8 {
  halo_buffer qs{}, d{};
  halo_q8_matrix m{};
};

struct Layer {
  bool attn = false;
  halo_buffer attn_norm{}, ffn_norm{};
  // Gated DeltaNet
  Q8 qkv, z, ab, out;  // ab: alpha | beta logits [2 Hv][H]
  halo_buffer conv_w{}, a{}, dt{}, norm_w{};
  // attention
  Q8 qg, k, v, o;
  halo_buffer q_norm{}, k_norm{}, k_pool{}, v_pool{};
  // MoE
  halo_buffer router{}, shared_gate{};
  Q8 gate, up, down, sgate, sup, sdown;
  halo_moe_weights moe{};
  std::uint32_t gdn_index = 0;  // index among DeltaNet layers (state slot)
};

}  // namespace

struct halo_model {
  halo_engine* eng = nullptr;
  halo_device* dev = nullptr;
  halo_model_config c{};
  std::vector<Layer> layers;
  Q8 embd, head;
  halo_buffer out_norm{};
  std::uint32_t n_gdn = 0, n_attn = 0, max_pages = 0, prefix_pages = 0, total_pages = 0, conv_ch = 0;
  // state
  halo_buffer gdn_state{}, conv_state{}, pages{}, nkv{}, tokens{}, prompt{}, prompt_len{}, history{}, produced{};
  // step scratch
  halo_buffer res{}, res2{}, xn{}, xq{}, xs{}, qkv{}, zo{}, abo{}, q{}, k{}, v{}, g{}, beta{}, o{}, oq{}, os{}, delta{};
  halo_buffer qgo{}, ko{}, vo{}, aq{}, agate{}, ao{}, moe_ws{}, attn_ws{}, logits{}, argmax_part{};
  std::size_t moe_ws_bytes = 0, attn_ws_bytes = 0;
  std::vector<halo_buffer> owned;
  std::map<std::tuple<std::uint32_t, std::uint32_t, bool>, halo_graph> graphs;
  // device sampling (halo_model_set_sampling): per-session parameters and penalty lists, the draws, workspace
  bool sampling = false;
  halo_buffer sample_params{}, sample_pen{}, sample_out{}, sample_ws{};
  // prefill batch scratch, allocated at the first prefill for the prefill batch cap tokens
  struct Prefill {
    bool ready = false;
    halo_buffer res{}, xn{}, xq{}, xs{}, qkv{}, zo{}, abo{}, qb{}, kb{}, vb{}, g{}, beta{}, o{}, oq{}, os{}, delta{};
    halo_buffer qgo{}, ko{}, vo{}, q{}, gate{}, tok{}, segs{}, chunks{}, seqs{}, gdn_ws{}, attn_ws{}, moe_ws{};
    halo_buffer lq{}, ls{};
    std::size_t gdn_ws_bytes = 0, attn_ws_bytes = 0, moe_ws_bytes = 0;
  } pf;
  std::uint64_t weight_bytes = 0, device_bytes = 0;
};

namespace {

int Alloc(halo_model* m, std::size_t bytes, halo_buffer* b, char* err, std::size_t errlen) {
  if (halo_alloc(m->dev, bytes, b, err, errlen) != 0) return -1;
  m->owned.push_back(*b);
  m->device_bytes += bytes;
  return 0;
}

int SynthF32(halo_model* m, halo_buffer* b, std::size_t n, std::uint64_t seed, float sigma, float mean, char* err,
             std::size_t errlen) {
  if (Alloc(m, n * 4, b, err, errlen) != 0) return -1;
  if (halo_op_synth_f32(m->eng, static_cast<float*>(b->device), n, seed, sigma, err, errlen) != 0) return -1;
  m->weight_bytes += n * 4;
  if (mean != 0.0f) {
    const halo_arg a[] = {Ptr(b->device), Val<std::uint64_t>(n), Val(1.0f), Val(mean)};
    return Launch(m->eng, "halo_affine_f32", D3(static_cast<std::uint32_t>(std::min<std::size_t>(CeilDiv(n, 256), 4096))),
                  D3(256), a, err, errlen);
  }
  return 0;
}

int SynthQ8(halo_model* m, Q8* w, std::uint32_t rows, std::uint32_t cols, std::uint64_t seed, char* err,
            std::size_t errlen) {
  const std::uint32_t qstride = cols;
  if (Alloc(m, static_cast<std::size_t>(rows) * qstride, &w->qs, err, errlen) != 0 ||
      Alloc(m, static_cast<std::size_t>(rows) * (cols / 32) * 2, &w->d, err, errlen) != 0)
    return -1;
  w->m = halo_q8_matrix{static_cast<const int8_t*>(w->qs.device), static_cast<const uint16_t*>(w->d.device), rows,
                        cols, qstride, 0};
  m->weight_bytes += static_cast<std::uint64_t>(rows) * (cols / 32) * 34;
  return halo_op_synth_q8(m->eng, static_cast<int8_t*>(w->qs.device), static_cast<uint16_t*>(w->d.device), rows, cols,
                          qstride, seed, 0.02f, err, errlen);
}

template <typename T>
T* P(const halo_buffer& b) {
  return static_cast<T*>(b.device);
}

halo_paged_kv KvDesc(halo_model* m, const Layer& L, std::uint32_t S, std::uint32_t prefix) {
  halo_paged_kv kv{};
  kv.k_pool = P<float>(L.k_pool);
  kv.v_pool = P<float>(L.v_pool);
  kv.pages = P<uint32_t>(m->pages);
  kv.nkv = P<uint32_t>(m->nkv);
  kv.sessions = S;
  kv.kv_heads = m->c.kv_heads;
  kv.head_dim = m->c.head_dim;
  kv.max_pages = m->max_pages;
  kv.prefix = prefix;
  kv.max_context = m->c.max_context;
  return kv;
}

int Check(const halo_model_config* c, char* err, std::size_t errlen) {
  if (c->hidden % 1024 != 0 || c->hidden > 4096)
    return SetErr(err, errlen, "model: hidden %u must be 1024..4096 in steps of 1024", c->hidden), -1;
  if (c->gdn_head_dim != 128 || c->head_dim != 256 || c->conv_kernel < 1 || c->conv_kernel > 8)
    return SetErr(err, errlen, "model: DeltaNet head dim 128, attention head dim 256, conv kernel 1..8"), -1;
  if (c->max_sessions == 0 || c->max_sessions > 16 || c->max_sessions * (c->q_heads / c->kv_heads) > 32)
    return SetErr(err, errlen, "model: %u sessions unsupported", c->max_sessions), -1;
  if (c->prefix_tokens % 64 != 0 || c->prefix_tokens > c->max_context || c->attn_interval == 0)
    return SetErr(err, errlen, "model: prefix %u must be a multiple of 64 within the context", c->prefix_tokens), -1;
  if ((2 * c->gdn_k_heads + c->gdn_v_heads) * c->gdn_head_dim % 256 != 0)
    return SetErr(err, errlen, "model: DeltaNet channels must be a multiple of 256"), -1;
  if (c->rotary_dim > 128 || c->rotary_dim % 64 != 0)
    return SetErr(err, errlen, "model: rotary dim must be 64 or 128"), -1;
  if (c->prefill_batch != 0 && (c->prefill_batch < 64 || c->prefill_batch > 65536))
    return SetErr(err, errlen, "model: prefill batch %u must be 0 (8192) or 64 ... 65536", c->prefill_batch), -1;
  return 0;
}

// Teacher-forcing trace of an eager step (halo_model_step_trace): after the launches that produce them, named device
// tensors are copied into the caller's trace buffer (one halo_copy launch each) and listed in `entries`.
struct Tracer {
  halo_engine* eng = nullptr;
  char* base = nullptr;
  std::size_t cap = 0, used = 0;
  halo_model_trace_entry* entries = nullptr;
  std::uint32_t max_entries = 0, n = 0;
  std::uint64_t mask = ~std::uint64_t{0};  // bit l: layer l (l < 63); bit 63: the final norm

  int Save(const char* name, std::uint32_t layer, std::uint32_t dtype, const void* src, std::size_t bytes, char* err,
           std::size_t errlen) {
    if (!((mask >> (layer < 63 ? layer : 63)) & 1u)) return 0;
    if (bytes % 4 != 0) return SetErr(err, errlen, "trace: %s has %zu bytes (not whole words)", name, bytes), -1;
    const std::size_t at = (used + 255) / 256 * 256;
    if (at + bytes > cap || n >= max_entries)
      return SetErr(err, errlen, "trace: buffer of %zu bytes / %u entries too small at %s of layer %u", cap,
                    max_entries, name, layer), -1;
    halo_model_trace_entry& e = entries[n++];
    e = halo_model_trace_entry{};
    std::snprintf(e.name, sizeof e.name, "%s", name);
    e.layer = layer;
    e.dtype = dtype;
    e.offset = at;
    e.bytes = bytes;
    used = at + bytes;
    const halo_arg a[] = {Ptr(base + at), Ptr(src), U32(static_cast<std::uint32_t>(bytes / 4))};
    return Launch(eng, "halo_copy", D3(CeilDiv(bytes / 4, 256 * 4)), D3(256), a, err, errlen);
  }
};

int Record(halo_model* m, std::uint32_t S, std::uint32_t prefix, char* err, std::size_t errlen,
           Tracer* tr = nullptr) {
  const halo_model_config& c = m->c;
  const std::uint32_t H = c.hidden, Hv = c.gdn_v_heads, Hk = c.gdn_k_heads, d = c.gdn_head_dim;
  const std::uint32_t Dv = Hv * d, C = m->conv_ch, Hq = c.q_heads, Hkv = c.kv_heads, hd = c.head_dim;
  const float eps = c.rms_eps;
  halo_engine* eng = m->eng;
  // embedding
  {
    const halo_arg a[] = {Ptr(m->embd.qs.device), Ptr(m->embd.d.device), Ptr(m->tokens.device), Ptr(m->res.device),
                          U32(H), U32(H)};
    if (Launch(eng, "halo_embed_q8", D3(S), D3(256), a, err, errlen) != 0) return -1;
  }
  // Residual stream: `cur` holds it. A projection prologue that adds a delta reads `cur` and writes the sum to
  // the other buffer (its blocks all read `cur` while block 0 writes), then the two swap.
  halo_buffer* cur = &m->res;
  halo_buffer* alt = &m->res2;
  bool have_delta = false;
  auto norm = [&](const halo_buffer& w, bool quant) {
    const halo_arg a[] = {Ptr(cur->device), Ptr(have_delta ? m->delta.device : nullptr), Ptr(w.device),
                          Ptr(m->xn.device), Ptr(quant ? m->xq.device : nullptr), Ptr(m->xs.device), U32(H), Val(eps)};
    have_delta = false;
    return Launch(eng, "halo_add_rmsnorm_q8", D3(S), D3(256), a, err, errlen);
  };
  // attention-side input norm fused into the layer's first projections (one launch)
  auto proj_norm = [&](const halo_buffer& w, std::initializer_list<const Q8*> mats,
                       std::initializer_list<const halo_buffer*> outs) {
    halo_q8_matrix ms[4];
    float* ys[4];
    std::uint32_t n = 0;
    for (const Q8* q : mats) ms[n++] = q->m;
    n = 0;
    for (const halo_buffer* b : outs) ys[n++] = P<float>(*b);
    halo_proj_input in{};
    if (S > 1) {
      // several sessions: the norm's per-token prologue would run in every block; one norm launch is cheaper
      if (norm(w, true) != 0) return -1;
      in.xq = P<int8_t>(m->xq);
      in.xs = P<float>(m->xs);
      in.mode = HALO_PROJ_Q;
      return halo_op_proj_q8(eng, ms, ys, n, &in, S, err, errlen);
    }
    in.x = P<float>(*cur);
    in.delta = have_delta ? P<float>(m->delta) : nullptr;
    in.norm_w = P<float>(w);
    in.res_out = have_delta ? P<float>(*alt) : nullptr;
    in.eps = eps;
    in.mode = HALO_PROJ_N;
    if (tr != nullptr) {  // the trace records the prologue's quantized activations
      in.xq_out = P<int8_t>(m->xq);
      in.xs_out = P<float>(m->xs);
    }
    if (halo_op_proj_q8(eng, ms, ys, n, &in, S, err, errlen) != 0) return -1;
    if (have_delta) std::swap(cur, alt);
    have_delta = false;
    return 0;
  };
  auto gemv = [&](const Q8& w, const halo_buffer& xq, const halo_buffer& xs, const halo_buffer& y) {
    return halo_op_matvec_q8a8(eng, &w.m, P<int8_t>(xq), P<float>(xs), P<float>(y), S, w.m.rows, err, errlen);
  };
  // trace helpers (no-ops without a tracer): fp32 / int8 / uint32 tensors of `count` elements
  std::uint32_t li = 0;
  auto save = [&](const char* name, std::uint32_t dtype, const void* src, std::size_t count) {
    if (tr == nullptr) return 0;
    return tr->Save(name, li, dtype, src, count * (dtype == HALO_TRACE_I8 ? 1 : 4), err, errlen);
  };
  auto save_input = [&]() {  // the layer's residual input and its quantized norm
    if (save("res_in", HALO_TRACE_F32, cur->device, static_cast<std::size_t>(S) * H) != 0 ||
        save("xq", HALO_TRACE_I8, m->xq.device, static_cast<std::size_t>(S) * H) != 0 ||
        save("xs", HALO_TRACE_F32, m->xs.device, static_cast<std::size_t>(S) * H / 32) != 0)
      return -1;
    return 0;
  };
  for (auto& L : m->layers) {
    if (!L.attn) {
      if (proj_norm(L.attn_norm, {&L.qkv, &L.z, &L.ab}, {&m->qkv, &m->zo, &m->abo}) != 0) return -1;
      if (save_input() != 0 || save("qkv", HALO_TRACE_F32, m->qkv.device, static_cast<std::size_t>(S) * C) != 0 ||
          save("z", HALO_TRACE_F32, m->zo.device, static_cast<std::size_t>(S) * Dv) != 0 ||
          save("ab", HALO_TRACE_F32, m->abo.device, static_cast<std::size_t>(S) * 2 * Hv) != 0)
        return -1;
      float* ring = P<float>(m->conv_state) + static_cast<std::size_t>(L.gdn_index) * c.max_sessions *
                                                  c.conv_kernel * C;
      float* st = P<float>(m->gdn_state) + static_cast<std::size_t>(L.gdn_index) * c.max_sessions * Hv * d * d;
      {  // conv + norms + gates + recurrence + gated output norm + quantization, one block per (session, head)
        const halo_arg a[] = {Ptr(m->qkv.device), Ptr(m->zo.device), Ptr(m->abo.device), Ptr(ring),
                              Ptr(L.conv_w.device), Ptr(L.a.device), Ptr(L.dt.device), Ptr(L.norm_w.device), Ptr(st),
                              Ptr(m->nkv.device), Ptr(m->oq.device), Ptr(m->os.device), U32(Hk), U32(Hv),
                              U32(c.conv_kernel), Val(eps)};
        if (Launch(eng, c.conv_kernel <= 4 ? "halo_gdn_step_q8" : "halo_gdn_step_q8_kn", D3(S * Hv), D3(512), a, err,
                   errlen) != 0)
          return -1;
      }
      if (save("oq", HALO_TRACE_I8, m->oq.device, static_cast<std::size_t>(S) * Dv) != 0 ||
          save("os", HALO_TRACE_F32, m->os.device, static_cast<std::size_t>(S) * Dv / 32) != 0)
        return -1;
      if (gemv(L.out, m->oq, m->os, m->delta) != 0) return -1;
    } else {
      if (proj_norm(L.attn_norm, {&L.qg, &L.k, &L.v}, {&m->qgo, &m->ko, &m->vo}) != 0) return -1;
      if (save_input() != 0 ||
          save("qg", HALO_TRACE_F32, m->qgo.device, static_cast<std::size_t>(S) * 2 * Hq * hd) != 0 ||
          save("k", HALO_TRACE_F32, m->ko.device, static_cast<std::size_t>(S) * Hkv * hd) != 0 ||
          save("v", HALO_TRACE_F32, m->vo.device, static_cast<std::size_t>(S) * Hkv * hd) != 0)
        return -1;
      // q / k norms, rotation and the K / V append run inside the attention's partial launch
      const halo_paged_kv kv = KvDesc(m, L, S, prefix);
      if (halo_op_attn_decode_step_q8(eng, &kv, P<float>(m->qgo), P<float>(m->ko), P<float>(m->vo),
                                      P<float>(L.q_norm), P<float>(L.k_norm), c.rotary_dim, c.rope_theta, eps, nullptr,
                                      P<int8_t>(m->oq), P<float>(m->os), Hq, m->attn_ws.device, m->attn_ws_bytes, err,
                                      errlen) != 0)
        return -1;
      if (save("oq", HALO_TRACE_I8, m->oq.device, static_cast<std::size_t>(S) * Hq * hd) != 0 ||
          save("os", HALO_TRACE_F32, m->os.device, static_cast<std::size_t>(S) * Hq * hd / 32) != 0)
        return -1;
      if (gemv(L.o, m->oq, m->os, m->delta) != 0) return -1;
    }
    if (save("delta", HALO_TRACE_F32, m->delta.device, static_cast<std::size_t>(S) * H) != 0) return -1;
    have_delta = true;
    if (S <= 4 && (H == 2048 || H == 4096) && S * H <= 8192) {
      // the FFN norm runs in the router's prologue
      halo_proj_input in{};
      in.x = P<float>(*cur);
      in.delta = P<float>(m->delta);
      in.norm_w = P<float>(L.ffn_norm);
      in.res_out = P<float>(*alt);
      in.eps = eps;
      in.mode = HALO_PROJ_N;
      if (halo_op_moe_decode_norm(eng, &L.moe, &in, P<float>(m->delta), S, m->moe_ws.device, m->moe_ws_bytes, err,
                                  errlen) != 0)
        return -1;
      std::swap(cur, alt);
    } else {
      if (norm(L.ffn_norm, false) != 0) return -1;
      if (halo_op_moe_decode(eng, &L.moe, P<float>(m->xn), P<float>(m->delta), S, m->moe_ws.device,
                             m->moe_ws_bytes, err, errlen) != 0)
        return -1;
    }
    if (tr != nullptr) {  // the MoE's input residual, routing, h and output
      halo_moe_views v;
      if (halo_op_moe_views(&L.moe, S, m->moe_ws.device, &v, err, errlen) != 0) return -1;
      const std::uint32_t k = c.n_used;
      if (save("mres", HALO_TRACE_F32, cur->device, static_cast<std::size_t>(S) * H) != 0 ||
          save("mxq", HALO_TRACE_I8, v.xq, static_cast<std::size_t>(S) * H) != 0 ||
          save("mxs", HALO_TRACE_F32, v.xs, static_cast<std::size_t>(S) * H / 32) != 0 ||
          save("mlogits", HALO_TRACE_F32, v.logits, static_cast<std::size_t>(S) * c.n_experts) != 0 ||
          save("mshared", HALO_TRACE_F32, v.shared_logit, S) != 0 ||
          save("mids", HALO_TRACE_U32, v.ids, static_cast<std::size_t>(S) * k) != 0 ||
          save("mweights", HALO_TRACE_F32, v.weights, static_cast<std::size_t>(S) * k) != 0 ||
          save("mh", HALO_TRACE_F32, v.h, static_cast<std::size_t>(S) * (k + 1) * v.hstride) != 0 ||
          save("mout", HALO_TRACE_F32, m->delta.device, static_cast<std::size_t>(S) * H) != 0)
        return -1;
    }
    have_delta = true;
    ++li;
  }
  if (norm(m->out_norm, true) != 0) return -1;
  li = UINT32_MAX;
  if (save("res_in", HALO_TRACE_F32, cur->device, static_cast<std::size_t>(S) * H) != 0 ||
      save("xq", HALO_TRACE_I8, m->xq.device, static_cast<std::size_t>(S) * H) != 0 ||
      save("xs", HALO_TRACE_F32, m->xs.device, static_cast<std::size_t>(S) * H / 32) != 0)
    return -1;
  if (gemv(m->head, m->xq, m->xs, m->logits) != 0) return -1;
  if (m->sampling) {
    // every session draws with its own parameters (temperature 0 is the argmax); the advance takes the drawn
    // tokens and carries each session's RNG state into the next step
    if (halo_op_sample(eng, P<float>(m->logits), S, c.vocab, c.vocab,
                       static_cast<const HaloSampleParams*>(m->sample_params.device),
                       static_cast<const HaloPenalty*>(m->sample_pen.device), HALO_SAMPLE_MAX_PENALTIES,
                       static_cast<HaloSampleOut*>(m->sample_out.device), m->sample_ws.device, m->sample_ws.bytes, err,
                       errlen) != 0)
      return -1;
    const halo_arg a[] = {Ptr(m->sample_out.device), Ptr(m->sample_params.device), Ptr(m->prompt.device),
                          Ptr(m->prompt_len.device), Ptr(m->tokens.device), Ptr(m->nkv.device),
                          Ptr(m->history.device), Ptr(m->produced.device), U32(S), U32(c.vocab),
                          U32(c.max_context), U32(c.max_context), U32(c.max_context)};
    return Launch(eng, "halo_step_advance_sampled", D3(1), D3(64), a, err, errlen);
  }
  constexpr std::uint32_t kParts = 64;
  float* pv = P<float>(m->argmax_part);
  std::uint32_t* pi = reinterpret_cast<std::uint32_t*>(pv + c.max_sessions * kParts);
  {
    const halo_arg a[] = {Ptr(m->logits.device), Ptr(pv), Ptr(pi), U32(c.vocab)};
    if (Launch(eng, "halo_argmax_part", D3(S, kParts), D3(256), a, err, errlen) != 0) return -1;
  }
  const halo_arg a[] = {Ptr(pv), Ptr(pi), Ptr(m->prompt.device), Ptr(m->prompt_len.device), Ptr(m->tokens.device),
                        Ptr(m->nkv.device), Ptr(m->history.device), Ptr(m->produced.device), U32(S), U32(kParts),
                        U32(c.max_context), U32(c.max_context), U32(c.max_context)};
  // one wave per session, up to 16 sessions per block
  return Launch(eng, "halo_step_advance", D3(CeilDiv(S, 16)), D3(64 * std::min<std::uint32_t>(S, 16)), a, err, errlen);
}


// Tokens per prefill batch: the config's prefill_batch, 8192 by default. Every expert's gate / up / down weights are
// read once per batch, so larger batches amortize them over more rows of the grouped GEMMs.
std::uint32_t PrefillCap(const halo_model_config& c) { return c.prefill_batch ? c.prefill_batch : 8192u; }

int PrefillAlloc(halo_model* m, char* err, std::size_t errlen) {
  if (m->pf.ready) return 0;
  const halo_model_config& c = m->c;
  const std::size_t T = PrefillCap(c), H = c.hidden, Dv = static_cast<std::size_t>(c.gdn_v_heads) * c.gdn_head_dim;
  const std::size_t Dk = static_cast<std::size_t>(c.gdn_k_heads) * c.gdn_head_dim, C = m->conv_ch;
  const std::size_t A = static_cast<std::size_t>(c.q_heads) * c.head_dim, KV = static_cast<std::size_t>(c.kv_heads) * c.head_dim;
  const std::size_t O = std::max(Dv, A);
  auto& p = m->pf;
  const std::uint32_t max_chunks = PrefillCap(c) / 64 + c.max_sessions;
  p.gdn_ws_bytes = halo_op_gdn_prefill_workspace_bytes(max_chunks, c.gdn_v_heads);
  p.moe_ws_bytes = halo_op_moe_prefill_workspace_bytes(&m->layers[0].moe, PrefillCap(c));
  p.attn_ws_bytes = (PrefillCap(c) / 8 + c.max_sessions) * 4 * sizeof(std::uint32_t);
  if (p.moe_ws_bytes == 0) return SetErr(err, errlen, "prefill: MoE shape unsupported by the batched path"), -1;
  struct B {
    halo_buffer* b;
    std::size_t bytes;
  };
  const B bufs[] = {
      {&p.res, T * H * 4}, {&p.xn, T * H * 4}, {&p.xq, T * H}, {&p.xs, T * H / 8}, {&p.qkv, T * C * 4},
      {&p.zo, T * Dv * 4}, {&p.abo, T * 2 * c.gdn_v_heads * 4}, {&p.qb, T * Dk * 4}, {&p.kb, T * Dk * 4},
      {&p.vb, T * Dv * 4}, {&p.g, T * c.gdn_v_heads * 4}, {&p.beta, T * c.gdn_v_heads * 4}, {&p.o, T * O * 4},
      {&p.oq, T * O}, {&p.os, T * O / 8}, {&p.delta, T * H * 4}, {&p.qgo, T * 2 * A * 4}, {&p.ko, T * KV * 4},
      {&p.vo, T * KV * 4}, {&p.q, T * A * 4}, {&p.gate, T * A * 4}, {&p.tok, T * 3 * 4},
      {&p.segs, static_cast<std::size_t>(c.max_sessions) * 16 * 4}, {&p.chunks, max_chunks * 3 * 4},
      {&p.seqs, static_cast<std::size_t>(c.max_sessions) * 2 * 4}, {&p.gdn_ws, p.gdn_ws_bytes},
      {&p.attn_ws, p.attn_ws_bytes}, {&p.moe_ws, p.moe_ws_bytes},
      {&p.lq, static_cast<std::size_t>(c.max_sessions) * H}, {&p.ls, static_cast<std::size_t>(c.max_sessions) * H / 8},
  };
  for (const auto& b : bufs)
    if (Alloc(m, b.bytes, b.b, err, errlen) != 0) return -1;
  p.ready = true;
  return 0;
}

// One prefill batch: segments with consecutive increasing sessions s0, s0 + 1, ..., positions already in the cache
// below each segment's start. T = sum of lengths <= the prefill batch cap.
int PrefillBatch(halo_model* m, const std::vector<halo_prefill_segment>& segs, char* err, std::size_t errlen,
                 Tracer* tr = nullptr) {
  const halo_model_config& c = m->c;
  halo_engine* eng = m->eng;
  auto& p = m->pf;
  const std::uint32_t H = c.hidden, Hv = c.gdn_v_heads, Hk = c.gdn_k_heads, d = c.gdn_head_dim, C = m->conv_ch;
  const std::uint32_t Hq = c.q_heads, Hkv = c.kv_heads, hd = c.head_dim;
  const float eps = c.rms_eps;
  const std::uint32_t nseg = static_cast<std::uint32_t>(segs.size()), s0 = segs[0].session;
  std::uint32_t T = 0;
  std::vector<std::uint32_t> tok_sess, tok_pos, seg_start, segtab, lens;
  for (const auto& g : segs) {
    segtab.insert(segtab.end(), {g.session, g.start, g.length, T});
    lens.push_back(g.length);
    for (std::uint32_t j = 0; j < g.length; ++j) {
      tok_sess.push_back(g.session);
      tok_pos.push_back(g.start + j);
      seg_start.push_back(g.start);
    }
    T += g.length;
  }
  std::vector<std::uint32_t> tok(tok_sess);
  tok.insert(tok.end(), tok_pos.begin(), tok_pos.end());
  tok.insert(tok.end(), seg_start.begin(), seg_start.end());
  const std::uint32_t nchunks = halo_gdn_chunk_table(lens.data(), nseg, nullptr, nullptr);
  std::vector<std::uint32_t> chunks(static_cast<std::size_t>(nchunks) * 3), seqs(static_cast<std::size_t>(nseg) * 2);
  halo_gdn_chunk_table(lens.data(), nseg, chunks.data(), seqs.data());
  if (halo_upload(m->dev, &p.tok, 0, tok.data(), tok.size() * 4, err, errlen) != 0 ||
      halo_upload(m->dev, &p.segs, 0, segtab.data(), segtab.size() * 4, err, errlen) != 0 ||
      halo_upload(m->dev, &p.chunks, 0, chunks.data(), chunks.size() * 4, err, errlen) != 0 ||
      halo_upload(m->dev, &p.seqs, 0, seqs.data(), seqs.size() * 4, err, errlen) != 0)
    return -1;
  const std::uint32_t* ts = P<std::uint32_t>(p.tok);
  const std::uint32_t* tp = ts + T;
  const std::uint32_t* tstart = tp + T;
  {
    const halo_arg a[] = {Ptr(m->embd.qs.device), Ptr(m->embd.d.device), Ptr(m->prompt.device), U32(c.max_context),
                          Ptr(ts), Ptr(tp), Ptr(p.res.device), U32(H), U32(H)};
    if (Launch(eng, "halo_embed_prompt_q8", D3(T), D3(256), a, err, errlen) != 0) return -1;
  }
  bool have_delta = false;
  auto norm = [&](const halo_buffer& w, bool xn) {
    const halo_arg a[] = {Ptr(p.res.device), Ptr(have_delta ? p.delta.device : nullptr), Ptr(w.device),
                          Ptr(xn ? p.xn.device : nullptr), Ptr(p.xq.device), Ptr(p.xs.device), U32(H), Val(eps)};
    have_delta = false;
    return Launch(eng, "halo_add_rmsnorm_q8", D3(T), D3(256), a, err, errlen);
  };
  auto gemm = [&](const Q8& w, const halo_buffer& xq, const halo_buffer& xs, const halo_buffer& y) {
    return halo_op_matvec_q8a8(eng, &w.m, P<int8_t>(xq), P<float>(xs), P<float>(y), T, w.m.rows, err, errlen);
  };
  std::vector<halo_prefill_segment> asegs(segs);
  for (std::uint32_t i = 0, f = 0; i < nseg; f += asegs[i].length, ++i) asegs[i].first = f;
  std::uint32_t li = 0;
  auto save = [&](const char* name, std::uint32_t dtype, const void* src, std::size_t count) {
    if (tr == nullptr) return 0;
    return tr->Save(name, li, dtype, src, count * (dtype == HALO_TRACE_I8 ? 1 : 4), err, errlen);
  };
  auto save_norm = [&](const char* res, const char* q, const char* sc) {
    if (save(res, HALO_TRACE_F32, p.res.device, static_cast<std::size_t>(T) * H) != 0 ||
        save(q, HALO_TRACE_I8, p.xq.device, static_cast<std::size_t>(T) * H) != 0 ||
        save(sc, HALO_TRACE_F32, p.xs.device, static_cast<std::size_t>(T) * H / 32) != 0)
      return -1;
    return 0;
  };
  for (auto& L : m->layers) {
    if (norm(L.attn_norm, false) != 0 || save_norm("res_in", "xq", "xs") != 0) return -1;
    if (!L.attn) {
      if (gemm(L.qkv, p.xq, p.xs, p.qkv) != 0 || gemm(L.z, p.xq, p.xs, p.zo) != 0 || gemm(L.ab, p.xq, p.xs, p.abo) != 0)
        return -1;
      if (save("qkv", HALO_TRACE_F32, p.qkv.device, static_cast<std::size_t>(T) * C) != 0 ||
          save("z", HALO_TRACE_F32, p.zo.device, static_cast<std::size_t>(T) * Hv * d) != 0 ||
          save("ab", HALO_TRACE_F32, p.abo.device, static_cast<std::size_t>(T) * 2 * Hv) != 0)
        return -1;
      float* ring = P<float>(m->conv_state) + static_cast<std::size_t>(L.gdn_index) * c.max_sessions * c.conv_kernel * C;
      {
        const halo_arg a[] = {Ptr(p.qkv.device), Ptr(ring), Ptr(L.conv_w.device), Ptr(p.abo.device), Ptr(L.a.device),
                              Ptr(L.dt.device), Ptr(ts), Ptr(tp), Ptr(tstart), Ptr(p.qb.device), Ptr(p.kb.device),
                              Ptr(p.vb.device), Ptr(p.g.device), Ptr(p.beta.device), U32(T), U32(Hk), U32(Hv),
                              U32(c.conv_kernel), Val(eps)};
        const char* prep = c.conv_kernel == 4 ? "halo_gdn_prep_prefill_k4" : "halo_gdn_prep_prefill";
        if (Launch(eng, prep, D3(CeilDiv(T, 16), C / 256), D3(64), a, err, errlen) != 0) return -1;
      }
      if (save("gq", HALO_TRACE_F32, p.qb.device, static_cast<std::size_t>(T) * Hk * d) != 0 ||
          save("gk", HALO_TRACE_F32, p.kb.device, static_cast<std::size_t>(T) * Hk * d) != 0 ||
          save("gv", HALO_TRACE_F32, p.vb.device, static_cast<std::size_t>(T) * Hv * d) != 0 ||
          save("g", HALO_TRACE_F32, p.g.device, static_cast<std::size_t>(T) * Hv) != 0 ||
          save("beta", HALO_TRACE_F32, p.beta.device, static_cast<std::size_t>(T) * Hv) != 0)
        return -1;
      {
        const halo_arg a[] = {Ptr(p.qkv.device), Ptr(ring), Ptr(p.segs.device), U32(c.conv_kernel), U32(C)};
        if (Launch(eng, "halo_gdn_ring_update", D3(nseg, C / 256), D3(256), a, err, errlen) != 0) return -1;
      }
      float* st = P<float>(m->gdn_state) +
                  (static_cast<std::size_t>(L.gdn_index) * c.max_sessions + s0) * Hv * d * d;
      if (halo_op_gdn_prefill_f32(eng, P<float>(p.qb), P<float>(p.kb), P<float>(p.vb), P<float>(p.g),
                              P<float>(p.beta), P<uint32_t>(p.chunks), P<uint32_t>(p.seqs), nchunks, nseg, st,
                              P<float>(p.o), Hv, Hk, d, p.gdn_ws.device, p.gdn_ws_bytes, err, errlen) != 0)
        return -1;
      if (save("o", HALO_TRACE_F32, p.o.device, static_cast<std::size_t>(T) * Hv * d) != 0) return -1;
      {
        const halo_arg a[] = {Ptr(p.o.device), Ptr(p.zo.device), Ptr(L.norm_w.device), Ptr(p.oq.device),
                              Ptr(p.os.device), U32(Hv), U32(d), Val(eps)};
        if (Launch(eng, "halo_gated_rmsnorm_q8", D3(T), D3(256), a, err, errlen) != 0) return -1;
      }
      if (save("oq", HALO_TRACE_I8, p.oq.device, static_cast<std::size_t>(T) * Hv * d) != 0 ||
          save("os", HALO_TRACE_F32, p.os.device, static_cast<std::size_t>(T) * Hv * d / 32) != 0)
        return -1;
      if (gemm(L.out, p.oq, p.os, p.delta) != 0) return -1;
    } else {
      if (gemm(L.qg, p.xq, p.xs, p.qgo) != 0 || gemm(L.k, p.xq, p.xs, p.ko) != 0 || gemm(L.v, p.xq, p.xs, p.vo) != 0)
        return -1;
      if (save("qg", HALO_TRACE_F32, p.qgo.device, static_cast<std::size_t>(T) * 2 * Hq * hd) != 0 ||
          save("k", HALO_TRACE_F32, p.ko.device, static_cast<std::size_t>(T) * Hkv * hd) != 0 ||
          save("v", HALO_TRACE_F32, p.vo.device, static_cast<std::size_t>(T) * Hkv * hd) != 0)
        return -1;
      {
        const halo_arg a[] = {Ptr(p.qgo.device), Ptr(p.ko.device), Ptr(p.vo.device), Ptr(L.q_norm.device),
                              Ptr(L.k_norm.device), Ptr(p.q.device), Ptr(p.gate.device), Ptr(L.k_pool.device),
                              Ptr(L.v_pool.device), Ptr(m->pages.device), Ptr(m->nkv.device), U32(Hq), U32(Hkv),
                              U32(m->max_pages), U32(c.rotary_dim), Val(c.rope_theta), Val(eps), Ptr(ts), Ptr(tp)};
        if (Launch(eng, "halo_attn_prep_decode", D3(T, Hq + 2 * Hkv), D3(64), a, err, errlen) != 0) return -1;
      }
      const halo_paged_kv kv = KvDesc(m, L, c.max_sessions, 0);
      if (halo_op_attn_prefill(eng, &kv, asegs.data(), nseg, P<float>(p.q), P<float>(p.gate), nullptr,
                               P<int8_t>(p.oq), P<float>(p.os), Hq, p.attn_ws.device, p.attn_ws_bytes, err,
                               errlen) != 0)
        return -1;
      if (save("aq", HALO_TRACE_F32, p.q.device, static_cast<std::size_t>(T) * Hq * hd) != 0 ||
          save("oq", HALO_TRACE_I8, p.oq.device, static_cast<std::size_t>(T) * Hq * hd) != 0 ||
          save("os", HALO_TRACE_F32, p.os.device, static_cast<std::size_t>(T) * Hq * hd / 32) != 0)
        return -1;
      if (gemm(L.o, p.oq, p.os, p.delta) != 0) return -1;
    }
    if (save("delta", HALO_TRACE_F32, p.delta.device, static_cast<std::size_t>(T) * H) != 0) return -1;
    have_delta = true;
    if (norm(L.ffn_norm, true) != 0) return -1;
    if (halo_op_moe_prefill(eng, &L.moe, P<float>(p.xn), P<float>(p.delta), T, p.moe_ws.device, p.moe_ws_bytes, err,
                            errlen) != 0)
      return -1;
    if (tr != nullptr) {  // the MoE's input residual, routing, h (sorted pairs), its codes and the output
      MoePrefillViews v;
      if (MoePrefillLayout(&L.moe, T, p.moe_ws.device, &v, err, errlen) != 0) return -1;
      const std::size_t k = c.n_used, G = T * k + T, F = c.expert_ff;
      if (save("mres", HALO_TRACE_F32, p.res.device, static_cast<std::size_t>(T) * H) != 0 ||
          save("mxq", HALO_TRACE_I8, v.xq, static_cast<std::size_t>(T) * H) != 0 ||
          save("mxs", HALO_TRACE_F32, v.xs, static_cast<std::size_t>(T) * H / 32) != 0 ||
          save("mlogits", HALO_TRACE_F32, v.logits, static_cast<std::size_t>(T) * c.n_experts) != 0 ||
          save("mshared", HALO_TRACE_F32, v.sgl, T) != 0 || save("mids", HALO_TRACE_U32, v.ids, T * k) != 0 ||
          save("mweights", HALO_TRACE_F32, v.weights, T * k) != 0 || save("mpos", HALO_TRACE_U32, v.pos, T * k) != 0 ||
          save("mh", HALO_TRACE_F32, v.h, G * F) != 0 || save("mhq", HALO_TRACE_I8, v.hq, G * F) != 0 ||
          save("mhs", HALO_TRACE_F32, v.hs, G * F / 32) != 0 ||
          save("mout", HALO_TRACE_F32, p.delta.device, static_cast<std::size_t>(T) * H) != 0)
        return -1;
    }
    have_delta = true;
    ++li;
  }
  if (norm(m->out_norm, false) != 0) return -1;
  li = UINT32_MAX;
  if (save_norm("res_in", "xq", "xs") != 0) return -1;
  {
    const halo_arg a[] = {Ptr(p.xq.device), Ptr(p.xs.device), Ptr(p.segs.device), Ptr(p.lq.device), Ptr(p.ls.device),
                          U32(H)};
    if (Launch(eng, "halo_prefill_gather_last", D3(nseg), D3(256), a, err, errlen) != 0) return -1;
  }
  float* lg = P<float>(m->logits) + static_cast<std::size_t>(s0) * c.vocab;
  if (halo_op_matvec_q8a8(eng, &m->head.m, P<int8_t>(p.lq), P<float>(p.ls), lg, nseg, c.vocab, err, errlen) != 0)
    return -1;
  constexpr std::uint32_t kParts = 64;
  float* pv = P<float>(m->argmax_part);
  std::uint32_t* pi = reinterpret_cast<std::uint32_t*>(pv + c.max_sessions * kParts);
  {
    const halo_arg a[] = {Ptr(lg), Ptr(pv), Ptr(pi), U32(c.vocab)};
    if (Launch(eng, "halo_argmax_part", D3(nseg, kParts), D3(256), a, err, errlen) != 0) return -1;
  }
  const halo_arg a[] = {Ptr(pv), Ptr(pi), Ptr(p.segs.device), Ptr(m->prompt.device), Ptr(m->prompt_len.device),
                        Ptr(m->tokens.device), Ptr(m->nkv.device), Ptr(m->history.device), Ptr(m->produced.device),
                        U32(nseg), U32(kParts), U32(c.max_context), U32(c.max_context)};
  return Launch(eng, "halo_prefill_advance", D3(1), D3(64), a, err, errlen);
}

}  // namespace

extern "C" {

int halo_model_create(halo_engine* eng, const halo_model_config* cfg, uint64_t seed, halo_model** out, char* err,
                      size_t errlen) {
  if (eng == nullptr || cfg == nullptr || out == nullptr) return SetErr(err, errlen, "null argument"), -1;
  *out = nullptr;
  if (Check(cfg, err, errlen) != 0) return -1;
  auto m = std::make_unique<halo_model>();
  m->eng = eng;
  m->dev = halo_engine_device(eng);
  m->c = *cfg;
  const halo_model_config& c = m->c;
  const std::uint32_t H = c.hidden, Hv = c.gdn_v_heads, Hk = c.gdn_k_heads, d = c.gdn_head_dim;
  const std::uint32_t Dk = Hk * d, Dv = Hv * d, Hq = c.q_heads, Hkv = c.kv_heads, hd = c.head_dim;
  const std::uint32_t S = c.max_sessions, E = c.n_experts, F = c.expert_ff, SF = c.shared_ff;
  m->conv_ch = 2 * Dk + Dv;
  m->max_pages = CeilDiv(c.max_context, 16);
  m->prefix_pages = c.prefix_tokens / 16;
  m->total_pages = m->prefix_pages + S * (m->max_pages - m->prefix_pages);
  std::uint64_t sd = seed * 1000003ull;
  auto next = [&]() { return ++sd; };
  m->layers.resize(c.layers);
  for (std::uint32_t l = 0; l < c.layers; ++l) {
    Layer& L = m->layers[l];
    L.attn = (l + 1) % c.attn_interval == 0;
    if (SynthF32(m.get(), &L.attn_norm, H, next(), 0.02f, 1.0f, err, errlen) != 0 ||
        SynthF32(m.get(), &L.ffn_norm, H, next(), 0.02f, 1.0f, err, errlen) != 0)
      return -1;
    if (!L.attn) {
      L.gdn_index = m->n_gdn++;
      if (SynthQ8(m.get(), &L.qkv, m->conv_ch, H, next(), err, errlen) != 0 ||
          SynthQ8(m.get(), &L.z, Dv, H, next(), err, errlen) != 0 ||
          SynthQ8(m.get(), &L.out, H, Dv, next(), err, errlen) != 0 ||
          SynthQ8(m.get(), &L.ab, 2 * Hv, H, next(), err, errlen) != 0 ||
          SynthF32(m.get(), &L.conv_w, static_cast<std::size_t>(m->conv_ch) * c.conv_kernel, next(), 0.3f, 0.0f, err,
                   errlen) != 0 ||
          SynthF32(m.get(), &L.a, Hv, next(), 0.1f, -1.0f, err, errlen) != 0 ||
          SynthF32(m.get(), &L.dt, Hv, next(), 0.5f, 0.0f, err, errlen) != 0 ||
          SynthF32(m.get(), &L.norm_w, d, next(), 0.02f, 1.0f, err, errlen) != 0)
        return -1;
    } else {
      ++m->n_attn;
      const std::size_t pool = static_cast<std::size_t>(m->total_pages) * Hkv * 16 * hd * 4;
      if (SynthQ8(m.get(), &L.qg, 2 * Hq * hd, H, next(), err, errlen) != 0 ||
          SynthQ8(m.get(), &L.k, Hkv * hd, H, next(), err, errlen) != 0 ||
          SynthQ8(m.get(), &L.v, Hkv * hd, H, next(), err, errlen) != 0 ||
          SynthQ8(m.get(), &L.o, H, Hq * hd, next(), err, errlen) != 0 ||
          SynthF32(m.get(), &L.q_norm, hd, next(), 0.02f, 1.0f, err, errlen) != 0 ||
          SynthF32(m.get(), &L.k_norm, hd, next(), 0.02f, 1.0f, err, errlen) != 0 ||
          Alloc(m.get(), pool, &L.k_pool, err, errlen) != 0 || Alloc(m.get(), pool, &L.v_pool, err, errlen) != 0)
        return -1;
    }
    if (SynthF32(m.get(), &L.router, static_cast<std::size_t>(E) * H, next(), 0.02f, 0.0f, err, errlen) != 0 ||
        SynthF32(m.get(), &L.shared_gate, H, next(), 0.02f, 0.0f, err, errlen) != 0 ||
        SynthQ8(m.get(), &L.gate, E * F, H, next(), err, errlen) != 0 ||
        SynthQ8(m.get(), &L.up, E * F, H, next(), err, errlen) != 0 ||
        SynthQ8(m.get(), &L.down, E * H, F, next(), err, errlen) != 0 ||
        SynthQ8(m.get(), &L.sgate, SF, H, next(), err, errlen) != 0 ||
        SynthQ8(m.get(), &L.sup, SF, H, next(), err, errlen) != 0 ||
        SynthQ8(m.get(), &L.sdown, H, SF, next(), err, errlen) != 0)
      return -1;
    halo_moe_weights& w = L.moe;
    w.router = P<float>(L.router);
    w.shared_gate = P<float>(L.shared_gate);
    w.gate = L.gate.m;
    w.up = L.up.m;
    w.down = L.down.m;
    w.shared_gate_proj = L.sgate.m;
    w.shared_up = L.sup.m;
    w.shared_down = L.sdown.m;
    w.n_experts = E;
    w.n_used = c.n_used;
    w.hidden = H;
    w.ff = F;
    w.shared_ff = SF;
  }
  if (SynthQ8(m.get(), &m->embd, c.vocab, H, next(), err, errlen) != 0 ||
      SynthQ8(m.get(), &m->head, c.vocab, H, next(), err, errlen) != 0 ||
      SynthF32(m.get(), &m->out_norm, H, next(), 0.02f, 1.0f, err, errlen) != 0)
    return -1;
  // sessions and step scratch
  const std::size_t ctx = c.max_context;
  struct B {
    halo_buffer* b;
    std::size_t bytes;
  };
  const std::uint32_t C = m->conv_ch;
  const B bufs[] = {
      {&m->gdn_state, static_cast<std::size_t>(m->n_gdn) * S * Hv * d * d * 4},
      {&m->conv_state, static_cast<std::size_t>(m->n_gdn) * S * c.conv_kernel * C * 4},  // ring of K slots
      {&m->pages, static_cast<std::size_t>(S) * m->max_pages * 4},
      {&m->nkv, S * 4},
      {&m->tokens, S * 4},
      {&m->prompt, S * ctx * 4},
      {&m->prompt_len, S * 4},
      {&m->history, S * ctx * 4},
      {&m->produced, S * 4},
      {&m->res, static_cast<std::size_t>(S) * H * 4},
      {&m->res2, static_cast<std::size_t>(S) * H * 4},
      {&m->xn, static_cast<std::size_t>(S) * H * 4},
      {&m->xq, static_cast<std::size_t>(S) * H},
      {&m->xs, static_cast<std::size_t>(S) * H / 8},
      {&m->qkv, static_cast<std::size_t>(S) * C * 4},
      {&m->zo, static_cast<std::size_t>(S) * Dv * 4},
      {&m->abo, static_cast<std::size_t>(S) * 2 * Hv * 4},
      {&m->q, static_cast<std::size_t>(S) * std::max(Hk * d, Hq * hd) * 4},
      {&m->k, static_cast<std::size_t>(S) * Hk * d * 4},
      {&m->v, static_cast<std::size_t>(S) * Dv * 4},
      {&m->g, S * Hv * 4},
      {&m->beta, S * Hv * 4},
      {&m->o, static_cast<std::size_t>(S) * Dv * 4},
      {&m->oq, static_cast<std::size_t>(S) * std::max(Dv, Hq * hd)},
      {&m->os, static_cast<std::size_t>(S) * std::max(Dv, Hq * hd) / 8},
      {&m->delta, static_cast<std::size_t>(S) * H * 4},
      {&m->qgo, static_cast<std::size_t>(S) * 2 * Hq * hd * 4},
      {&m->ko, static_cast<std::size_t>(S) * Hkv * hd * 4},
      {&m->vo, static_cast<std::size_t>(S) * Hkv * hd * 4},
      {&m->agate, static_cast<std::size_t>(S) * Hq * hd * 4},
      {&m->ao, static_cast<std::size_t>(S) * Hq * hd * 4},
      {&m->logits, static_cast<std::size_t>(S) * c.vocab * 4},
      {&m->argmax_part, static_cast<std::size_t>(S) * 64 * 8},
  };
  for (const auto& b : bufs)
    if (Alloc(m.get(), b.bytes, b.b, err, errlen) != 0) return -1;
  m->moe_ws_bytes = halo_op_moe_workspace_bytes(&m->layers[0].moe, S);
  std::size_t aw = 0;
  for (std::uint32_t s = 1; s <= S; ++s)
    for (std::uint32_t pre : {0u, c.prefix_tokens}) {
      halo_paged_kv kv{};
      kv.k_pool = reinterpret_cast<float*>(1);
      kv.v_pool = kv.k_pool;
      kv.pages = reinterpret_cast<const uint32_t*>(1);
      kv.nkv = kv.pages;
      kv.sessions = s;
      kv.kv_heads = Hkv;
      kv.head_dim = hd;
      kv.max_pages = m->max_pages;
      kv.prefix = pre;
      kv.max_context = c.max_context;
      aw = std::max(aw, halo_op_attn_decode_workspace_bytes(&kv, Hq));
    }
  m->attn_ws_bytes = aw;
  if (m->moe_ws_bytes == 0 || Alloc(m.get(), m->moe_ws_bytes, &m->moe_ws, err, errlen) != 0 ||
      Alloc(m.get(), aw, &m->attn_ws, err, errlen) != 0)
    return SetErr(err, errlen, "model: workspace sizing failed"), -1;
  // page tables: [0, prefix_pages) shared, the rest per session
  std::vector<std::uint32_t> pt(static_cast<std::size_t>(S) * m->max_pages);
  std::uint32_t nextp = m->prefix_pages;
  for (std::uint32_t s = 0; s < S; ++s)
    for (std::uint32_t p = 0; p < m->max_pages; ++p)
      pt[static_cast<std::size_t>(s) * m->max_pages + p] = p < m->prefix_pages ? p : nextp++;
  if (halo_upload(m->dev, &m->pages, 0, pt.data(), pt.size() * 4, err, errlen) != 0) return -1;
  if (halo_model_reset(m.get(), err, errlen) != 0) return -1;
  if (halo_synchronize(m->dev, err, errlen) != 0) return -1;
  *out = m.release();
  return 0;
}

void halo_model_destroy(halo_model* m) {
  if (m == nullptr) return;
  (void)halo_synchronize(m->dev, nullptr, 0);
  for (auto& [key, g] : m->graphs) halo_free_graph(m->dev, &g);
  for (auto& b : m->owned) halo_free(m->dev, &b);
  delete m;
}

uint64_t halo_model_weight_bytes(const halo_model* m) { return m ? m->weight_bytes : 0; }
uint64_t halo_model_device_bytes(const halo_model* m) { return m ? m->device_bytes : 0; }

int halo_model_reset(halo_model* m, char* err, size_t errlen) {
  for (halo_buffer* b : {&m->gdn_state, &m->conv_state, &m->nkv, &m->tokens, &m->prompt_len, &m->history})
    if (halo_fill(m->dev, b, 0, err, errlen) != 0) return -1;
  return 0;
}

int halo_model_set_sampling(halo_model* m, uint32_t s, const HaloSampleParams* params, const HaloPenalty* penalties,
                            uint32_t n_penalties, char* err, size_t errlen) {
  if (m == nullptr || s >= m->c.max_sessions || params == nullptr || (n_penalties && penalties == nullptr))
    return SetErr(err, errlen, "set_sampling: bad session %u or null argument", s), -1;
  const HaloSampleParams& p = *params;
  if (!std::isfinite(p.temperature) || p.temperature < 0.0f || !(p.top_p >= 0.0f && p.top_p <= 1.0f) ||
      !(p.min_p >= 0.0f && p.min_p <= 1.0f) || !std::isfinite(p.repeat_penalty) || !(p.repeat_penalty > 0.0f) ||
      !std::isfinite(p.frequency_penalty) || !std::isfinite(p.presence_penalty) || p.top_k > 0x7FFFFFFFu ||
      n_penalties > HALO_SAMPLE_MAX_PENALTIES)
    return SetErr(err, errlen, "set_sampling: parameters outside the sampler's ranges"), -1;
  for (std::uint32_t i = 0; i < n_penalties; ++i)
    if (penalties[i].token >= m->c.vocab || (i && penalties[i].token <= penalties[i - 1].token))
      return SetErr(err, errlen, "set_sampling: penalty tokens must be below the vocabulary and strictly increasing"),
             -1;
  const std::uint32_t S = m->c.max_sessions;
  if (m->sample_params.device == nullptr) {
    const std::size_t ws = halo_op_sample_workspace_bytes(S, m->c.vocab);
    if (Alloc(m, sizeof(HaloSampleParams) * S, &m->sample_params, err, errlen) != 0 ||
        Alloc(m, sizeof(HaloPenalty) * HALO_SAMPLE_MAX_PENALTIES * S, &m->sample_pen, err, errlen) != 0 ||
        Alloc(m, sizeof(HaloSampleOut) * S, &m->sample_out, err, errlen) != 0 ||
        Alloc(m, ws, &m->sample_ws, err, errlen) != 0)
      return -1;
    // every session starts greedy
    std::vector<HaloSampleParams> g(S);
    for (auto& q : g) {
      q = HaloSampleParams{};
      q.top_p = 1.0f;
      q.repeat_penalty = 1.0f;
      q.vocab = m->c.vocab;
    }
    if (halo_upload(m->dev, &m->sample_params, 0, g.data(), sizeof(HaloSampleParams) * S, err, errlen) != 0)
      return -1;
  }
  HaloSampleParams q = p;
  q.vocab = m->c.vocab;
  q.n_penalties = n_penalties;
  if (halo_upload(m->dev, &m->sample_params, sizeof(HaloSampleParams) * s, &q, sizeof q, err, errlen) != 0) return -1;
  if (n_penalties &&
      halo_upload(m->dev, &m->sample_pen, sizeof(HaloPenalty) * HALO_SAMPLE_MAX_PENALTIES * s, penalties,
                  sizeof(HaloPenalty) * n_penalties, err, errlen) != 0)
    return -1;
  m->sampling = true;
  return 0;
}

int halo_model_sample_state(halo_model* m, uint32_t s, HaloSampleParams* params, char* err, size_t errlen) {
  if (m == nullptr || params == nullptr || s >= m->c.max_sessions || m->sample_params.device == nullptr)
    return SetErr(err, errlen, "sample_state: no sampling set for session %u", s), -1;
  return halo_download(m->dev, &m->sample_params, sizeof(HaloSampleParams) * s, params, sizeof *params, err, errlen);
}

int halo_model_set_session(halo_model* m, uint32_t s, const uint32_t* prompt, uint32_t len, uint32_t nkv, char* err,
                           size_t errlen) {
  if (s >= m->c.max_sessions || len > m->c.max_context || (len ? nkv >= len : nkv != 0) || nkv >= m->c.max_context)
    return SetErr(err, errlen, "session %u: prompt %u / position %u out of range", s, len, nkv), -1;
  for (std::uint32_t i = 0; i < len; ++i)
    if (prompt[i] >= m->c.vocab) return SetErr(err, errlen, "session %u: token %u out of range", s, prompt[i]), -1;
  const std::size_t stride = m->c.max_context;
  if (len && halo_upload(m->dev, &m->prompt, static_cast<std::size_t>(s) * stride * 4, prompt, len * 4ull, err,
                         errlen) != 0)
    return -1;
  const std::uint32_t first = len ? prompt[nkv] : 0;
  if (halo_upload(m->dev, &m->prompt_len, s * 4ull, &len, 4, err, errlen) != 0 ||
      halo_upload(m->dev, &m->nkv, s * 4ull, &nkv, 4, err, errlen) != 0 ||
      halo_upload(m->dev, &m->tokens, s * 4ull, &first, 4, err, errlen) != 0)
    return -1;
  // the first step reads token nkv and writes position nkv: nkv counts it
  const std::uint32_t n1 = nkv + 1;
  return halo_upload(m->dev, &m->nkv, s * 4ull, &n1, 4, err, errlen);
}

int halo_model_fork(halo_model* m, uint32_t src, uint32_t dst, char* err, size_t errlen) {
  const halo_model_config& c = m->c;
  if (src >= c.max_sessions || dst >= c.max_sessions) return SetErr(err, errlen, "fork: bad session"), -1;
  const std::size_t st = static_cast<std::size_t>(c.gdn_v_heads) * c.gdn_head_dim * c.gdn_head_dim * 4;
  const std::size_t cv = static_cast<std::size_t>(c.conv_kernel) * m->conv_ch * 4;
  for (std::uint32_t l = 0; l < m->n_gdn; ++l) {
    const std::size_t base = static_cast<std::size_t>(l) * c.max_sessions;
    char* sp = P<char>(m->gdn_state);
    char* cp = P<char>(m->conv_state);
    const halo_arg a[] = {Ptr(sp + (base + src) * st), Ptr(sp + (base + dst) * st), Val<std::uint64_t>(st / 16)};
    if (Launch(m->eng, "halo_copy16", D3(1024), D3(256), a, err, errlen) != 0) return -1;
    if (cv) {
      const halo_arg b[] = {Ptr(cp + (base + src) * cv), Ptr(cp + (base + dst) * cv), Val<std::uint64_t>(cv / 16)};
      if (Launch(m->eng, "halo_copy16", D3(64), D3(256), b, err, errlen) != 0) return -1;
    }
  }
  return 0;
}

int halo_model_step_eager(halo_model* m, uint32_t S, uint32_t prefix, char* err, size_t errlen) {
  if (S == 0 || S > m->c.max_sessions || prefix % 64 != 0 || prefix > m->c.prefix_tokens)
    return SetErr(err, errlen, "step: %u sessions / prefix %u unsupported", S, prefix), -1;
  return Record(m, S, prefix, err, errlen);
}

int halo_model_step_trace(halo_model* m, uint32_t S, uint32_t prefix, void* trace, size_t trace_bytes,
                          halo_model_trace_entry* entries, uint32_t max_entries, uint32_t* n_entries, char* err,
                          size_t errlen) {
  if (m == nullptr || trace == nullptr || entries == nullptr || n_entries == nullptr)
    return SetErr(err, errlen, "trace: null argument"), -1;
  if (S == 0 || S > m->c.max_sessions || prefix % 64 != 0 || prefix > m->c.prefix_tokens)
    return SetErr(err, errlen, "trace: %u sessions / prefix %u unsupported", S, prefix), -1;
  Tracer tr;
  tr.eng = m->eng;
  tr.base = static_cast<char*>(trace);
  tr.cap = trace_bytes;
  tr.entries = entries;
  tr.max_entries = max_entries;
  const int rc = Record(m, S, prefix, err, errlen, &tr);
  *n_entries = tr.n;
  return rc;
}

int halo_model_run(halo_model* m, uint32_t S, uint32_t prefix, uint32_t steps, char* err, size_t errlen) {
  if (S == 0 || S > m->c.max_sessions || prefix % 64 != 0 || prefix > m->c.prefix_tokens)
    return SetErr(err, errlen, "run: %u sessions / prefix %u unsupported", S, prefix), -1;
  const auto key = std::make_tuple(S, prefix, m->sampling);
  auto it = m->graphs.find(key);
  if (it == m->graphs.end()) {
    if (halo_begin_capture(m->dev, err, errlen) != 0) return -1;
    const int rc = Record(m, S, prefix, err, errlen);
    halo_graph g{};
    char e2[256];
    const int rc2 = halo_end_capture(m->dev, &g, e2, sizeof e2);
    if (rc != 0) return -1;
    if (rc2 != 0) return SetErr(err, errlen, "%s", e2), -1;
    it = m->graphs.emplace(key, g).first;
  }
  for (std::uint32_t i = 0; i < steps; ++i)
    if (halo_launch_graph(m->dev, &it->second, err, errlen) != 0) return -1;
  return 0;
}

int halo_model_tensor(const halo_model* m, uint32_t layer, const char* name, halo_model_tensor_view* out, char* err,
                      size_t errlen) {
  if (m == nullptr || name == nullptr || out == nullptr) return SetErr(err, errlen, "null argument"), -1;
  *out = halo_model_tensor_view{};
  const std::string n(name);
  auto f32 = [&](const halo_buffer& b, std::uint32_t rows, std::uint32_t cols) {
    if (b.device == nullptr) return SetErr(err, errlen, "tensor %s absent in layer %u", name, layer), -1;
    *out = halo_model_tensor_view{b.device, nullptr, HALO_TENSOR_F32, rows, cols, cols};
    return 0;
  };
  auto f32Raw = [&](void* p, std::uint32_t rows, std::uint32_t cols) {
    *out = halo_model_tensor_view{p, nullptr, HALO_TENSOR_F32, rows, cols, cols};
    return 0;
  };
  auto q8 = [&](const Q8& w) {
    if (w.qs.device == nullptr) return SetErr(err, errlen, "tensor %s absent in layer %u", name, layer), -1;
    *out = halo_model_tensor_view{w.qs.device, w.d.device, HALO_TENSOR_Q8, w.m.rows, w.m.cols, w.m.qstride};
    return 0;
  };
  const halo_model_config& c = m->c;
  if (layer == UINT32_MAX) {
    if (n == "embd") return q8(m->embd);
    if (n == "head") return q8(m->head);
    if (n == "out_norm") return f32(m->out_norm, 1, c.hidden);
    // page tables [max_sessions][max_pages] and positions [max_sessions], uint32 (viewed as 4-byte words)
    if (n == "pages") return f32(m->pages, c.max_sessions, m->max_pages);
    if (n == "nkv") return f32(m->nkv, 1, c.max_sessions);
    return SetErr(err, errlen, "unknown tensor %s", name), -1;
  }
  if (layer >= m->layers.size()) return SetErr(err, errlen, "layer %u out of range", layer), -1;
  const Layer& L = m->layers[layer];
  const std::uint32_t H = c.hidden, Hv = c.gdn_v_heads, d = c.gdn_head_dim, hd = c.head_dim;
  // recurrent state and caches (parity instrumentation): DeltaNet state [max_sessions][Hv][d][d] key-major and the
  // conv ring [max_sessions][K][C] (position p's projection in slot p % K); attention KV pools [pages][Hkv][16][hd]
  if (!L.attn && n == "state")
    return f32Raw(P<float>(m->gdn_state) + static_cast<std::size_t>(L.gdn_index) * c.max_sessions * Hv * d * d,
                  c.max_sessions * Hv * d, d);
  if (!L.attn && n == "conv_ring")
    return f32Raw(P<float>(m->conv_state) + static_cast<std::size_t>(L.gdn_index) * c.max_sessions *
                                                c.conv_kernel * m->conv_ch,
                  c.max_sessions * c.conv_kernel, m->conv_ch);
  if (L.attn && n == "k_pool") return f32(L.k_pool, m->total_pages * c.kv_heads * 16, hd);
  if (L.attn && n == "v_pool") return f32(L.v_pool, m->total_pages * c.kv_heads * 16, hd);
  if (n == "attn_norm") return f32(L.attn_norm, 1, H);
  if (n == "ffn_norm") return f32(L.ffn_norm, 1, H);
  if (n == "router") return f32(L.router, c.n_experts, H);
  if (n == "shared_gate") return f32(L.shared_gate, 1, H);
  if (n == "gate") return q8(L.gate);
  if (n == "up") return q8(L.up);
  if (n == "down") return q8(L.down);
  if (n == "sgate") return q8(L.sgate);
  if (n == "sup") return q8(L.sup);
  if (n == "sdown") return q8(L.sdown);
  if (!L.attn) {
    if (n == "qkv") return q8(L.qkv);
    if (n == "z") return q8(L.z);
    if (n == "ab") return q8(L.ab);
    if (n == "out") return q8(L.out);
    if (n == "conv_w") return f32(L.conv_w, m->conv_ch, c.conv_kernel);
    if (n == "a") return f32(L.a, 1, Hv);
    if (n == "dt") return f32(L.dt, 1, Hv);
    if (n == "norm_w") return f32(L.norm_w, 1, d);
  } else {
    if (n == "qg") return q8(L.qg);
    if (n == "k") return q8(L.k);
    if (n == "v") return q8(L.v);
    if (n == "o") return q8(L.o);
    if (n == "q_norm") return f32(L.q_norm, 1, hd);
    if (n == "k_norm") return f32(L.k_norm, 1, hd);
  }
  return SetErr(err, errlen, "unknown tensor %s for layer %u", name, layer), -1;
}

int halo_model_logits(halo_model* m, uint32_t s, float* out, char* err, size_t errlen) {
  if (m == nullptr || out == nullptr || s >= m->c.max_sessions) return SetErr(err, errlen, "bad session"), -1;
  return halo_download(m->dev, &m->logits, static_cast<std::size_t>(s) * m->c.vocab * 4, out, m->c.vocab * 4ull, err,
                       errlen);
}

int halo_model_prefill(halo_model* m, const halo_prefill_segment* segs, uint32_t nseg, char* err, size_t errlen) {
  if (m == nullptr || segs == nullptr || nseg == 0 || nseg > m->c.max_sessions)
    return SetErr(err, errlen, "prefill: 1..%u segments", m ? m->c.max_sessions : 0), -1;
  for (std::uint32_t i = 0; i < nseg; ++i) {
    const halo_prefill_segment& g = segs[i];
    if (g.session != segs[0].session + i)
      return SetErr(err, errlen, "prefill: segment sessions must be consecutive (s0, s0 + 1, ...)"), -1;
    if (g.length == 0 || g.start + g.length >= m->c.max_context)
      return SetErr(err, errlen, "prefill: segment %u (%u + %u) outside the context", i, g.start, g.length), -1;
  }
  if (PrefillAlloc(m, err, errlen) != 0) return -1;
  // batches of at most the prefill batch cap tokens; a long segment continues in the next batch
  std::vector<halo_prefill_segment> rest(segs, segs + nseg);
  while (!rest.empty()) {
    std::vector<halo_prefill_segment> batch, next;
    std::uint32_t room = PrefillCap(m->c);
    for (auto& g : rest) {
      const std::uint32_t n = std::min(g.length, room);
      if (n > 0) batch.push_back(halo_prefill_segment{g.session, g.start, n, 0});
      if (n < g.length) next.push_back(halo_prefill_segment{g.session, g.start + n, g.length - n, 0});
      room -= n;
    }
    // sessions of a batch must stay consecutive: a batch that could not take every segment is cut at the first
    // missing one
    std::vector<halo_prefill_segment> ok;
    for (const auto& g : batch) {
      if (!ok.empty() && g.session != ok.back().session + 1) break;
      ok.push_back(g);
    }
    if (ok.size() < batch.size()) {
      next.clear();
      for (const auto& g : rest) {
        const auto it = std::find_if(ok.begin(), ok.end(), [&](const halo_prefill_segment& o) { return o.session == g.session; });
        if (it == ok.end()) next.push_back(g);
        else if (it->length < g.length) next.push_back(halo_prefill_segment{g.session, g.start + it->length, g.length - it->length, 0});
      }
    }
    if (PrefillBatch(m, ok, err, errlen) != 0) return -1;
    rest.swap(next);
  }
  return 0;
}

int halo_model_prefill_trace(halo_model* m, const halo_prefill_segment* segs, uint32_t nseg, void* trace,
                             size_t trace_bytes, halo_model_trace_entry* entries, uint32_t max_entries,
                             uint32_t* n_entries, char* err, size_t errlen) {
  return halo_model_prefill_trace_layers(m, segs, nseg, ~std::uint64_t{0}, trace, trace_bytes, entries, max_entries,
                                         n_entries, err, errlen);
}

int halo_model_prefill_trace_layers(halo_model* m, const halo_prefill_segment* segs, uint32_t nseg,
                                    uint64_t layer_mask, void* trace, size_t trace_bytes,
                                    halo_model_trace_entry* entries, uint32_t max_entries, uint32_t* n_entries,
                                    char* err, size_t errlen) {
  if (m == nullptr || segs == nullptr || trace == nullptr || entries == nullptr || n_entries == nullptr ||
      nseg == 0 || nseg > m->c.max_sessions)
    return SetErr(err, errlen, "prefill trace: null argument or bad segment count"), -1;
  std::uint32_t total = 0;
  for (std::uint32_t i = 0; i < nseg; ++i) {
    const halo_prefill_segment& g = segs[i];
    if (g.session != segs[0].session + i || g.length == 0 || g.start + g.length >= m->c.max_context)
      return SetErr(err, errlen, "prefill trace: segment %u invalid", i), -1;
    total += g.length;
  }
  if (total > PrefillCap(m->c))
    return SetErr(err, errlen, "prefill trace: %u tokens > one batch of %u", total, PrefillCap(m->c)), -1;
  if (m->c.shared_ff != m->c.expert_ff) return SetErr(err, errlen, "prefill trace: shared ff != expert ff"), -1;
  if (PrefillAlloc(m, err, errlen) != 0) return -1;
  if (m->c.layers > 63 && layer_mask != ~std::uint64_t{0})
    return SetErr(err, errlen, "prefill trace: a layer mask needs at most 63 layers"), -1;
  Tracer tr;
  tr.eng = m->eng;
  tr.base = static_cast<char*>(trace);
  tr.cap = trace_bytes;
  tr.entries = entries;
  tr.max_entries = max_entries;
  tr.mask = layer_mask;
  std::vector<halo_prefill_segment> batch(segs, segs + nseg);
  for (auto& g : batch) g.first = 0;
  const int rc = PrefillBatch(m, batch, err, errlen, &tr);
  *n_entries = tr.n;
  return rc;
}

int halo_model_history(halo_model* m, uint32_t s, uint32_t* out, uint32_t n, char* err, size_t errlen) {
  if (s >= m->c.max_sessions || n > m->c.max_context) return SetErr(err, errlen, "history: bad range"), -1;
  return halo_download(m->dev, &m->history, static_cast<std::size_t>(s) * m->c.max_context * 4, out, n * 4ull, err,
                       errlen);
}

int halo_model_positions(halo_model* m, uint32_t* nkv_out, uint32_t S, char* err, size_t errlen) {
  if (S > m->c.max_sessions) return SetErr(err, errlen, "positions: bad count"), -1;
  return halo_download(m->dev, &m->nkv, 0, nkv_out, S * 4ull, err, errlen);
}

}  // extern "C"

halo_engine* halo_model_engine_of(const halo_model* m) { return m->eng; }
