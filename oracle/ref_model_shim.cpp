// Test infrastructure only: a C shim over the reference's own ReferenceModel layer functions (LinearAttention,
// Attention, Moe; src/model/reference.cpp:278-578), compiled from the reference's source where it lies, so the host
// restatement of the synthetic model's layers can be pinned against the reference's code. The layer functions are
// private members; this translation unit includes reference.cpp itself with `private` widened to `public` (layout is
// unchanged; nothing here is shipped). One layer at a time: a Config with one layer of the requested kind, weights
// given as raw GGUF Q8_0 blocks (projections, stacked experts) or fp32 (router, norms, conv taps, gates), state in
// the reference's own layouts. Storage::kFloat32: projections are cpu::MatVec over fp32 activations.
// Every header but reference.hpp first, so that only ReferenceModel sees the widened access.
#include <algorithm>
#include <array>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <map>
#include <memory>
#include <numeric>
#include <optional>
#include <set>
#include <span>
#include <sstream>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "core/quant.hpp"
#include "model/cpu_ops.hpp"
#include "model/lora.hpp"
#include "model/ngram.hpp"
#include "model/weights.hpp"

#define private public
#include "model/reference.cpp"
#undef private

#include <cstring>
#include <vector>

using halo::core::GgmlType;
using halo::model::Config;
using halo::model::LayerWeights;
using halo::model::ModelWeights;
using halo::model::ReferenceModel;
using halo::model::TensorRef;

namespace {

TensorRef Q8(const void* raw, std::uint64_t rows, std::uint64_t cols, std::uint64_t experts = 1) {
  TensorRef t;
  t.data = raw;
  t.type = GgmlType::kQ8_0;
  t.rows = rows;
  t.cols = cols;
  t.experts = experts;
  return t;
}
TensorRef F32(const float* p, std::uint64_t rows, std::uint64_t cols) {
  TensorRef t;
  t.data = p;
  t.type = GgmlType::kF32;
  t.rows = rows;
  t.cols = cols;
  return t;
}

// Shapes shared by the entry points (the synthetic model's; no hyper-connections, no PLE).
struct Shape {
  std::uint32_t hidden, k_heads, v_heads, head_dim, conv_kernel;  // DeltaNet
  std::uint32_t q_heads, kv_heads, attn_head_dim, rotary_dim;      // attention
  float rope_theta, rms_eps;
  std::uint32_t n_experts, n_used, expert_ff, shared_ff;          // MoE
};

Config MakeConfig(const Shape& s, bool linear) {
  Config c;
  c.num_layers = 1;
  c.num_layers_all = 1;
  c.hidden_size = s.hidden;
  c.vocab_size = 1;
  c.context_length = 1 << 20;
  c.rms_eps = s.rms_eps;
  c.hc_count = 1;
  c.full_attention_interval = linear ? 2 : 1;  // layer 0 is linear iff (0 + 1) % interval != 0
  c.num_heads = s.q_heads;
  c.num_kv_heads = s.kv_heads;
  c.head_dim = s.attn_head_dim;
  c.rotary_dim = s.rotary_dim;
  c.rope_theta = s.rope_theta;
  // the QSA indexer keeps every position visible: its block budget exceeds any context used here
  c.indexer_heads = 1;
  c.indexer_head_dim = s.rotary_dim;
  c.indexer_top_k = 1u << 30;
  c.compress_ratio = 4;
  c.ssm_conv_kernel = s.conv_kernel;
  c.ssm_head_dim = s.head_dim;
  c.ssm_num_k_heads = s.k_heads;
  c.ssm_num_v_heads = s.v_heads;
  c.ssm_inner_size = s.v_heads * s.head_dim;
  c.num_experts = s.n_experts;
  c.num_experts_used = s.n_used;
  c.expert_ff = s.expert_ff;
  c.shared_expert_ff = s.shared_ff;
  return c;
}

}  // namespace

extern "C" {

// One ReferenceModel::LinearAttention call. qkv/z/alpha/beta/out: raw Q8_0 [rows][hidden] (out [hidden][v dim]);
// conv_w fp32 [channels][kern]; a, dt fp32 [v_heads]; norm fp32 [head_dim]. conv [kern-1][channels] (oldest first)
// and state [v_heads][d][d] (S[h][j][i], j value, i key) in place; x [hidden]; y [hidden].
void ref_linear_attention(const std::uint32_t* shape_u, const float* shape_f, const void* qkv, const void* z,
                          const void* alpha, const void* beta, const void* out_w, const float* conv_w, const float* a,
                          const float* dt, const float* norm, float* conv, float* state, const float* x, float* y) {
  Shape s{shape_u[0], shape_u[1], shape_u[2], shape_u[3], shape_u[4], 0, 0, 0, 0, 0.0f, shape_f[0], 0, 0, 0, 0};
  ModelWeights w;
  w.config = MakeConfig(s, true);
  const Config& c = w.config;
  LayerWeights l;
  l.linear = true;
  const std::uint32_t C = c.SsmConvChannels(), Dv = c.SsmValueDim();
  l.ssm_qkv = Q8(qkv, C, s.hidden);
  l.ssm_gate = Q8(z, Dv, s.hidden);
  l.ssm_alpha = Q8(alpha, s.v_heads, s.hidden);
  l.ssm_beta = Q8(beta, s.v_heads, s.hidden);
  l.ssm_out = Q8(out_w, s.hidden, Dv);
  l.ssm_conv1d = F32(conv_w, C, s.conv_kernel);
  l.ssm_a = F32(a, 1, s.v_heads);
  l.ssm_dt = F32(dt, 1, s.v_heads);
  l.ssm_norm = F32(norm, 1, s.head_dim);
  w.layers.push_back(l);
  ReferenceModel m(w, nullptr, 16);
  auto& st = m.linear_[0];
  std::memcpy(st.conv.data(), conv, st.conv.size() * sizeof(float));
  std::memcpy(st.state.data(), state, st.state.size() * sizeof(float));
  m.LinearAttention(w.layers[0], st, std::span<const float>(x, s.hidden), std::span<float>(y, s.hidden));
  std::memcpy(conv, st.conv.data(), st.conv.size() * sizeof(float));
  std::memcpy(state, st.state.data(), st.state.size() * sizeof(float));
}

// ReferenceModel::Attention over `steps` consecutive positions 0 .. steps-1 (inputs x [steps][hidden], outputs
// y [steps][hidden]), all positions visible. q: raw Q8_0 [q_heads * 2 * hd][hidden] (q | gate per head), k, v
// [kv_heads * hd][hidden], o [hidden][q_heads * hd]; q_norm, k_norm fp32 [hd].
void ref_attention(const std::uint32_t* shape_u, const float* shape_f, const void* q, const void* k, const void* v,
                   const void* o, const float* q_norm, const float* k_norm, const float* x, float* y,
                   std::uint32_t steps) {
  Shape s{shape_u[0], 0, 0, 0, 0, shape_u[1], shape_u[2], shape_u[3], shape_u[4], shape_f[1], shape_f[0],
          0, 0, 0, 0};
  ModelWeights w;
  w.config = MakeConfig(s, false);
  const Config& c = w.config;
  LayerWeights l;
  const std::uint32_t hd = s.attn_head_dim;
  l.attn_q = Q8(q, 2 * c.AttentionQDim(), s.hidden);
  l.attn_k = Q8(k, c.AttentionKvDim(), s.hidden);
  l.attn_v = Q8(v, c.AttentionKvDim(), s.hidden);
  l.attn_out = Q8(o, s.hidden, c.AttentionQDim());
  l.attn_q_norm = F32(q_norm, 1, hd);
  l.attn_k_norm = F32(k_norm, 1, hd);
  // the indexer's projections are unused for visibility (every position is visible); zeros
  std::vector<float> zeros(static_cast<std::size_t>(s.hidden) * c.indexer_head_dim, 0.0f);
  std::vector<float> ones(c.indexer_head_dim, 1.0f);
  l.indexer_q = F32(zeros.data(), c.indexer_head_dim, s.hidden);
  l.indexer_k = F32(zeros.data(), c.indexer_head_dim, s.hidden);
  l.indexer_q_norm = F32(ones.data(), 1, c.indexer_head_dim);
  l.indexer_k_norm = F32(ones.data(), 1, c.indexer_head_dim);
  w.layers.push_back(l);
  ReferenceModel m(w, nullptr, steps + 1);
  for (std::uint32_t t = 0; t < steps; ++t)
    m.Attention(w.layers[0], m.attention_[0], std::span<const float>(x + static_cast<std::size_t>(t) * s.hidden,
                                                                      s.hidden),
                t, std::span<float>(y + static_cast<std::size_t>(t) * s.hidden, s.hidden));
}

// ReferenceModel::Moe for one token. router fp32 [E][hidden]; gate, up raw Q8_0 stacked [E][ff][hidden], down
// [E][hidden][ff]; shared gate_inp fp32 [hidden]; shared gate / up [sff][hidden], down [hidden][sff].
void ref_moe(const std::uint32_t* shape_u, const float* router, const void* gate, const void* up, const void* down,
             const float* sgate_inp, const void* sgate, const void* sup, const void* sdown, const float* x, float* y) {
  Shape s{shape_u[0], 0, 0, 0, 0, 0, 0, 0, 0, 0.0f, 1e-6f, shape_u[1], shape_u[2], shape_u[3], shape_u[4]};
  ModelWeights w;
  w.config = MakeConfig(s, true);
  LayerWeights l;
  l.router = F32(router, s.n_experts, s.hidden);
  l.ffn_gate_exps = Q8(gate, s.expert_ff, s.hidden, s.n_experts);
  l.ffn_up_exps = Q8(up, s.expert_ff, s.hidden, s.n_experts);
  l.ffn_down_exps = Q8(down, s.hidden, s.expert_ff, s.n_experts);
  l.shexp_gate_inp = F32(sgate_inp, 1, s.hidden);
  l.shexp_gate = Q8(sgate, s.shared_ff, s.hidden);
  l.shexp_up = Q8(sup, s.shared_ff, s.hidden);
  l.shexp_down = Q8(sdown, s.hidden, s.shared_ff);
  w.layers.push_back(l);
  ReferenceModel m(w, nullptr, 4);
  m.Moe(w.layers[0], std::span<const float>(x, s.hidden), std::span<float>(y, s.hidden));
}

}  // extern "C"
