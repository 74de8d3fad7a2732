// C entry points over the reference's own CPU code (casselc/halo-flash src/core/quant.cpp,
// src/model/cpu_ops.cpp), compiled from the sources where they lie by oracle/Makefile into oracle/_ref/.
// TEST INFRASTRUCTURE ONLY: used to validate the C restatement in oracle.c and, in bench.py's cpu_baseline leg,
// as the timed reference CPU path. Nothing here is linked into the product library.
#include <cstdint>
#include <cstring>
#include <cstdio>
#include <string>
#include <variant>
#include <span>
#include <thread>

#include "core/gguf.hpp"
#include "core/quant.hpp"
#include "core/sampling.hpp"
#include "model/cpu_ops.hpp"
#include "model/weights.hpp"

using halo::core::GgmlType;
using halo::model::TensorRef;

extern "C" {

float ref_fp16_to_f32(std::uint16_t h) { return halo::quant::Fp16ToFloat(h); }

void ref_dequant_q8_0(const void* blocks, float* out, std::size_t k) { halo::quant::DequantizeQ8_0(blocks, out, k); }

float ref_dot_q8_0(const void* blocks, const float* x, std::size_t k) {
  return halo::quant::DotProductQ8_0(blocks, std::span<const float>(x, k), k);
}

// cpu::MatVec over a raw GGUF Q8_0 matrix (rows x cols, 34-byte blocks); threads as the reference picks them.
void ref_matvec_q8_0(const void* raw, std::uint64_t rows, std::uint64_t cols, const float* x, float* y) {
  TensorRef t;
  t.data = raw;
  t.type = GgmlType::kQ8_0;
  t.rows = rows;
  t.cols = cols;
  halo::model::cpu::MatVec(t, 0, std::span<const float>(x, cols), std::span<float>(y, rows));
}

void ref_matvec_f32(const float* w, std::uint64_t rows, std::uint64_t cols, const float* x, float* y) {
  TensorRef t;
  t.data = w;
  t.type = GgmlType::kF32;
  t.rows = rows;
  t.cols = cols;
  halo::model::cpu::MatVec(t, 0, std::span<const float>(x, cols), std::span<float>(y, rows));
}

void ref_route_topk(const float* logits, std::uint32_t n, std::uint32_t k, std::uint32_t* ids, float* w) {
  halo::model::cpu::RouteTopK(std::span<const float>(logits, n), std::span<std::uint32_t>(ids, k),
                              std::span<float>(w, k));
}

void ref_rmsnorm(float* x, std::size_t n, const float* w, float eps) {
  halo::model::cpu::RmsNorm(std::span<float>(x, n), w, eps);
}
void ref_l2norm(float* x, std::size_t n, float eps) { halo::model::cpu::L2Norm(std::span<float>(x, n), eps); }
void ref_rope(float* x, std::uint32_t heads, std::uint32_t hd, std::uint32_t rot, std::uint32_t pos, float theta) {
  halo::model::cpu::Rope(x, heads, hd, rot, pos, theta);
}
float ref_silu(float x) { return halo::model::cpu::Silu(x); }
float ref_sigmoid(float x) { return halo::model::cpu::Sigmoid(x); }
float ref_softplus(float x) { return halo::model::cpu::Softplus(x); }
unsigned ref_hw_threads() { return std::thread::hardware_concurrency(); }

// One draw of the reference's sampler: BuildDistribution (penalties from the prompt and generated token lists)
// then Sample with the given RNG state (advanced in place). Returns the token, 0xFFFFFFFF on an exception.
std::uint32_t ref_sample(const float* logits, std::uint32_t n, float temperature, std::int32_t top_k, float top_p,
                         float min_p, std::uint32_t min_keep, float repeat_penalty, std::uint32_t repeat_last_n,
                         float frequency_penalty, float presence_penalty, const std::uint32_t* prompt,
                         std::uint32_t n_prompt, const std::uint32_t* generated, std::uint32_t n_gen,
                         std::uint64_t* rng) {
  halo::sampling::SamplingConfig c;
  c.temperature = temperature;
  c.top_k = top_k;
  c.top_p = top_p;
  c.min_p = min_p;
  c.min_keep = min_keep;
  c.seed = 0;
  c.repeat_penalty = repeat_penalty;
  c.repeat_last_n = repeat_last_n;
  c.frequency_penalty = frequency_penalty;
  c.presence_penalty = presence_penalty;
  try {
    const auto d = halo::sampling::BuildDistribution(std::span<const float>(logits, n), c,
                                                     std::span<const std::uint32_t>(prompt, n_prompt),
                                                     std::span<const std::uint32_t>(generated, n_gen));
    return d.Sample(rng);
  } catch (...) {
    return 0xFFFFFFFFu;
  }
}

// SamplerState (sampling.cpp:407-415, 467-563): history = prompt, then the generated tokens accepted; its penalty
// list is written out (token, generated_count, repeated; at most cap entries) and one Sample drawn from `rng`.
std::uint32_t ref_sampler_state(const float* logits, std::uint32_t n, float temperature, std::int32_t top_k,
                                float top_p, float min_p, std::uint32_t min_keep, float repeat_penalty,
                                std::uint32_t repeat_last_n, float frequency_penalty, float presence_penalty,
                                const std::uint32_t* prompt, std::uint32_t n_prompt, const std::uint32_t* generated,
                                std::uint32_t n_gen, std::uint64_t* rng, std::uint32_t* pen_token,
                                std::uint32_t* pen_generated, std::uint32_t* pen_repeated, std::uint32_t cap,
                                std::uint32_t* n_pen) {
  halo::sampling::SamplingConfig c;
  c.temperature = temperature;
  c.top_k = top_k;
  c.top_p = top_p;
  c.min_p = min_p;
  c.min_keep = min_keep;
  c.seed = 0;
  c.repeat_penalty = repeat_penalty;
  c.repeat_last_n = repeat_last_n;
  c.frequency_penalty = frequency_penalty;
  c.presence_penalty = presence_penalty;
  halo::sampling::SamplerState s(c, std::span<const std::uint32_t>(prompt, n_prompt));
  s.Accept(std::span<const std::uint32_t>(generated, n_gen));
  std::uint32_t k = 0;
  for (const auto& p : s.penalties()) {
    if (k == cap) break;
    pen_token[k] = p.token;
    pen_generated[k] = p.generated_count;
    pen_repeated[k] = p.repeated;
    ++k;
  }
  *n_pen = k;
  s.SetRngState(*rng);
  std::uint32_t t = 0xFFFFFFFFu;
  try {
    t = s.Sample(std::span<const float>(logits, n));
  } catch (...) {
  }
  *rng = s.rng_state();
  return t;
}

// ---- GGUF reader (src/core/gguf.cpp GgufReader::OpenMemory and its getters) ------------------------------------
void* ref_gguf_open(const void* data, std::size_t size) {
  return halo::core::GgufReader::OpenMemory(data, size).release();
}
void ref_gguf_close(void* h) { delete static_cast<halo::core::GgufReader*>(h); }
void ref_gguf_header(const void* h, std::uint32_t* version, std::uint64_t* alignment, std::uint64_t* n_meta,
                     std::uint64_t* n_tensors) {
  const auto* r = static_cast<const halo::core::GgufReader*>(h);
  *version = r->GetVersion();
  *alignment = r->GetAlignment();
  *n_meta = r->GetMetadataCount();
  *n_tensors = r->GetTensorCount();
}
// Tensor i: name (copied, NUL-terminated), type, dims, offset, size and the data pointer's offset from `base`.
int ref_gguf_tensor(const void* h, std::uint64_t i, const void* base, char* name, std::size_t cap,
                    std::uint32_t* type, std::uint64_t* dims, std::uint32_t* n_dims, std::uint64_t* offset,
                    std::uint64_t* size, std::uint64_t* data_offset) {
  const auto* r = static_cast<const halo::core::GgufReader*>(h);
  const auto ts = r->GetTensors();
  if (i >= ts.size()) return -1;
  const auto& t = ts[i];
  const std::size_t n = std::min(cap - 1, t.name.size());
  std::memcpy(name, t.name.data(), n);
  name[n] = 0;
  *type = static_cast<std::uint32_t>(t.type);
  *n_dims = static_cast<std::uint32_t>(t.dimensions.size());
  for (std::size_t k = 0; k < t.dimensions.size() && k < 8; ++k) dims[k] = t.dimensions[k];
  *offset = t.offset;
  *size = t.size_bytes;
  *data_offset = static_cast<std::uint64_t>(static_cast<const std::uint8_t*>(t.data) -
                                            static_cast<const std::uint8_t*>(base));
  return static_cast<int>(t.name.size());
}
// A metadata value as text: u:<n> i:<n> f:<bits hex> b:<0|1> s:<hex> S:<n>:<hex,...> U:<n,...> I:<n,...>
// F:<bits hex,...>; returns the length, or -1 when the key is absent.
static void HexBytes(std::string* o, std::string_view s) {
  char b[3];
  for (unsigned char ch : s) {
    std::snprintf(b, sizeof b, "%02x", ch);
    *o += b;
  }
}
static void HexDouble(std::string* o, double v) {
  std::uint64_t u;
  std::memcpy(&u, &v, 8);
  char b[17];
  std::snprintf(b, sizeof b, "%016llx", static_cast<unsigned long long>(u));
  *o += b;
}
int ref_gguf_meta(const void* h, const char* key, char* out, std::size_t cap) {
  const auto* r = static_cast<const halo::core::GgufReader*>(h);
  const auto* m = r->FindMetadata(key);
  if (m == nullptr) return -1;
  std::string o;
  const auto& v = m->value;
  if (const auto* x = std::get_if<std::uint64_t>(&v)) {
    o = "u:" + std::to_string(*x);
  } else if (const auto* x = std::get_if<std::int64_t>(&v)) {
    o = "i:" + std::to_string(*x);
  } else if (const auto* x = std::get_if<double>(&v)) {
    o = "f:";
    HexDouble(&o, *x);
  } else if (const auto* x = std::get_if<bool>(&v)) {
    o = std::string("b:") + (*x ? "1" : "0");
  } else if (const auto* x = std::get_if<std::string_view>(&v)) {
    o = "s:";
    HexBytes(&o, *x);
  } else if (const auto* x = std::get_if<std::vector<std::string_view>>(&v)) {
    o = "S:" + std::to_string(x->size()) + ":";
    for (const auto& e : *x) {
      HexBytes(&o, e);
      o += ",";
    }
  } else if (const auto* x = std::get_if<std::vector<std::uint64_t>>(&v)) {
    o = "U:";
    for (auto e : *x) o += std::to_string(e) + ",";
  } else if (const auto* x = std::get_if<std::vector<std::int64_t>>(&v)) {
    o = "I:";
    for (auto e : *x) o += std::to_string(e) + ",";
  } else if (const auto* x = std::get_if<std::vector<double>>(&v)) {
    o = "F:";
    for (auto e : *x) {
      HexDouble(&o, e);
      o += ",";
    }
  }
  o = std::to_string(static_cast<int>(m->type)) + "|" + o;
  const std::size_t n = std::min(cap - 1, o.size());
  std::memcpy(out, o.data(), n);
  out[n] = 0;
  return static_cast<int>(o.size());
}
std::uint32_t ref_gguf_label(const void* h, char* out, std::size_t cap) {
  const std::string l = static_cast<const halo::core::GgufReader*>(h)->GetQuantizationLabel();
  const std::size_t n = std::min(cap - 1, l.size());
  std::memcpy(out, l.data(), n);
  out[n] = 0;
  return static_cast<std::uint32_t>(l.size());
}
std::uint64_t ref_encoded_bytes(std::uint32_t type, std::uint64_t elements) {
  return halo::quant::EncodedSizeBytes(static_cast<halo::core::GgmlType>(type), elements);
}
}
