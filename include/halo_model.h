/* halo-flash MI355X hybrid model: the decode step of the engine over the hot-path operators.
 *
 * The reference's FlashNextGpu (src/engine/flash_next_gpu.hpp:38-925) owns weights, sessions and the captured decode
 * step; Step/StepBatch (flash_next_gpu.cpp:899-1047, batch_decode.cpp:629-817) run one token per session through
 * every layer and sample. halo_model is that object for the synthetic hybrid model of the benchmark: Gated DeltaNet
 * and gated GQA layers (every attn_interval-th layer is attention), a routed MoE FFN with a shared expert in every
 * layer, Q8_0 projections, greedy decoding. Weights are seeded on the device. Sessions share the first
 * prefix_tokens positions of their KV cache (paged, 16 tokens per page). One step for S sessions is recorded once
 * into a HIP graph and replayed; the per-step token and position live in device memory and a final launch advances
 * them (prompt tokens are fed while a session's prompt lasts, its own argmax afterwards).
 * Functions return 0 / -1 with a message in err (halo_rt.h convention). */
#ifndef HALO_MODEL_H_
#define HALO_MODEL_H_

#include <stddef.h>
#include <stdint.h>

#include "halo_ops.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct halo_model_config {
  uint32_t vocab, hidden, layers, attn_interval;
  uint32_t gdn_k_heads, gdn_v_heads, gdn_head_dim, conv_kernel;
  uint32_t q_heads, kv_heads, head_dim, rotary_dim;
  uint32_t n_experts, n_used, expert_ff, shared_ff;
  float rope_theta, rms_eps;
  uint32_t max_sessions, max_context; /* context per session, including the shared prefix */
  uint32_t prefix_tokens;             /* shared-prefix capacity (multiple of 64; 0: none) */
  uint32_t prefill_batch;             /* tokens per prefill batch (0: 8192; 64 ... 65536) */
} halo_model_config;

typedef struct halo_model halo_model;

/* Allocates and seeds every weight and state buffer on the engine's device. */
int halo_model_create(halo_engine* eng, const halo_model_config* cfg, uint64_t seed, halo_model** out, char* err,
                      size_t errlen);
void halo_model_destroy(halo_model* m);
/* Bytes of weights (algorithmic: Q8_0 at 34 bytes per 32 weights, fp32 tensors at 4) and of device allocations. */
uint64_t halo_model_weight_bytes(const halo_model* m);
uint64_t halo_model_device_bytes(const halo_model* m);

/* Session s: its prompt (host tokens, copied to the device), and the number of positions already in its cache
 * (0 for a fresh session; prefix_tokens for a session forked after the shared prefix). The next step feeds
 * prompt[nkv]. Not capturable (uploads). */
int halo_model_set_session(halo_model* m, uint32_t s, const uint32_t* prompt, uint32_t prompt_len, uint32_t nkv,
                           char* err, size_t errlen);
/* Copies session src's recurrent state (DeltaNet state and conv history of every layer) to dst; the shared prefix
 * pages are common to both already (the reference's ForkSession, flash_next_gpu.hpp:347-350). */
int halo_model_fork(halo_model* m, uint32_t src, uint32_t dst, char* err, size_t errlen);
/* Zeroes every session's recurrent state and position. */
int halo_model_reset(halo_model* m, char* err, size_t errlen);

/* Enqueues `steps` decode steps for sessions 0..S-1 (one token each). attn_prefix: positions read once for all
 * sessions (the shared prefix, a multiple of 64, <= each session's position; 0 when S == 1 or nothing is shared).
 * The first call with a given (S, attn_prefix) records the step into a HIP graph; later calls replay it. */
int halo_model_run(halo_model* m, uint32_t S, uint32_t attn_prefix, uint32_t steps, char* err, size_t errlen);
/* The same step launched eagerly (no graph): for profilers and debugging. */
int halo_model_step_eager(halo_model* m, uint32_t S, uint32_t attn_prefix, char* err, size_t errlen);

/* Batched prefill (the reference's PrefillChunk / prompt ingestion, src/engine/prefill_chunk.cpp): positions
 * [start, start + length) of each segment's session, tokens from the session's prompt, all layers run on the whole
 * batch (projections as int8 MFMA GEMMs, DeltaNet through the chunked recurrence on fp32 q / k / v, causal
 * attention over the paged cache, grouped MoE). Segment sessions must be
 * consecutive and increasing (s0, s0 + 1, ...); positions below start must already be in the cache. Afterwards each
 * session is where the same number of decode steps would leave it: history[start + length] holds the argmax after
 * the last position, the next input token is prompt[start + length] when the prompt goes on, nkv = start + length + 1.
 * Not capturable (uploads per batch of up to 2048 tokens). `first` is ignored. */
int halo_model_prefill(halo_model* m, const halo_prefill_segment* segs, uint32_t nseg, char* err, size_t errlen);

/* Device sampling for session s (the reference's per-request sampler upload, FlashNextGpu::Step /
 * BatchDecode, src/engine/flash_next_gpu.cpp:876-893, src/engine/batch_decode.cpp:605-621): host copies of the
 * parameters and the penalty list (sorted by token, at most HALO_SAMPLE_MAX_PENALTIES) go to device memory; from
 * then on every step of the model draws each session's token with halo_op_sample (sessions without parameters stay
 * greedy through temperature 0) and carries the RNG state forward on the device, so a multi-step run draws the
 * sequence the CPU sampler would from that state. The penalty list is what the caller uploaded last: a caller
 * whose penalties follow the generated tokens sets them again between steps. Not capturable (uploads); steps
 * recorded before the first call keep argmax decoding in their own graphs. */
int halo_model_set_sampling(halo_model* m, uint32_t s, const HaloSampleParams* params, const HaloPenalty* penalties,
                            uint32_t n_penalties, char* err, size_t errlen);
/* Host copy of session s's sampling parameters as the device holds them (the RNG state after the last draw). */
int halo_model_sample_state(halo_model* m, uint32_t s, HaloSampleParams* params, char* err, size_t errlen);

/* Host copies of session s's produced tokens history[pos] (the argmax after position pos-1 ... ) and nkv. */
int halo_model_history(halo_model* m, uint32_t s, uint32_t* out, uint32_t n, char* err, size_t errlen);
int halo_model_positions(halo_model* m, uint32_t* nkv_out, uint32_t S, char* err, size_t errlen);

/* A weight tensor of the model, for inspection (the reference's GGUF tensor table, src/core/gguf.hpp; used by
 * parity tests to recompute a step on the host). kind: HALO_TENSOR_F32 (data [rows][cols] fp32) or
 * HALO_TENSOR_Q8 (data = qs [rows][qstride] int8, scales = d [rows][cols / 32] fp16 bits). Device pointers. */
enum { HALO_TENSOR_F32 = 0, HALO_TENSOR_Q8 = 1 };
typedef struct halo_model_tensor_view {
  void* data;
  void* scales;
  uint32_t kind, rows, cols, qstride;
} halo_model_tensor_view;
/* layer < layers: per-layer tensors by name: attn_norm, ffn_norm; DeltaNet layers: qkv, z, ab (alpha | beta rows),
 * out, conv_w [C][K], a, dt, norm_w, and the recurrent state: state ([max_sessions Hv d][d], key-major per head),
 * conv_ring ([max_sessions K][C]); attention layers: qg (per head q | gate rows), k, v, o, q_norm, k_norm, and the
 * KV pools k_pool, v_pool ([pages Hkv 16][hd]); every layer: router [E][H], shared_gate [H], gate, up
 * ([E * ff][H]), down ([E * H][ff]), sgate, sup, sdown. layer == UINT32_MAX: embd, head, out_norm, pages
 * ([max_sessions][max_pages] uint32) and nkv ([max_sessions] uint32), both viewed as 4-byte words. */
int halo_model_tensor(const halo_model* m, uint32_t layer, const char* name, halo_model_tensor_view* out, char* err,
                      size_t errlen);
/* Teacher-forcing trace (parity instrumentation; the reference has no counterpart): one eager step, like
 * halo_model_step_eager, that also copies the tensors a host restatement needs to check each layer from the GPU's own
 * inputs into `trace` (device memory of trace_bytes) and lists them in entries[0 .. *n_entries). Per layer (entry
 * layer = layer index): res_in (residual entering the layer, fp32 [S][H]), xq / xs (its RMSNorm quantized: int8
 * [S][H], fp32 [S][H/32]); DeltaNet layers qkv [S][C], z [S][Hv d], ab [S][2 Hv]; attention layers qg [S][2 Hq hd],
 * k, v [S][Hkv hd]; then oq / os (the mixer output quantized for the output projection), delta (its output
 * [S][H]); mres (residual entering the MoE), mxq / mxs, mlogits [S][E], mshared [S], mids (uint32 [S][k]),
 * mweights [S][k], mh (h rows [S (k + 1)][hstride], as halo_moe_views), mout (MoE output [S][H]). After the layers
 * (layer = UINT32_MAX): res_in, xq, xs of the final norm. Each entry starts 256-byte aligned. The recurrent state
 * before the step is read with halo_model_tensor ("state", "conv_ring", "k_pool", "v_pool", "pages", "nkv"). */
enum { HALO_TRACE_F32 = 0, HALO_TRACE_I8 = 1, HALO_TRACE_U32 = 2 };
typedef struct halo_model_trace_entry {
  char name[24];
  uint32_t layer, dtype;
  uint64_t offset, bytes;
} halo_model_trace_entry;
int halo_model_step_trace(halo_model* m, uint32_t S, uint32_t attn_prefix, void* trace, size_t trace_bytes,
                          halo_model_trace_entry* entries, uint32_t max_entries, uint32_t* n_entries, char* err,
                          size_t errlen);

/* The same trace for one batched prefill call (halo_model_prefill) whose segments fit one batch (<= the prefill batch;
 * shared_ff == expert_ff): entries per layer for all T tokens of the batch, [T][...] in batch order: res_in, xq,
 * xs; DeltaNet qkv, z, ab, gq / gk (the conv + L2 outputs [T][Hk d]), gv [T][Hv d], g / beta [T][Hv], o (the
 * recurrence output [T][Hv d]); attention qg, k, v, aq (normalised, rotated queries [T][Hq hd]); oq, os, delta;
 * MoE mres, mxq, mxs, mlogits, mshared, mids, mweights, mpos (uint32 [T][k]: each pair's row among the pairs
 * sorted by expert; the shared expert's pair of token t is row T k + t), mh / mhq / mhs (h of the sorted pairs
 * [T (k + 1)][ff] fp32, its codes and scales), mout; then the final norm's res_in, xq, xs. */
int halo_model_prefill_trace(halo_model* m, const halo_prefill_segment* segs, uint32_t nseg, void* trace,
                             size_t trace_bytes, halo_model_trace_entry* entries, uint32_t max_entries,
                             uint32_t* n_entries, char* err, size_t errlen);
/* The prefill trace restricted to some layers: bit l of layer_mask (l < 63) selects layer l's entries, bit 63 the
 * final norm's; the prefill itself runs every layer. Lets a long batch (thousands of tokens) be traced in a few
 * layers within device memory. Models of more than 63 layers accept only the all-ones mask. */
int halo_model_prefill_trace_layers(halo_model* m, const halo_prefill_segment* segs, uint32_t nseg, uint64_t layer_mask,
                                    void* trace, size_t trace_bytes, halo_model_trace_entry* entries,
                                    uint32_t max_entries, uint32_t* n_entries, char* err, size_t errlen);

/* Host copy of session s's logits of the last step ([vocab] fp32). Not capturable. */
int halo_model_logits(halo_model* m, uint32_t s, float* out, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif

#endif /* HALO_MODEL_H_ */
