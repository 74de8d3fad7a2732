/* halo-flash MI355X operators: the engine-side dispatch of the hot path, as a C ABI.
 *
 * The reference's engine (src/engine/flash_next_gpu.cpp, batch_decode.cpp, prefill_chunk.cpp) decides which
 * kernel and grid run each operator and launches them by name through rt::Device. halo_engine is that dispatch
 * layer for gfx950: it owns the loaded code object and resolves kernels once; each halo_op_* call enqueues the
 * launches of one operator on the device stream (no synchronization, no allocation unless stated). All tensor
 * arguments are device addresses. Functions return 0 / -1 with a message in err, as halo_rt.h.
 */
#ifndef HALO_OPS_H_
#define HALO_OPS_H_

#include <stddef.h>
#include <stdint.h>

#include "halo_rt.h"
#include "halo_sample.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct halo_engine halo_engine;

/* A repacked Q8_0 matrix in device memory: int8 qs[rows][qstride] + fp16 d[rows][cols/32]
 * (reference src/kernels/core.hip:2116-2124; FlashNextGpu::RepackQ8, src/engine/flash_next_gpu.cpp:414-432). */
typedef struct halo_q8_matrix {
  const int8_t* qs;
  const uint16_t* d;
  uint32_t rows, cols, qstride;
  uint32_t pad;
} halo_q8_matrix;

/* FlashNextGpu::Init's LoadModule(CoreHsaco()) (src/engine/flash_next_gpu.cpp:273) plus kernel lookup. */
int halo_engine_create(halo_device* dev, halo_engine** out, char* err, size_t errlen);
void halo_engine_destroy(halo_engine* eng);
halo_device* halo_engine_device(halo_engine* eng);
/* Launches a kernel of the loaded code object by name (the engine's Launch(name, ...),
 * src/engine/flash_next_gpu.cpp:125-158). */
int halo_engine_launch(halo_engine* eng, const char* kernel, halo_dim3 grid, halo_dim3 block, const halo_arg* args,
                       size_t nargs, char* err, size_t errlen);

/* RepackQ8 (src/engine/flash_next_gpu.cpp:414-432): raw GGUF 34-byte blocks -> qs/d. */
int halo_op_repack_q8_0(halo_engine* eng, const void* raw, int8_t* qs, uint16_t* d, uint32_t rows, uint32_t cols,
                        uint32_t qstride, char* err, size_t errlen);

/* Activation quantizer (halo_quantize_q8_rows, src/kernels/core.hip:3089-3101): x [T][cols] fp32 ->
 * xq [T][cols] int8, xs [T][cols/32] fp32. */
int halo_op_quantize_q8(halo_engine* eng, const float* x, int8_t* xq, float* xs, uint32_t tokens, uint32_t cols,
                        char* err, size_t errlen);
/* Two independent activation sets quantized in one launch (each exactly as halo_op_quantize_q8): x0 [tokens][cols0]
 * and x1 [tokens][cols1]. For a step whose two inputs are ready together (the C1 pass's x and a); no counterpart
 * in the reference. */
int halo_op_quantize_q8_pair(halo_engine* eng, const float* x0, int8_t* xq0, float* xs0, uint32_t cols0,
                             const float* x1, int8_t* xq1, float* xs1, uint32_t cols1, uint32_t tokens, char* err,
                             size_t errlen);

/* Q8_0 x int8-activation projection for M tokens (FlashNextGpu::MatVec + the batched int8 GEMV,
 * src/engine/flash_next_gpu.cpp:212-254, src/kernels/batch_decode.hip:226-345):
 *   y[t * ystride + r] = sum_b d[r][b] * xs[t][b] * isum(r, b, t),   t < M.
 * M <= 8 streams the weights with v_dot4 (in groups of up to 8 columns); 9 <= M <= 16 with dense rows of 1024,
 * 2048 or 4096 columns runs the grouped projection's int8 matrix-core kernel (16 weight rows x 16 tokens per
 * v_mfma_i32_16x16x64_i8, two Q8_0 blocks per step, one launch); M >= 16 otherwise runs int8 MFMA tiles of 16 rows
 * x 16 tokens (x 64 tokens from M = 64), one v_mfma_i32_16x16x32_i8 per Q8_0 block. */
int halo_op_matvec_q8a8(halo_engine* eng, const halo_q8_matrix* w, const int8_t* xq, const float* xs, float* y,
                        uint32_t m, uint32_t ystride, char* err, size_t errlen);
/* Grouped projections with the activation prologue fused in: up to 4 Q8_0 matrices sharing the input row(s) of
 * `tokens` (<= 8; <= 16 in mode Q with 1024, 2048 or 4096 columns) tokens, in ONE launch. Replaces the reference's sequence [RMSNorm] -> halo_quantize_q8_rows ->
 * one MatVec per matrix (src/engine/flash_next_gpu.cpp:212-254, src/kernels/core.hip:3089-3101) for the
 * projections that read the same activations (q|k|v + z + alpha|beta of a DeltaNet layer, q|gate + k + v of an
 * attention layer). ys[i] [tokens][mats[i].rows]. All matrices have cols = in cols (<= 4096, % 32 == 0) and
 * qstride == cols. Modes:
 *   HALO_PROJ_Q: in->xq / in->xs already quantized;
 *   HALO_PROJ_F: in->x fp32 [tokens][cols] quantized in the prologue;
 *   HALO_PROJ_N: x = RMSNorm(in->x + in->delta) * in->norm_w (delta may be null), then quantized; when delta is
 *                non-null and res_out non-null, x + delta is written to res_out (which must not alias in->x);
 *   HALO_PROJ_G: x = per 128-value head RMSNorm(in->x) * in->norm_w [128] * sigmoid(in->delta), the DeltaNet
 *                output norm (ReferenceModel::LinearAttention, src/model/reference.cpp:359-364); cols % 128 == 0.
 * xq_out / xs_out (may be null) receive the quantized activations (bit-identical to halo_op_quantize_q8 of the
 * same fp32 row). */
enum { HALO_PROJ_Q = 0, HALO_PROJ_F = 1, HALO_PROJ_N = 2, HALO_PROJ_G = 3 };
typedef struct halo_proj_input {
  const float* x;
  const float* delta;
  const float* norm_w;
  float* res_out;
  const int8_t* xq;
  const float* xs;
  int8_t* xq_out;
  float* xs_out;
  float eps;
  uint32_t mode;
} halo_proj_input;
int halo_op_proj_q8(halo_engine* eng, const halo_q8_matrix* mats, float* const* ys, uint32_t n_mats,
                    const halo_proj_input* in, uint32_t tokens, char* err, size_t errlen);
/* The same with an explicit tiling for tuning: tasks per wave (1 / 2 / 4 rows groups per wave, so the prologue
 * runs once per 4 x that many groups) and lanes per row (16 / 32 / 64); 0 keeps the default of each. Mode Q with
 * 9..16 tokens and 1024, 2048 or 4096 columns runs on int8 matrix cores (halo_proj_q8m_c*, 16-row tasks);
 * tasks_per_wave = lanes_per_row = 2 selects that kernel from 1 token, = 1 the VALU kernel (8 tokens at most).
 * Mode N at one token with 16 or 32 lanes per row runs the 8-wave form (halo_proj_q8w_*: waves 4-7 stream weights
 * while waves 0-3 form the normalized row); its outputs equal the 4-wave kernel's bit for bit. */
int halo_op_proj_q8_grid(halo_engine* eng, const halo_q8_matrix* mats, float* const* ys, uint32_t n_mats,
                         const halo_proj_input* in, uint32_t tokens, uint32_t tasks_per_wave, uint32_t lanes_per_row,
                         char* err, size_t errlen);

/* Two grouped mode-Q projections with different quantized inputs in one launch (halo_proj_q8q2_*): matrices
 * [0, n_first) (n_first 1 or 2) read in, matrix n_first reads in2; 2..16 tokens (9..16 on int8 matrix cores,
 * halo_proj_q8m2_c2x4: 2048 then 4096 columns); the same bits as two halo_op_proj_q8 calls. For a decode pass whose projections read two activation row sets that are both ready (the
 * C1 q | gate + kv and o projections), one launch instead of two. No counterpart in the reference: it issues one
 * FlashNextGpu::MatVec per matrix (src/engine/flash_next_gpu.cpp:212-254). */
int halo_op_proj_q8_pair(halo_engine* eng, const halo_q8_matrix* mats, float* const* ys, uint32_t n_first,
                         const halo_proj_input* in, const halo_proj_input* in2, uint32_t tokens, char* err,
                         size_t errlen);

/* The same with an explicit GEMV tiling (lanes per row 16/32/64, rows per lane group 1/2/4, waves per block) for
 * tuning sweeps; m <= 8. */
int halo_op_matvec_q8a8_tiled(halo_engine* eng, const halo_q8_matrix* w, const int8_t* xq, const float* xs,
                              float* y, uint32_t m, uint32_t ystride, uint32_t lanes_per_row, uint32_t rows_per_lane,
                              uint32_t waves, char* err, size_t errlen);

/* fp32-activation Q8_0 GEMV (halo_gemv_q8r_r2 / _r4 as FlashNextGpu::MatVec picks them: r2 below 2048 rows). */
int halo_op_matvec_q8_f32x(halo_engine* eng, const halo_q8_matrix* w, const float* x, float* y, char* err,
                           size_t errlen);

/* Exact int32 half-block dots isum[r][c/16] (parity instrumentation; same loads and dot chain as the GEMV). */
int halo_op_q8_half_dots(halo_engine* eng, const halo_q8_matrix* w, const int8_t* xq, int32_t* isum, char* err,
                         size_t errlen);

/* Seeded synthetic tensors generated on the device: Q8_0 with q ~ U{-127..127}, d = fp16(|N(0, sigma)|/127);
 * fp32 ~ N(0, sigma). */
int halo_op_synth_q8(halo_engine* eng, int8_t* qs, uint16_t* d, uint32_t rows, uint32_t cols, uint32_t qstride,
                     uint64_t seed, float sigma, char* err, size_t errlen);
int halo_op_synth_f32(halo_engine* eng, float* x, uint64_t n, uint64_t seed, float sigma, char* err, size_t errlen);

/* ---- MoE decode layer ----------------------------------------------------------------------------------------
 * ReferenceModel::Moe (src/model/reference.cpp:530-578) / FlashNextGpu::Moe (src/engine/flash_next_gpu.cpp:697-845)
 * for T <= 16 tokens: router (fp32) -> softmax/top-k -> union of experts over tokens -> grouped gate/up + SwiGLU
 * -> down with the routed combine in slot order + the shared expert scaled by sigmoid(shared gate logit).
 * Expert tensors are stacked repacked Q8_0 with qstride == cols: gate/up rows = n_experts * ff (cols hidden),
 * down rows = n_experts * hidden (cols ff). The shared expert is absent when shared_gate_proj.qs is NULL. */
typedef struct halo_moe_weights {
  const float* router;      /* [n_experts][hidden] */
  const float* shared_gate; /* [hidden] scalar-gate row, or NULL */
  halo_q8_matrix gate, up, down;
  halo_q8_matrix shared_gate_proj, shared_up, shared_down;
  uint32_t n_experts, n_used, hidden, ff, shared_ff;
  uint32_t pad;
} halo_moe_weights;

/* Device workspace the layer needs for `tokens` tokens (routing tables, quantized activations, h). */
size_t halo_op_moe_workspace_bytes(const halo_moe_weights* w, uint32_t tokens);

/* out [T][hidden] = MoE(x [T][hidden]); 4 launches (router, top-k, gate/up over the union of experts, down +
 * combine; at T = 1, 3: the top-k runs inside the gate/up launch), no allocation, no host round trip (routing stays
 * on the device). `ws` holds halo_op_moe_workspace_bytes; its layout is returned through halo_moe_views for
 * inspection. */
typedef struct halo_moe_views {
  float* logits;          /* [T][n_experts] */
  float* shared_logit;    /* [T] */
  int8_t* xq;             /* [T][hidden] */
  float* xs;              /* [T][hidden/32] */
  uint32_t* ids;          /* [T][n_used], descending probability */
  float* weights;         /* [T][n_used], renormalized */
  float* h;               /* [T * n_used + T][hstride] SiLU(gate) * up: row t*n_used+s routed, T*n_used+t shared */
  uint32_t hstride;
  uint32_t pad;
  size_t bytes;           /* workspace bytes the views span */
} halo_moe_views;
int halo_op_moe_views(const halo_moe_weights* w, uint32_t tokens, void* ws, halo_moe_views* out, char* err,
                      size_t errlen);
int halo_op_moe_decode(halo_engine* eng, const halo_moe_weights* w, const float* x, float* out, uint32_t tokens,
                       void* ws, size_t ws_bytes, char* err, size_t errlen);
/* halo_op_moe_decode with no workspace argument and no allocation: the workspace is a fixed 512 KiB device array of
 * this library (one per GPU, held until the process ends), located once per device on the first call. No reference
 * counterpart: for callers that cannot allocate device memory (code under stream capture, serving loops that forbid
 * hipMalloc). Layers whose halo_op_moe_workspace_bytes exceeds 512 KiB are refused with an error (the C2 layer at 16
 * tokens needs 422 KiB). Calls that overlap on one GPU (other streams or threads) race on the shared array. The array
 * used is the one on the engine's device (halo_device_ordinal), whichever device is current in the calling thread. */
int halo_op_moe_decode_noalloc(halo_engine* eng, const halo_moe_weights* w, const float* x, float* out,
                               uint32_t tokens, char* err, size_t errlen);
/* The same layer with the FFN input norm folded into the router launch (the reference's post-attention
 * residual add + RMSNorm before Moe, src/engine/flash_next_gpu.cpp:697-845): in->x = residual, in->delta = the
 * attention / DeltaNet output, in->norm_w = the FFN norm weights, in->eps; in->res_out (not in->x) receives
 * x + delta. MoE(RMSNorm(x + delta) * norm_w) goes to out. tokens <= 4, hidden 2048 or 4096, tokens * hidden <= 8192.
 * The router launch of halo_op_moe_decode is replaced, so four launches replace five. */
int halo_op_moe_decode_norm(halo_engine* eng, const halo_moe_weights* w, const halo_proj_input* in, float* out,
                            uint32_t tokens, void* ws, size_t ws_bytes, char* err, size_t errlen);

/* MoE layer for a batch of T tokens (prefill; the reference's GroupedMoe, src/engine/prefill_chunk.cpp:1156-1222, and
 * ReferenceModel::Moe semantics, src/model/reference.cpp:530-578): fp32 router GEMM (+ shared gate logit), top-k per
 * token, pairs grouped by expert in token order, grouped int8 MFMA gate/up (SwiGLU) and down per expert group (the
 * shared expert is one more group), slot-order combine. x [T][hidden] fp32 (normalized), out [T][hidden]. Requires
 * shared_ff == ff when the shared expert is present, n_experts + 1 <= 1024; out and ws 16-byte aligned. Workspace from
 * halo_op_moe_prefill_workspace_bytes(w, T) (0: unsupported). The routing (ids / weights [T][k]) is at the start of
 * the workspace: ws + align(T * n_experts * 4) + align(T * 4) + align(T * hidden) + align(T * hidden / 8). */
size_t halo_op_moe_prefill_workspace_bytes(const halo_moe_weights* w, uint32_t tokens);
int halo_op_moe_prefill(halo_engine* eng, const halo_moe_weights* w, const float* x, float* out, uint32_t tokens,
                        void* ws, size_t ws_bytes, char* err, size_t errlen);

/* ---- Gated DeltaNet ------------------------------------------------------------------------------------------
 * The recurrence of ReferenceModel::LinearAttention (src/model/reference.cpp:329-364) / halo_gdn_step_d128
 * (src/kernels/core.hip:2620-2646) per value head h (key head h % Hk), decay = exp(g):
 *   u = (decay S)^T k,  delta = (v - u) * beta,  S <- decay S + k delta^T,  o = S^T q / sqrt(d).
 * State: fp32 [S][Hv][d][d] key-major (S[i][j], i key, j value). d = 128. */

/* One decode step for S sessions: q, k [S][Hk][d], v [S][Hv][d], g, beta [S][Hv] (g = log decay, beta after its
 * sigmoid), o [S][Hv][d]; state updated in place. One launch. */
int halo_op_gdn_decode(halo_engine* eng, float* state, const float* q, const float* k, const float* v,
                       const float* g, const float* beta, float* o, uint32_t sessions, uint32_t v_heads,
                       uint32_t k_heads, uint32_t head_dim, char* err, size_t errlen);

/* ---- GQA decode attention over a paged, prefix-shared KV cache ---------------------------------------------------
 * ReferenceModel::Attention's dense branch (src/model/reference.cpp:492-527) / halo_attention_select_b
 * (src/kernels/core.hip:898): per query head h (kv head h / (Hq/Hkv)), o = softmax(q.K^T/sqrt(d)) V * sigmoid(gate).
 * KV pools [pages][Hkv][16][d] fp32, page tables [S][max_pages] (uint32), nkv [S] visible positions (device
 * memory, so a captured graph replays at every position). The first `prefix` tokens (a multiple of 64) have the same
 * pages in every session's table and are read once for all sessions. d = 256, S * Hq / Hkv <= 32, context <= 32K. */
typedef struct halo_paged_kv {
  float* k_pool;
  float* v_pool;
  const uint32_t* pages; /* [S][max_pages] */
  const uint32_t* nkv;   /* [S] */
  uint32_t sessions, kv_heads, head_dim, max_pages, prefix, max_context;
} halo_paged_kv;

/* Arithmetic: one session runs fp32 dot products; two or more sessions (and the prefill below) run the products on
 * split-fp16 matrix cores (each operand as hi + lo halves after a power-of-two scaling: q, k and V by 2^8, the
 * probabilities by 2^14), within 2^-22 of each product for operands of magnitude about 1e-4 to 255. A query row, K
 * chunk or V chunk holding a magnitude of 255.875 or more takes a smaller power-of-two scale (largest value below
 * 2^15), so no finite operand overflows; that group's small values then keep a coarser absolute precision. */
/* Scratch for the partials of one decode attention call. */
size_t halo_op_attn_decode_workspace_bytes(const halo_paged_kv* kv, uint32_t q_heads);
/* o [S][Hq][d] = attention(q [S][Hq][d]) over each session's nkv positions; gate [S][Hq][d] or NULL. Two launches. */
int halo_op_attn_decode(halo_engine* eng, const halo_paged_kv* kv, const float* q, const float* gate, float* o,
                        uint32_t q_heads, void* ws, size_t ws_bytes, char* err, size_t errlen);
/* The same, o optional (may be NULL), also writing o's Q8 quantization for the output projection:
 * oq [S][Hq * d] int8, os [S][Hq * d / 32]. */
int halo_op_attn_decode_q8(halo_engine* eng, const halo_paged_kv* kv, const float* q, const float* gate, float* o,
                           int8_t* oq, float* os, uint32_t q_heads, void* ws, size_t ws_bytes, char* err,
                           size_t errlen);
/* One decode step of the attention block from its input projections: every q head RMSNorm(q_norm) and rotated
 * (NEOX, the first `rot` <= 128 dims) at its session's position nkv[s] - 1, that position's K (RMSNorm k_norm,
 * rotated) and V appended to the pools, then the attention as above with gate = the second half of each qg head.
 * Replaces the prologue of ReferenceModel::Attention (src/model/reference.cpp:368-416) plus halo_op_attn_decode_q8
 * in two launches (the prologue runs inside the partial launch). qg [S][Hq][2 d] (per head: q | gate), k, v
 * [S][Hkv][d]; every nkv[s] - 1 must lie at or past the shared prefix. Bitwise equal to halo_attn_prep_decode followed
 * by halo_op_attn_decode_q8. */
int halo_op_attn_decode_step_q8(halo_engine* eng, const halo_paged_kv* kv, const float* qg, const float* k,
                                const float* v, const float* q_norm, const float* k_norm, uint32_t rot, float theta,
                                float eps, float* o, int8_t* oq, float* os, uint32_t q_heads, void* ws,
                                size_t ws_bytes, char* err, size_t errlen);
/* A run of consecutive prompt positions of one session inside a prefill batch: tokens [first, first + length) of
 * the batch are positions [start, start + length) of session `session`. */
typedef struct halo_prefill_segment {
  uint32_t session, start, length, first;
} halo_prefill_segment;

/* Causal GQA attention for a ragged batch of prefill tokens (ReferenceModel::Attention, src/model/reference.cpp:
 * 368-416, 492-527, per prompt token): every token attends to positions 0 .. its own of its session (shared prefix
 * pages included); K / V of the batch must already be in the pools. q, gate [T][Hq][256]; o [T][Hq][256] fp32 and /
 * or its Q8 quantization oq [T][Hq 256] / os [T][Hq 8] (either may be null). segs is a host array; the op uploads
 * the tile table into ws (halo_op_attn_prefill_workspace_bytes) and is therefore not capturable. */
size_t halo_op_attn_prefill_workspace_bytes(const halo_prefill_segment* segs, uint32_t nseg);
int halo_op_attn_prefill(halo_engine* eng, const halo_paged_kv* kv, const halo_prefill_segment* segs, uint32_t nseg,
                         const float* q, const float* gate, float* o, int8_t* oq, float* os, uint32_t Hq, void* ws,
                         size_t ws_bytes, char* err, size_t errlen);
/* Writes one token's k, v [S][Hkv][d] at position nkv[s] - 1 of each session. */
int halo_op_kv_append(halo_engine* eng, const halo_paged_kv* kv, const float* k, const float* v, char* err,
                      size_t errlen);

/* Chunked prefill (C = 64) over a ragged batch of sequences (halo_gdn_c16_prep / halo_gdn_c16_scan*,
 * src/kernels/core.hip:6592-7421, here with 64-token chunks): the same recurrence over every token of every
 * sequence, outputs o [tokens][Hv][d] fp32, state [seq][Hv][d][d] read as the initial state and overwritten with the
 * final one. q, k [tokens][Hk][d] and v [tokens][Hv][d] bf16; g, beta [tokens][Hv] fp32. The chunk tables are
 * device buffers built by halo_gdn_chunk_table. Two launches: a parallel pass over all (chunk, head) pairs, then a
 * scan per (sequence, head, 32 value columns). */
/* Host helper: from seqlens [n_seq] fills chunks [n][3] = {first token, length, sequence} and seqs [n_seq][2] =
 * {first chunk, chunk count} (either output may be NULL to count); returns the number of chunks. */
uint32_t halo_gdn_chunk_table(const uint32_t* seqlens, uint32_t n_seq, uint32_t* chunks, uint32_t* seqs);
size_t halo_op_gdn_prefill_workspace_bytes(uint32_t n_chunks, uint32_t v_heads);
int halo_op_gdn_prefill(halo_engine* eng, const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                        const float* beta, const uint32_t* chunks, const uint32_t* seqs, uint32_t n_chunks,
                        uint32_t n_seq, float* state, float* o, uint32_t v_heads, uint32_t k_heads, uint32_t head_dim,
                        void* ws, size_t ws_bytes, char* err, size_t errlen);
/* The same recurrence with fp32 q, k, v (the reference's default prefill reads its fp32 conv outputs,
 * src/engine/prefill_chunk.cpp:556-640); the model's batched prefill uses it so that prefill and decode see the same
 * inputs. */
int halo_op_gdn_prefill_f32(halo_engine* eng, const float* q, const float* k, const float* v, const float* g,
                            const float* beta, const uint32_t* chunks, const uint32_t* seqs, uint32_t n_chunks,
                            uint32_t n_seq, float* state, float* o, uint32_t v_heads, uint32_t k_heads,
                            uint32_t head_dim, void* ws, size_t ws_bytes, char* err, size_t errlen);

/* Device sampling, one draw per row (replaces the launches of halo_sample / halo_sample_blocks + halo_sample_final,
 * src/engine/flash_next_gpu.cpp:876-893, src/engine/batch_decode.cpp:605-621, with the semantics of
 * SamplerState::Sample, src/core/sampling.cpp:542-563). logits [rows][row_stride] fp32; params [rows]; penalties
 * [rows][pen_stride]; out [rows]; all device memory. Each out[r] holds the token (or a HALO_SAMPLE_* code), the
 * nonzero-probability count and the advanced RNG state. ws: halo_op_sample_workspace_bytes(rows, vocab). */
size_t halo_op_sample_workspace_bytes(uint32_t rows, uint32_t vocab);
int halo_op_sample(halo_engine* eng, const float* logits, uint32_t rows, uint64_t row_stride, uint32_t vocab,
                   const HaloSampleParams* params, const HaloPenalty* penalties, uint32_t pen_stride,
                   HaloSampleOut* out, void* ws, size_t ws_bytes, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif

#endif /* HALO_OPS_H_ */
