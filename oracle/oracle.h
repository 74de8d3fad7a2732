/* CPU oracle for the quantized decode / ragged-prefill hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is
 * compared against; it is loaded by tests/, by __graft_entry__.smoke() and by
 * bench.py's cpu_baseline leg, never by the product library. Every function
 * restates (in plain C, no SIMD) the algorithm of the reference file:line it
 * cites. Reference paths are relative to the casselc/halo-flash tree.
 *
 * Layout conventions (shared with the product, reference `model/weights.hpp:38-64`):
 *   a matrix has `rows` outputs and `cols` contiguous inputs; Q8_0 rows are
 *   cols/32 blocks of 34 bytes {uint16 fp16 d, int8 qs[32]}; the repacked form
 *   is int8 qs[rows][qstride] plus uint16 d[rows][cols/32].
 */
#ifndef HALO_ORACLE_H_
#define HALO_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats ---------------------------------------------------- */
float or_fp16_to_f32(uint16_t h);
uint16_t or_f32_to_fp16(float f); /* round to nearest even, IEEE binary16 */
float or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f); /* round to nearest even */

/* ---- Q8_0 blocks --------------------------------------------------------- */
void or_dequant_q8_0(const uint8_t* blocks, float* out, size_t k);
void or_repack_q8_0(const uint8_t* raw, int8_t* qs, uint16_t* d, uint32_t rows, uint32_t cols, uint32_t qstride);
void or_pack_q8_0(const int8_t* qs, const uint16_t* d, uint8_t* raw, uint32_t rows, uint32_t cols, uint32_t qstride);

/* Activation quantizer: per 32 values scale = amax/127 (fp32), q = rint(x/scale). */
void or_quantize_q8_act(const float* x, int8_t* xq, float* xs, size_t n);

/* Exact per-block integer dots isum[r][b] = sum_{i<32} qs[r][32b+i] * xq[32b+i]. */
void or_q8_block_dots(const int8_t* qs, uint32_t rows, uint32_t cols, uint32_t qstride, const int8_t* xq,
                      int32_t* isum);

/* y[r] = sum_b d_w[r][b] * xs[b] * isum[r][b], accumulated in double, rounded once to fp32. */
void or_gemv_q8a8(const int8_t* qs, const uint16_t* d, uint32_t rows, uint32_t cols, uint32_t qstride,
                  const int8_t* xq, const float* xs, float* y);
/* The same bound the tolerance uses: mag[r] = sum_b |d_w * xs * isum| (double). */
void or_gemv_q8a8_mag(const int8_t* qs, const uint16_t* d, uint32_t rows, uint32_t cols, uint32_t qstride,
                      const int8_t* xq, const float* xs, double* mag);

/* fp32-activation Q8_0 GEMV as cpu::MatVec computes it (dequant row, double accumulate). `threads` > 1 splits
 * rows over pthreads exactly as the reference splits them (each row is computed identically). */
void or_matvec_q8_0_f32x(const int8_t* qs, const uint16_t* d, uint32_t rows, uint32_t cols, uint32_t qstride,
                         const float* x, float* y, int threads);
/* Dense fp32 W[rows][cols] x, double accumulate (the router). */
void or_matvec_f32(const float* w, uint32_t rows, uint32_t cols, const float* x, float* y);

/* ---- elementwise --------------------------------------------------------- */
float or_sigmoid(float x);
float or_silu(float x);
float or_softplus(float x);
void or_rmsnorm(float* x, size_t n, const float* w, float eps);
void or_l2norm(float* x, size_t n, float eps);
void or_rope_neox(float* x, uint32_t heads, uint32_t head_dim, uint32_t rotary_dim, uint32_t pos, float theta);

/* ---- MoE ----------------------------------------------------------------- */
void or_route_topk(const float* logits, uint32_t n, uint32_t k, uint32_t* ids, float* weights);

/* ---- Gated DeltaNet ------------------------------------------------------ */
/* One decode step for one value head. S is [d][d] value-major (S[j][i], j value, i key) in place; q, k, v
 * length d; decay = exp(g); o[j] = (S_new q)[j] / sqrt(d). */
void or_gdn_step(float* S, uint32_t d, const float* q, const float* k, const float* v, float g, float beta, float* o);

/* A whole sequence of T tokens through or_gdn_step for one value head; q, k, v rows at the given strides (floats),
 * g, beta at stride gstride; S value-major [d][d] in place; o rows at ostride. */
void or_gdn_sequence(float* S, uint32_t d, uint32_t T, const float* q, size_t qstride, const float* k, size_t kstride,
                     const float* v, size_t vstride, const float* g, const float* beta, size_t gstride, float* o,
                     size_t ostride);

/* The magnitude of the terms behind or_gdn_sequence's values (an error bar): M [d][d] value-major, starting at
 * |S0|, in place; omag rows [T][d] at ostride. */
void or_gdn_sequence_mag(double* M, uint32_t d, uint32_t T, const float* q, size_t qstride, const float* k,
                         size_t kstride, const float* v, size_t vstride, const float* g, const float* beta,
                         size_t gstride, double* omag, size_t ostride);

/* ---- GQA decode attention ------------------------------------------------ */
/* One query head over n positions: k, v rows of length hd at stride `kv_stride` floats;
 * o = softmax(q.k / sqrt(hd)) v. */
void or_attention_head(const float* q, const float* k, const float* v, uint32_t n, uint32_t hd, size_t kv_stride,
                       float* o);

/* token sampling (reference src/core/sampling.cpp) */
uint64_t or_next_random(uint64_t* state);
double or_uniform(uint64_t* state);
uint32_t or_sample(const float* logits, uint32_t n, float temperature, int32_t top_k, float top_p, float min_p,
                   uint32_t min_keep, float repeat_penalty, float frequency_penalty, float presence_penalty,
                   const uint32_t* pen_token, const uint32_t* pen_generated, const uint32_t* pen_repeated,
                   uint32_t n_pen, uint64_t* rng);
uint32_t or_sample_penalties(const uint32_t* prompt, uint32_t n_prompt, const uint32_t* generated, uint32_t n_gen,
                             float repeat_penalty, uint32_t repeat_last_n, float frequency_penalty,
                             float presence_penalty, uint32_t* token, uint32_t* gen_count, uint32_t* repeated,
                             uint32_t cap);
uint32_t or_sample_state(const float* logits, uint32_t n, float temperature, int32_t top_k, float top_p,
                         float min_p, uint32_t min_keep, float repeat_penalty, float frequency_penalty,
                         float presence_penalty, const uint32_t* pen_token, const uint32_t* pen_generated,
                         const uint32_t* pen_repeated, uint32_t n_pen, uint64_t* rng);
/* or_sample_state with the draw's uniform given (u_fixed non-null: the RNG is left alone) and the number of
 * tokens with nonzero probability written to *live (when non-null). */
uint32_t or_sample_state_ex(const float* logits, uint32_t n, float temperature, int32_t top_k, float top_p,
                            float min_p, uint32_t min_keep, float repeat_penalty, float frequency_penalty,
                            float presence_penalty, const uint32_t* pen_token, const uint32_t* pen_generated,
                            const uint32_t* pen_repeated, uint32_t n_pen, uint64_t* rng, const double* u_fixed,
                            uint32_t* live);

#ifdef __cplusplus
}
#endif

#endif /* HALO_ORACLE_H_ */
