/* CPU oracle for the quantized decode / ragged-prefill hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against. Only tests/, smoke() and bench.py's
 * cpu_baseline leg load it. Each function cites the reference (casselc/halo-flash) file:line it restates.
 *
 * Parity pins (what checks each function independently of this file):
 *   fp16/bf16 decode, Q8_0 dequant   -- tests/golden/quant_q8_0_f16_bf16.tsv (gguf-py outputs) + oracle/_ref
 *   quantizer, block dots, gemv_q8a8 -- closed forms, brute force over edge blocks, oracle/_ref dot product
 *   matvec_q8_0_f32x, route_topk, rmsnorm, l2norm, rope, silu -- oracle/_ref (the reference's own cpu_ops.cpp)
 *   moe_token                        -- composition of the above, re-derived in numpy in tests
 *   gdn_step                         -- closed-form invariants (zero state, beta=0 decay-only, delta rule fixes
 *                                      S k = v when beta=1 and |k|=1), numpy restatement on tiny sizes
 *   attention_head                   -- one position returns v; equal keys average v; numpy softmax
 *   sample                           -- oracle/_ref (the reference's own sampling.cpp BuildDistribution + Sample),
 *                                      token and RNG state equal over seeded random rows and every filter
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* reference: src/core/quant.cpp:13-39 (IEEE binary16 -> binary32, subnormals exact). */
float or_fp16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  const uint32_t mant = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      /* value = mant * 2^-24: exact in fp32 */
      float f = (float)mant * 5.9604644775390625e-8f;
      return (h & 0x8000u) ? -f : f;
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t or_f32_to_fp16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
  if (ax < 0x38800000u) {
    /* subnormal half (or zero): value / 2^-24 rounded to nearest even */
    float a;
    memcpy(&a, &ax, 4);
    const float scaled = a * 16777216.0f; /* exact: power of two */
    const float r = nearbyintf(scaled);   /* default rounding mode is RNE */
    return (uint16_t)(sign | (uint16_t)r);
  }
  /* normal: drop 13 mantissa bits with RNE */
  const uint32_t lsb = (ax >> 13) & 1u;
  const uint32_t rounded = ax + 0xFFFu + lsb;
  return (uint16_t)(sign | (uint16_t)((rounded - 0x38000000u) >> 13));
}

float or_bf16_to_f32(uint16_t h) {
  const uint32_t bits = (uint32_t)h << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t or_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* reference: src/core/quant.cpp:411-421 (value = fp16(d) * q), block layout src/core/quant.hpp:58-61. */
void or_dequant_q8_0(const uint8_t* blocks, float* out, size_t k) {
  for (size_t b = 0; b < k / 32; ++b) {
    const uint8_t* blk = blocks + b * 34;
    const float d = or_fp16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
  }
}

/* reference: src/kernels/core.hip:2126-2138 (halo_repack_q8_0): int8 rows at stride qstride + fp16 scale array. */
void or_repack_q8_0(const uint8_t* raw, int8_t* qs, uint16_t* d, uint32_t rows, uint32_t cols, uint32_t qstride) {
  const uint32_t nb = cols / 32;
  for (uint32_t r = 0; r < rows; ++r)
    for (uint32_t b = 0; b < nb; ++b) {
      const uint8_t* src = raw + ((size_t)r * nb + b) * 34;
      d[(size_t)r * nb + b] = (uint16_t)(src[0] | (src[1] << 8));
      memcpy(qs + (size_t)r * qstride + (size_t)b * 32, src + 2, 32);
    }
}

void or_pack_q8_0(const int8_t* qs, const uint16_t* d, uint8_t* raw, uint32_t rows, uint32_t cols, uint32_t qstride) {
  const uint32_t nb = cols / 32;
  for (uint32_t r = 0; r < rows; ++r)
    for (uint32_t b = 0; b < nb; ++b) {
      uint8_t* dst = raw + ((size_t)r * nb + b) * 34;
      const uint16_t s = d[(size_t)r * nb + b];
      dst[0] = (uint8_t)(s & 0xFF);
      dst[1] = (uint8_t)(s >> 8);
      memcpy(dst + 2, qs + (size_t)r * qstride + (size_t)b * 32, 32);
    }
}

/* reference: src/kernels/core.hip:3089-3101 (halo_quantize_q8_rows), host pin tests/gpu/quant_gpu_test.cpp:980-986
 * and src/model/reference.cpp:58-66: scale = amax / 127.0f in fp32, q = nearbyint(x / scale) (round half to even,
 * correctly rounded fp32 division), an all-zero block gives scale 0 and q 0. */
void or_quantize_q8_act(const float* x, int8_t* xq, float* xs, size_t n) {
  for (size_t b = 0; b < n / 32; ++b) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
      const float a = fabsf(x[b * 32 + i]);
      if (a > amax) amax = a;
    }
    const float scale = amax / 127.0f;
    xs[b] = scale;
    for (int i = 0; i < 32; ++i) {
      const float t = x[b * 32 + i] / scale;
      xq[b * 32 + i] = (int8_t)(scale > 0.0f ? (int)nearbyintf(t) : 0);
    }
  }
}

/* Exact integer block sums: reference src/kernels/batch_decode.hip:249-252 (sudot4 chain over 16 values, two halves
 * per block) and tests/gpu/quant_gpu_test.cpp:987-1002 (host sums in `long`). |isum| <= 32*127*128 fits int32. */
void or_q8_block_dots(const int8_t* qs, uint32_t rows, uint32_t cols, uint32_t qstride, const int8_t* xq,
                      int32_t* isum) {
  const uint32_t nb = cols / 32;
  for (uint32_t r = 0; r < rows; ++r) {
    const int8_t* w = qs + (size_t)r * qstride;
    for (uint32_t b = 0; b < nb; ++b) {
      int32_t s = 0;
      for (int i = 0; i < 32; ++i) s += (int32_t)w[b * 32 + i] * (int32_t)xq[b * 32 + i];
      isum[(size_t)r * nb + b] = s;
    }
  }
}

/* reference: tests/gpu/quant_gpu_test.cpp:987-1002 (sum over blocks of dw * sx * dot in double) and the kernel's
 * epilogue src/kernels/batch_decode.hip:253-265 (acc += s_w * (s_x * isum)). */
void or_gemv_q8a8(const int8_t* qs, const uint16_t* d, uint32_t rows, uint32_t cols, uint32_t qstride,
                  const int8_t* xq, const float* xs, float* y) {
  const uint32_t nb = cols / 32;
  for (uint32_t r = 0; r < rows; ++r) {
    const int8_t* w = qs + (size_t)r * qstride;
    double acc = 0.0;
    for (uint32_t b = 0; b < nb; ++b) {
      int32_t s = 0;
      for (int i = 0; i < 32; ++i) s += (int32_t)w[b * 32 + i] * (int32_t)xq[b * 32 + i];
      acc += (double)or_fp16_to_f32(d[(size_t)r * nb + b]) * (double)xs[b] * (double)s;
    }
    y[r] = (float)acc;
  }
}

void or_gemv_q8a8_mag(const int8_t* qs, const uint16_t* d, uint32_t rows, uint32_t cols, uint32_t qstride,
                      const int8_t* xq, const float* xs, double* mag) {
  const uint32_t nb = cols / 32;
  for (uint32_t r = 0; r < rows; ++r) {
    const int8_t* w = qs + (size_t)r * qstride;
    double acc = 0.0;
    for (uint32_t b = 0; b < nb; ++b) {
      int32_t s = 0;
      for (int i = 0; i < 32; ++i) s += (int32_t)w[b * 32 + i] * (int32_t)xq[b * 32 + i];
      acc += fabs((double)or_fp16_to_f32(d[(size_t)r * nb + b]) * (double)xs[b] * (double)s);
    }
    mag[r] = acc;
  }
}

/* reference: src/model/cpu_ops.cpp:108-132 (cpu::MatVec: dequantize each row to fp32, accumulate w*x in double,
 * cast to float; rows split into ceil(rows/threads) chunks, one std::thread each). */
struct mv_job {
  const int8_t* qs;
  const uint16_t* d;
  uint32_t cols, qstride, r0, r1;
  const float* x;
  float* y;
};

static void* mv_work(void* p) {
  const struct mv_job* j = (const struct mv_job*)p;
  const uint32_t nb = j->cols / 32;
  float* w = (float*)malloc(sizeof(float) * j->cols);
  for (uint32_t r = j->r0; r < j->r1; ++r) {
    const int8_t* q = j->qs + (size_t)r * j->qstride;
    for (uint32_t b = 0; b < nb; ++b) {
      const float s = or_fp16_to_f32(j->d[(size_t)r * nb + b]);
      for (int i = 0; i < 32; ++i) w[b * 32 + i] = s * (float)q[b * 32 + i];
    }
    double acc = 0.0;
    for (uint32_t i = 0; i < j->cols; ++i) acc += (double)w[i] * (double)j->x[i];
    j->y[r] = (float)acc;
  }
  free(w);
  return NULL;
}

void or_matvec_q8_0_f32x(const int8_t* qs, const uint16_t* d, uint32_t rows, uint32_t cols, uint32_t qstride,
                         const float* x, float* y, int threads) {
  if (threads < 1) threads = 1;
  if (threads == 1 || rows < 2u * (uint32_t)threads) {
    struct mv_job j = {qs, d, cols, qstride, 0, rows, x, y};
    mv_work(&j);
    return;
  }
  const uint32_t chunk = (rows + (uint32_t)threads - 1) / (uint32_t)threads;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
  struct mv_job* jobs = (struct mv_job*)malloc(sizeof(struct mv_job) * (size_t)threads);
  int n = 0;
  for (uint32_t b = 0; b < rows; b += chunk, ++n) {
    jobs[n] = (struct mv_job){qs, d, cols, qstride, b, b + chunk < rows ? b + chunk : rows, x, y};
    pthread_create(&th[n], NULL, mv_work, &jobs[n]);
  }
  for (int i = 0; i < n; ++i) pthread_join(th[i], NULL);
  free(th);
  free(jobs);
}

void or_matvec_f32(const float* w, uint32_t rows, uint32_t cols, const float* x, float* y) {
  for (uint32_t r = 0; r < rows; ++r) {
    double acc = 0.0;
    for (uint32_t i = 0; i < cols; ++i) acc += (double)w[(size_t)r * cols + i] * (double)x[i];
    y[r] = (float)acc;
  }
}

/* reference: src/model/cpu_ops.cpp:158-166 */
float or_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
float or_silu(float x) { return x * or_sigmoid(x); }
float or_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

/* reference: src/model/cpu_ops.cpp:134-145 (sum of squares in double, scale computed in fp32). */
void or_rmsnorm(float* x, size_t n, const float* w, float eps) {
  double ss = 0.0;
  for (size_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
  const float scale = 1.0f / sqrtf((float)(ss / (double)n) + eps);
  for (size_t i = 0; i < n; ++i) x[i] = x[i] * scale * (w ? w[i] : 1.0f);
}

/* reference: src/model/cpu_ops.cpp:147-156 */
void or_l2norm(float* x, size_t n, float eps) {
  double ss = 0.0;
  for (size_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
  const float scale = 1.0f / sqrtf((float)ss + eps);
  for (size_t i = 0; i < n; ++i) x[i] *= scale;
}

/* reference: src/model/cpu_ops.cpp:168-185 (NEOX pairs (i, i + rotary/2), freq = theta^(-2i/rotary)). */
void or_rope_neox(float* x, uint32_t heads, uint32_t head_dim, uint32_t rotary_dim, uint32_t pos, float theta) {
  const uint32_t half = rotary_dim / 2;
  for (uint32_t h = 0; h < heads; ++h) {
    float* v = x + (size_t)h * head_dim;
    for (uint32_t i = 0; i < half; ++i) {
      const float freq = powf(theta, -2.0f * (float)i / (float)rotary_dim);
      const float angle = (float)pos * freq;
      const float c = cosf(angle), s = sinf(angle);
      const float a = v[i], b = v[i + half];
      v[i] = a * c - b * s;
      v[i + half] = a * s + b * c;
    }
  }
}

/* reference: src/model/cpu_ops.cpp:187-207 (softmax with a double denominator, k largest probabilities with ties to
 * the lower id, renormalized by max(sum, 2^-14)). Selection by repeated arg-max, which orders exactly as the
 * reference's partial_sort comparator. */
void or_route_topk(const float* logits, uint32_t n, uint32_t k, uint32_t* ids, float* weights) {
  float mx = logits[0];
  for (uint32_t i = 1; i < n; ++i)
    if (logits[i] > mx) mx = logits[i];
  float* prob = (float*)malloc(sizeof(float) * n);
  unsigned char* taken = (unsigned char*)calloc(n, 1);
  double den = 0.0;
  for (uint32_t i = 0; i < n; ++i) {
    prob[i] = expf(logits[i] - mx);
    den += prob[i];
  }
  for (uint32_t i = 0; i < n; ++i) prob[i] = (float)(prob[i] / den);
  float sum = 0.0f;
  for (uint32_t s = 0; s < k; ++s) {
    uint32_t best = n;
    for (uint32_t i = 0; i < n; ++i)
      if (!taken[i] && (best == n || prob[i] > prob[best])) best = i;
    taken[best] = 1;
    ids[s] = best;
    sum += prob[best];
  }
  if (sum < 6.103515625e-5f) sum = 6.103515625e-5f;
  for (uint32_t s = 0; s < k; ++s) weights[s] = prob[ids[s]] / sum;
  free(prob);
  free(taken);
}

/* reference: src/model/reference.cpp:329-364 (ReferenceModel::LinearAttention, one value head):
 *   S <- decay * S; u = S k; delta = (v - u) * beta; S <- S + delta k^T; o = (S q) / sqrt(d)
 * with S[j][i] (j value, i key), dot products in double. The layer's decay = exp(a * softplus(alpha + dt)) is
 * passed here as its logarithm g. */
void or_gdn_step(float* S, uint32_t d, const float* q, const float* k, const float* v, float g, float beta, float* o) {
  const float decay = expf(g);
  const float q_scale = 1.0f / sqrtf((float)d);
  float* u = (float*)malloc(sizeof(float) * d);
  for (uint32_t j = 0; j < d; ++j) {
    float* row = S + (size_t)j * d;
    double acc = 0.0;
    for (uint32_t i = 0; i < d; ++i) {
      row[i] *= decay;
      acc += (double)row[i] * k[i];
    }
    u[j] = (float)acc;
  }
  for (uint32_t j = 0; j < d; ++j) {
    const float delta = (v[j] - u[j]) * beta;
    float* row = S + (size_t)j * d;
    double acc = 0.0;
    for (uint32_t i = 0; i < d; ++i) {
      row[i] += delta * k[i];
      acc += (double)row[i] * q[i];
    }
    o[j] = (float)acc * q_scale;
  }
  free(u);
}

/* Token-serial prefill: the reference's prefill is defined as T decode steps (tests/gpu DeltaNetPrefillEqualsDecodeSteps,
 * reference tests/gpu/quant_gpu_test.cpp:1043-1303). */
void or_gdn_sequence(float* S, uint32_t d, uint32_t T, const float* q, size_t qstride, const float* k, size_t kstride,
                     const float* v, size_t vstride, const float* g, const float* beta, size_t gstride, float* o,
                     size_t ostride) {
  for (uint32_t t = 0; t < T; ++t)
    or_gdn_step(S, d, q + t * qstride, k + t * kstride, v + t * vstride, g[t * gstride], beta[t * gstride],
                o + t * ostride);
}

/* Error bar of or_gdn_sequence (no reference counterpart: the magnitude of the terms each value sums): the same
 * recurrence over absolute values, M <- decay M; u = M |k|; M[j][i] += (|v_j| + u_j) |beta| |k_i|; o_mag[j] =
 * (M |q|)[j] / sqrt(d). M starts at |S0| (value-major, in place); per-token o_mag rows at ostride. A computed
 * value's rounding error is a small multiple of its magnitude, whatever order its terms are summed in. */
void or_gdn_sequence_mag(double* M, uint32_t d, uint32_t T, const float* q, size_t qstride, const float* k,
                         size_t kstride, const float* v, size_t vstride, const float* g, const float* beta,
                         size_t gstride, double* omag, size_t ostride) {
  const double q_scale = 1.0 / sqrt((double)d);
  double* u = (double*)malloc(sizeof(double) * d);
  for (uint32_t t = 0; t < T; ++t) {
    const float* qt = q + t * qstride;
    const float* kt = k + t * kstride;
    const float* vt = v + t * vstride;
    const double decay = exp((double)g[t * gstride]);
    const double b = fabs((double)beta[t * gstride]);
    for (uint32_t j = 0; j < d; ++j) {
      double* row = M + (size_t)j * d;
      double acc = 0.0;
      for (uint32_t i = 0; i < d; ++i) {
        row[i] *= decay;
        acc += row[i] * fabs((double)kt[i]);
      }
      u[j] = acc;
    }
    for (uint32_t j = 0; j < d; ++j) {
      const double dm = (fabs((double)vt[j]) + u[j]) * b;
      double* row = M + (size_t)j * d;
      double acc = 0.0;
      for (uint32_t i = 0; i < d; ++i) {
        row[i] += dm * fabs((double)kt[i]);
        acc += row[i] * fabs((double)qt[i]);
      }
      omag[t * ostride + j] = acc * q_scale;
    }
  }
  free(u);
}

/* reference: src/model/reference.cpp:492-521 (dense branch: scores in double rounded to fp32, scaled by 1/sqrt(hd),
 * max-subtracted exp, double denominator, p = score/denom in fp32, o += p * v). */
void or_attention_head(const float* q, const float* k, const float* v, uint32_t n, uint32_t hd, size_t kv_stride,
                       float* o) {
  const float scale = 1.0f / sqrtf((float)hd);
  float* sc = (float*)malloc(sizeof(float) * (n ? n : 1));
  float mx = -INFINITY;
  for (uint32_t j = 0; j < n; ++j) {
    double dot = 0.0;
    for (uint32_t i = 0; i < hd; ++i) dot += (double)q[i] * k[(size_t)j * kv_stride + i];
    sc[j] = (float)dot * scale;
    if (sc[j] > mx) mx = sc[j];
  }
  double den = 0.0;
  for (uint32_t j = 0; j < n; ++j) {
    sc[j] = expf(sc[j] - mx);
    den += sc[j];
  }
  for (uint32_t i = 0; i < hd; ++i) o[i] = 0.0f;
  for (uint32_t j = 0; j < n; ++j) {
    const float p = (float)(sc[j] / den);
    for (uint32_t i = 0; i < hd; ++i) o[i] += p * v[(size_t)j * kv_stride + i];
  }
  free(sc);
}

/* ---- token sampling (reference src/core/sampling.cpp:1-162, 214-293, 330-394, 845-863) -------------------------
 * Semantics: penalties, then top-k (sort by logit descending, ties to the lower token; keep
 * max(top_k, min_keep, 1) when top_k > 0), greedy when temperature == 0, then top-p and min-p on the sorted list,
 * softmax over the survivors (double, max-subtracted, sum in list order), renormalization, zero weights dropped,
 * order (probability descending, token ascending), and one xorshift64* draw (advanced only when more than one
 * token remains). Penalties are a list sorted by token: {token, generated_count, repeated}. Returns the token, or
 * 0xFFFFFFFF when no logit is finite. */
typedef struct {
  uint32_t token;
  double v;
} or_cand;

static int or_cand_cmp(const void* a, const void* b) {
  const or_cand* x = (const or_cand*)a;
  const or_cand* y = (const or_cand*)b;
  if (x->v == y->v) return x->token < y->token ? -1 : (x->token > y->token ? 1 : 0);
  return x->v > y->v ? -1 : 1;
}

/* reference sampling.cpp:845-863 */
uint64_t or_next_random(uint64_t* state) {
  uint64_t v = *state;
  if (v == 0) v = UINT64_C(0x9e3779b97f4a7c15);
  v ^= v >> 12;
  v ^= v << 25;
  v ^= v >> 27;
  *state = v;
  return v * UINT64_C(0x2545f4914f6cdd1d);
}
double or_uniform(uint64_t* state) { return (double)(or_next_random(state) >> 11) * 0x1.0p-53; }

/* reference sampling.cpp:46-67 (weights in list order; sum accumulated in that order) */
static void or_softmax_w(const or_cand* c, size_t n, double temperature, double* w) {
  const double maximum = c[0].v;
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) {
    w[i] = exp((c[i].v - maximum) / temperature);
    sum += w[i];
  }
  for (size_t i = 0; i < n; ++i) w[i] /= sum;
}

uint32_t or_sample(const float* logits, uint32_t n, float temperature, int32_t top_k, float top_p, float min_p,
                   uint32_t min_keep, float repeat_penalty, float frequency_penalty, float presence_penalty,
                   const uint32_t* pen_token, const uint32_t* pen_generated, const uint32_t* pen_repeated,
                   uint32_t n_pen, uint64_t* rng) {
  or_cand* c = (or_cand*)malloc(sizeof(or_cand) * (n ? n : 1));
  double* w = (double*)malloc(sizeof(double) * (n ? n : 1));
  size_t m = 0;
  for (uint32_t i = 0; i < n; ++i)
    if (isfinite(logits[i])) {
      c[m].token = i;
      c[m].v = (double)logits[i];
      ++m;
    }
  uint32_t result = 0xFFFFFFFFu;
  if (m == 0) goto done;
  /* penalties, sampling.cpp:69-93 */
  for (size_t i = 0; i < m; ++i) {
    uint32_t lo = 0, hi = n_pen;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) / 2;
      if (pen_token[mid] < c[i].token) lo = mid + 1; else hi = mid;
    }
    if (lo < n_pen && pen_token[lo] == c[i].token) {
      double l = c[i].v;
      if (pen_repeated[lo] && repeat_penalty != 1.0f) l = l <= 0 ? l * repeat_penalty : l / repeat_penalty;
      l -= (double)frequency_penalty * pen_generated[lo];
      if (pen_generated[lo] != 0) l -= presence_penalty;
      c[i].v = l;
    }
  }
  /* top-k, sampling.cpp:95-113 (a full sort orders the same as the partial sort's prefix) */
  qsort(c, m, sizeof(or_cand), or_cand_cmp);
  const size_t minimum = m < (min_keep > 1 ? min_keep : 1) ? m : (min_keep > 1 ? min_keep : 1);
  if (top_k > 0) {
    size_t keep = (size_t)top_k > minimum ? (size_t)top_k : minimum;
    if (keep < m) m = keep;
  }
  if (temperature == 0.0f) {
    result = c[0].token;
    goto done;
  }
  const double T = (double)temperature;
  /* top-p, sampling.cpp:115-133 */
  if (top_p < 1.0f && m > 1) {
    const size_t mn = m < (min_keep > 1 ? min_keep : 1) ? m : (min_keep > 1 ? min_keep : 1);
    or_softmax_w(c, m, T, w);
    double cumulative = 0.0;
    size_t keep = 0;
    while (keep < m) {
      cumulative += w[keep];
      ++keep;
      if (keep >= mn && cumulative >= (double)top_p) break;
    }
    m = keep;
  }
  /* min-p, sampling.cpp:135-150 */
  if (min_p > 0.0f && m > 1) {
    const size_t mn = m < (min_keep > 1 ? min_keep : 1) ? m : (min_keep > 1 ? min_keep : 1);
    const double threshold = T * log((double)min_p);
    const double maximum = c[0].v;
    size_t keep = 0;
    while (keep < m && c[keep].v - maximum >= threshold) ++keep;
    if (keep < mn) keep = mn;
    if (keep < m) m = keep;
  }
  /* final softmax, then SamplingDistribution: renormalize, drop zeros, order (sampling.cpp:214-242) */
  or_softmax_w(c, m, T, w);
  {
    double sum = 0.0;
    for (size_t i = 0; i < m; ++i) sum += w[i];
    size_t k = 0;
    for (size_t i = 0; i < m; ++i) {
      const double v = w[i] / sum;
      if (v == 0) continue;
      c[k].token = c[i].token;
      c[k].v = v;
      ++k;
    }
    qsort(c, k, sizeof(or_cand), or_cand_cmp);
    /* Sample, sampling.cpp:278-293 */
    if (k == 1) {
      result = c[0].token;
    } else {
      double u = or_uniform(rng);
      result = c[k - 1].token;
      for (size_t i = 0; i < k; ++i) {
        u -= c[i].v;
        if (u < 0.0) {
          result = c[i].token;
          break;
        }
      }
    }
  }
done:
  free(c);
  free(w);
  return result;
}

/* The penalty list of BuildDistribution (reference sampling.cpp:366-394): generated counts when a frequency or
 * presence penalty is set; the last repeat_last_n tokens of prompt + generated marked repeated when repeat_penalty
 * != 1. Writes at most `cap` entries sorted by token; returns the count. */
uint32_t or_sample_penalties(const uint32_t* prompt, uint32_t n_prompt, const uint32_t* generated, uint32_t n_gen,
                             float repeat_penalty, uint32_t repeat_last_n, float frequency_penalty,
                             float presence_penalty, uint32_t* token, uint32_t* gen_count, uint32_t* repeated,
                             uint32_t cap) {
  uint32_t n = 0;
  #define OR_FIND(t, idx)                                    \
    do {                                                     \
      idx = n;                                               \
      for (uint32_t j_ = 0; j_ < n; ++j_)                    \
        if (token[j_] == (t)) { idx = j_; break; }           \
      if (idx == n && n < cap) {                             \
        token[n] = (t); gen_count[n] = 0; repeated[n] = 0; ++n; \
      }                                                      \
    } while (0)
  if (frequency_penalty != 0 || presence_penalty != 0)
    for (uint32_t i = 0; i < n_gen; ++i) {
      uint32_t idx;
      OR_FIND(generated[i], idx);
      if (idx < n) ++gen_count[idx];
    }
  if (repeat_penalty != 1 && repeat_last_n != 0) {
    const uint32_t tail = n_gen < repeat_last_n ? n_gen : repeat_last_n;
    const uint32_t ptail = n_prompt < repeat_last_n - tail ? n_prompt : repeat_last_n - tail;
    for (uint32_t i = n_prompt - ptail; i < n_prompt; ++i) {
      uint32_t idx;
      OR_FIND(prompt[i], idx);
      if (idx < n) repeated[idx] = 1;
    }
    for (uint32_t i = n_gen - tail; i < n_gen; ++i) {
      uint32_t idx;
      OR_FIND(generated[i], idx);
      if (idx < n) repeated[idx] = 1;
    }
  }
  #undef OR_FIND
  /* sort by token (insertion: penalty lists are short) */
  for (uint32_t i = 1; i < n; ++i) {
    const uint32_t t = token[i], g = gen_count[i], r = repeated[i];
    uint32_t j = i;
    while (j > 0 && token[j - 1] > t) {
      token[j] = token[j - 1]; gen_count[j] = gen_count[j - 1]; repeated[j] = repeated[j - 1];
      --j;
    }
    token[j] = t; gen_count[j] = g; repeated[j] = r;
  }
  return n;
}

/* ---- the stateful sampler (reference src/core/sampling.cpp:494-563 SamplerState::Distribution / Sample,
 * 616-700 SampleGreedy / LinearDistribution, 702-842 PrepareSelected) with its penalty list given. This is the
 * path the engine's samplers take and the one the device sampler follows. It differs from or_sample in
 * summation order and in entry order: the weights are exp((v - max) / T) divided by their sum, zeros dropped,
 * and the draw walks the entries in candidate order (token order on the linear path; logit descending, token
 * ascending otherwise) without a re-sort by probability.
 *   - temperature 0: the (penalized) argmax, ties to the lower token, no draw;
 *   - top_k == 0, top_p == 1 and not (min_p > 0 and min_keep > 1): the linear path in token order, min-p as a
 *     threshold max + T log(min_p) that zeroes weights;
 *   - otherwise: candidates sorted, cut to max(top_k, min_keep, 1) when top_k > 0, then top-p (cumulative exp
 *     weights against top_p times their sum; the sum runs over the whole vocabulary in token order when
 *     top_k == 0 and the vocabulary exceeds 1024, else over the sorted candidates), then min-p with the
 *     min_keep floor.
 * Returns the token, or 0xFFFFFFFF when no logit is finite. */
static double or_penalized(const float* logits, uint32_t i, float repeat_penalty, float frequency_penalty,
                           float presence_penalty, const uint32_t* pen_token, const uint32_t* pen_generated,
                           const uint32_t* pen_repeated, uint32_t n_pen) {
  double l = (double)logits[i];
  uint32_t lo = 0, hi = n_pen;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) / 2;
    if (pen_token[mid] < i) lo = mid + 1; else hi = mid;
  }
  if (lo < n_pen && pen_token[lo] == i) {
    if (pen_repeated[lo] && repeat_penalty != 1.0f) l = l <= 0 ? l * repeat_penalty : l / repeat_penalty;
    l -= (double)frequency_penalty * pen_generated[lo];
    if (pen_generated[lo] != 0) l -= presence_penalty;
  }
  return l;
}

static uint32_t or_draw(const or_cand* e, size_t k, uint64_t* rng, const double* u_fixed) {
  if (k == 1) return e[0].token;
  double u = u_fixed ? *u_fixed : or_uniform(rng);
  for (size_t i = 0; i < k; ++i) {
    u -= e[i].v;
    if (u < 0.0) return e[i].token;
  }
  return e[k - 1].token;
}

uint32_t or_sample_state_ex(const float* logits, uint32_t n, float temperature, int32_t top_k, float top_p,
                            float min_p, uint32_t min_keep, float repeat_penalty, float frequency_penalty,
                            float presence_penalty, const uint32_t* pen_token, const uint32_t* pen_generated,
                            const uint32_t* pen_repeated, uint32_t n_pen, uint64_t* rng, const double* u_fixed,
                            uint32_t* live) {
  uint32_t live_ = 0;
  if (live == NULL) live = &live_;
  *live = 0;
  or_cand* c = (or_cand*)malloc(sizeof(or_cand) * (n ? n : 1));
  size_t m = 0;
  for (uint32_t i = 0; i < n; ++i)
    if (isfinite(logits[i])) {
      c[m].token = i;
      c[m].v = or_penalized(logits, i, repeat_penalty, frequency_penalty, presence_penalty, pen_token,
                            pen_generated, pen_repeated, n_pen);
      ++m;
    }
  uint32_t result = 0xFFFFFFFFu;
  if (m == 0) goto done;
  const double T = (double)temperature;
  if (temperature == 0.0f) {
    size_t best = 0;
    for (size_t i = 1; i < m; ++i)
      if (c[i].v > c[best].v) best = i;
    result = c[best].token;
    *live = 1;
    goto done;
  }
  const uint32_t floor_keep = min_keep > 1 ? min_keep : 1;
  if (top_k == 0 && top_p == 1.0f && !(min_p > 0.0f && min_keep > 1)) {
    double maximum = -INFINITY;
    for (size_t i = 0; i < m; ++i)
      if (c[i].v > maximum) maximum = c[i].v;
    const double threshold = min_p > 0.0f ? maximum + T * log((double)min_p) : -INFINITY;
    double total = 0.0;
    for (size_t i = 0; i < m; ++i) {
      c[i].v = c[i].v >= threshold ? exp((c[i].v - maximum) / T) : 0.0;
      total += c[i].v;
    }
    size_t k = 0;
    for (size_t i = 0; i < m; ++i) {
      const double v = c[i].v / total;
      if (v == 0) continue;
      c[k].token = c[i].token;
      c[k].v = v;
      ++k;
    }
    *live = (uint32_t)k;
    result = or_draw(c, k, rng, u_fixed);
    goto done;
  }
  {
    double full_sum = 0.0;
    const int has_full = top_k == 0 && top_p < 1.0f && n > 1024;
    if (has_full) {
      double maximum = -INFINITY;
      for (size_t i = 0; i < m; ++i)
        if (c[i].v > maximum) maximum = c[i].v;
      for (size_t i = 0; i < m; ++i) full_sum += exp((c[i].v - maximum) / T);
    }
    qsort(c, m, sizeof(or_cand), or_cand_cmp);
    if (top_k > 0) {
      size_t keep = (size_t)top_k > floor_keep ? (size_t)top_k : floor_keep;
      if (keep > n) keep = n;
      if (keep < m) m = keep;
    }
    size_t keep = m;
    const size_t minimum = m < floor_keep ? m : floor_keep;
    const double maximum = c[0].v;
    if (top_p < 1.0f && keep > 1) {
      double sum = full_sum;
      if (!has_full) {
        sum = 0.0;
        for (size_t i = 0; i < m; ++i) sum += exp((c[i].v - maximum) / T);
      }
      const double target = (double)top_p * sum;
      double cumulative = 0.0;
      size_t k = 0;
      while (k < keep) {
        cumulative += exp((c[k].v - maximum) / T);
        ++k;
        if (k >= minimum && cumulative >= target) break;
      }
      keep = k;
    }
    if (min_p > 0.0f && keep > 1) {
      const double threshold = maximum + T * log((double)min_p);
      size_t k = 0;
      while (k < keep && c[k].v >= threshold) ++k;
      if (k < minimum) k = minimum;
      if (k < keep) keep = k;
    }
    double total = 0.0;
    for (size_t i = 0; i < keep; ++i) {
      c[i].v = exp((c[i].v - maximum) / T);
      total += c[i].v;
    }
    size_t k = 0;
    for (size_t i = 0; i < keep; ++i) {
      const double v = c[i].v / total;
      if (v == 0) continue;
      c[k].token = c[i].token;
      c[k].v = v;
      ++k;
    }
    *live = (uint32_t)k;
    result = or_draw(c, k, rng, u_fixed);
  }
done:
  free(c);
  return result;
}

uint32_t or_sample_state(const float* logits, uint32_t n, float temperature, int32_t top_k, float top_p,
                         float min_p, uint32_t min_keep, float repeat_penalty, float frequency_penalty,
                         float presence_penalty, const uint32_t* pen_token, const uint32_t* pen_generated,
                         const uint32_t* pen_repeated, uint32_t n_pen, uint64_t* rng) {
  return or_sample_state_ex(logits, n, temperature, top_k, top_p, min_p, min_keep, repeat_penalty,
                            frequency_penalty, presence_penalty, pen_token, pen_generated, pen_repeated, n_pen, rng,
                            NULL, NULL);
}
