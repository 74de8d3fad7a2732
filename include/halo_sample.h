/* Device-side token sampling: one draw per row of logits with the reference's SamplerState semantics.
 *
 * Record layouts follow the reference's kernel/engine contract (src/kernels/sample_params.h:13-35, 54-58) so an
 * engine that fills them for the reference's kernels fills them for these:
 *   HaloSampleParams  the request's filters, its penalty-list length, the vocabulary and the RNG state before the
 *                     draw (fallback_only is accepted and ignored: this sampler has no separate fallback kernel);
 *   HaloPenalty       one entry per penalized token, sorted by token (core/sampling's TokenPenalty);
 *   HaloSampleOut     the token, the number of tokens with nonzero probability, the RNG state after the draw.
 * Shared by the kernels (HIP) and the host. */
#ifndef HALO_SAMPLE_H_
#define HALO_SAMPLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct HaloSampleParams {
  float temperature;
  float top_p;
  float min_p;
  float repeat_penalty;
  float frequency_penalty;
  float presence_penalty;
  uint32_t top_k; /* 0: off */
  uint32_t min_keep;
  uint32_t n_penalties;
  uint32_t vocab;
  uint64_t rng; /* xorshift64* state before this draw */
  uint32_t fallback_only;
  uint32_t pad;
} HaloSampleParams;

typedef struct HaloPenalty {
  uint32_t token;
  uint32_t generated_count;
  uint32_t repeated;
  uint32_t pad;
} HaloPenalty;

typedef struct HaloSampleOut {
  uint32_t token; /* or one of the HALO_SAMPLE_* codes below */
  uint32_t live;  /* tokens with nonzero probability (1 for a greedy pick, 0 with a code) */
  uint64_t rng;   /* RNG state after this draw (advanced only when more than one token can be drawn) */
} HaloSampleOut;

/* Token codes. */
#define HALO_SAMPLE_NO_FINITE 0xFFFFFFFFu  /* no finite logit (the reference's code) */
#define HALO_SAMPLE_BAD_PARAMS 0xFFFFFFFCu /* parameters outside SamplingConfig::Validate's ranges or the limits */

/* Limits: the penalized-token bitmap lives in LDS (as the reference's). */
#define HALO_SAMPLE_MAX_VOCAB 262144u
#define HALO_SAMPLE_MAX_PENALTIES 8192u

#ifdef __cplusplus
}
#endif

#endif /* HALO_SAMPLE_H_ */
