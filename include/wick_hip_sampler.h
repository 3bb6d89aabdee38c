/*
 * wick_hip_sampler.h -- wick's token sampler on the GPU, next to the logits.
 *
 * Replaces (and mirrors) /root/reference/src/sampler.rs:
 *   SamplerConfig   (:3-27)   -> wick_hip_sampler_config
 *   Rng             (:29-60)  -> the generator state kept in device memory
 *   Sampler::new    (:67-71)  -> wick_hip_sampler_create
 *   Sampler::sample (:73-127) -> wick_hip_sampler_sample / _sample_device
 * and the token loop of Session::generate (/root/reference/src/engine.rs:170-204)
 * as wick_hip_model_generate in wick_hip_model.h.
 *
 * One draw is one kernel launch of a single workgroup: the repetition penalty,
 * then greedy argmax (temperature <= 0) or top-k by logit (f32::total_cmp
 * order), the softmax at the temperature, min-p, top-p and the draw from
 * xoshiro256** -- each step in wick's f32 operation order.  Equal logits at the
 * top-k boundary or inside the kept set are ordered by token id (wick's
 * unstable sort leaves their order unspecified).  The exponentials follow
 * glibc's expf (the function wick's f32::exp calls on x86-64 Linux) to the bit
 * on every f32 input, so probabilities and draws equal wick's for the same
 * seed and logits.
 *
 * Return codes and wick_hip_last_error() as in wick_hip.h.
 */
#ifndef WICK_HIP_SAMPLER_H
#define WICK_HIP_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct wick_hip_sampler wick_hip_sampler;

/* SamplerConfig (src/sampler.rs:3-14); wick's defaults (:16-20) are
 * {0.7, 40, 0.9, 0.0, 1.0, 0x5EED}. */
typedef struct wick_hip_sampler_config {
    float temperature;        /* <= 0: greedy */
    uint32_t top_k;           /* 0: the whole vocabulary */
    float top_p;              /* >= 1: off */
    float min_p;              /* <= 0: off */
    float repetition_penalty; /* 1: off */
    uint64_t seed;            /* Rng::new (src/sampler.rs:33-43) */
} wick_hip_sampler_config;

/* Sampler::new for logits of `vocab` entries, launching on `stream` (a
 * hipStream_t; NULL = the default stream).  Device scratch for the largest
 * candidate set (the whole vocabulary) is allocated here, once. */
int wick_hip_sampler_create(const wick_hip_sampler_config *cfg, int vocab, void *stream, wick_hip_sampler **out);
void wick_hip_sampler_destroy(wick_hip_sampler *s);

/* Sampler::sample on device memory, asynchronous on the sampler's stream:
 * logits_dev [vocab] (the repetition penalty is applied in place, as wick's
 * &mut [f32]), history_dev [n_history] token ids (read only when the
 * repetition penalty is not 1), and the drawn id written to *out_dev. */
int wick_hip_sampler_sample_device(wick_hip_sampler *s, float *logits_dev, const uint32_t *history_dev,
                                   int n_history, uint32_t *out_dev);

/* The same on host arrays, synchronous: logits [vocab] are updated in place
 * (penalised) like wick's, and the id is returned in *out. */
int wick_hip_sampler_sample(wick_hip_sampler *s, float *logits, const uint32_t *history, int n_history,
                            uint32_t *out);

/* The generator's four state words (Rng's [u64; 4]) after the draws so far. */
int wick_hip_sampler_rng_state(wick_hip_sampler *s, uint64_t state[4]);

/* The candidate list of the last sampling draw, for inspection: *k candidates
 * in wick's order (ids, and the probabilities after normalisation by their
 * sum), *keep of them left by min-p and top-p.  Copies min(*k, cap) entries;
 * either array may be NULL.  After a greedy draw *k = *keep = 0. */
int wick_hip_sampler_last_candidates(wick_hip_sampler *s, int *k, int *keep, uint32_t *ids, float *probs, int cap);

#ifdef __cplusplus
}
#endif

#endif /* WICK_HIP_SAMPLER_H */
