/*
 * wick_hip_model.h -- a device-resident Model::forward over the attention path
 * of wick_hip.h: projections, norms, SwiGLU, the LM head and the greedy
 * sampler run on the GPU next to the KV cache, so a decode step never copies
 * activations between host and device.
 *
 * Replaces, for f32 weights:
 *   - Model::from_tensors (/root/reference/src/model.rs:178-228): the weights
 *     are copied to HBM once;
 *   - Model::forward (/root/reference/src/model.rs:420-516): matmul_into
 *     (:306-383), rmsnorm (src/kernels.rs:343-349), silu_mul (:373-378) and the
 *     per-token preparation + Model::attention of wick_hip.h;
 *   - sampler::argmax (/root/reference/src/sampler.rs:129-137) and the greedy
 *     loop of cmd_bench (/root/reference/src/main.rs:223-258) with its 256-token
 *     prefill chunks (Session::prefill, /root/reference/src/engine.rs:107, :134);
 *   - the token loop of Session::generate (/root/reference/src/engine.rs:164-204)
 *     with the sampler of wick_hip_sampler.h.
 *
 * Conventions are those of wick_hip.h: int status codes (WICK_HIP_OK or a
 * negative WICK_HIP_E*), wick_hip_last_error() for the message, borrowed host
 * pointers, one stream per model (its caches launch on it), no CPU fallback.
 * Numerics: f32 throughout with FMA dot products in a fixed (deterministic)
 * order that differs from wick's AVX2 order, so logits agree with the CPU to
 * f32 rounding, not bit for bit.
 */
#ifndef WICK_HIP_MODEL_H
#define WICK_HIP_MODEL_H

#include <stdint.h>

#include "wick_hip.h"
#include "wick_hip_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct wick_hip_model wick_hip_model;

/* The Config fields forward uses (src/config.rs:55-133). */
typedef struct {
    int hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
    float rms_eps;
} wick_hip_model_config;

/* Per layer, in this order (NULL for an absent optional tensor):
 * attn_norm, wq, wk, wv, wo, bq, bk, bv, q_norm, k_norm, ffn_norm, w_gate, w_up, w_down.
 * Shapes as wick stores them: wq [heads*head_dim][hidden], wo [hidden][heads*head_dim],
 * w_gate / w_up [intermediate][hidden], w_down [hidden][intermediate]. */
#define WICK_HIP_MODEL_LAYER_TENSORS 14

/* Model::from_tensors for f32 weights: copies every tensor to the device.
 * inv_freq [head_dim/2] is Config::rope_inv_freq (src/config.rs:153-185);
 * lm_head == NULL ties the head to embed (src/model.rs:190-192).
 * hidden, head_dim*heads and intermediate must be multiples of 4. */
int wick_hip_model_create(const wick_hip_model_config *cfg, const float *inv_freq, const float *embed,
                          const float *lm_head, const float *norm, const float *const *layer_tensors,
                          wick_hip_model **out);
void wick_hip_model_destroy(wick_hip_model *m);

/* State::new (src/model.rs:300-302): a KV cache of `capacity` positions for
 * this model, with its RoPE table and per-layer biases / QK-norm registered
 * and its launches on the model's stream.  Destroy it with wick_hip_kv_destroy. */
int wick_hip_model_new_cache(wick_hip_model *m, int capacity, wick_hip_kv **out);

/* Model::forward: tokens [t] (host) at positions start..start+t of `kv`.
 * logits (host) receives the last token's logits [vocab], or every token's
 * [t][vocab] when all_logits is nonzero.  Synchronous. */
int wick_hip_model_forward(wick_hip_model *m, wick_hip_kv *kv, const uint32_t *tokens, int t, int start,
                           int all_logits, float *logits);

/* Session::prefill + sampler::argmax: the prompt [n] (host) in chunks of 256
 * tokens at positions start..start+n, then the greedy next token, written to
 * *next.  Synchronous. */
int wick_hip_model_prefill(wick_hip_model *m, wick_hip_kv *kv, const uint32_t *prompt, int n, int start,
                           uint32_t *next);

/* The greedy loop of cmd_bench: `steps` single-token forwards starting with
 * token `first` at position `start`; after forward i the argmax becomes
 * out[i] and the input of forward i+1.  Ids stay on the device between
 * steps; runs of steps that share a decode launch plan replay one captured
 * step as a HIP graph (same results as launching each step).  The call
 * returns when out [steps] (host) is filled. */
int wick_hip_model_decode(wick_hip_model *m, wick_hip_kv *kv, uint32_t first, int start, int steps, uint32_t *out);

/* Sampler::new (src/sampler.rs:67-71) for this model's vocabulary, launching
 * on the model's stream (wick_hip_sampler.h).  Destroy it with
 * wick_hip_sampler_destroy. */
int wick_hip_model_new_sampler(wick_hip_model *m, const wick_hip_sampler_config *cfg, wick_hip_sampler **out);

/* The token loop of Session::generate (/root/reference/src/engine.rs:164-204)
 * on the device; detokenising and stop strings stay with the caller.
 *   tokens [n] (host) is the session's whole token list; the cache already
 *   holds the first `start` of them (0 <= start < n), and tokens[start..n) run
 *   in chunks of 256 (Session::prefill, :120-139).
 *   Up to max_tokens ids are then drawn with the sampler, clamped to the room
 *   left in the cache (:167-169); every drawn id but the last is fed back
 *   (:200-202).  The repetition penalty reads tokens plus the ids drawn so
 *   far (self.tokens, :179).
 *   An id listed in stops [n_stops] ends the loop; it is neither output nor
 *   fed (:181-184).  With stops the host reads each id while the next step
 *   runs, so one step past a stop is computed and discarded.
 * out [max_tokens] (host) receives *n_out ids; *cache_len receives the number
 * of positions the cache holds afterwards (n plus the ids fed). */
int wick_hip_model_generate(wick_hip_model *m, wick_hip_kv *kv, wick_hip_sampler *s, const uint32_t *tokens, int n,
                            int start, int max_tokens, const uint32_t *stops, int n_stops, uint32_t *out, int *n_out,
                            int *cache_len);

#ifdef __cplusplus
}
#endif
#endif
