/*
 * wick_oracle.h -- CPU restatement of wick's attention path and f32 forward pass.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product (wick_amd/) never links or calls it.
 *
 * Every function restates the arithmetic of the Rust reference (file:line under
 * /root/reference): the same operation order, rounding points and libm calls, so
 * that on x86-64 it reproduces what wick computes with its AVX2 kernels
 * (order WO_ORDER_AVX2) or with WICK_SCALAR=1 (order WO_ORDER_SCALAR).
 */
#ifndef WICK_ORACLE_H
#define WICK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { WO_ORDER_AVX2 = 0, WO_ORDER_SCALAR = 1 };

/* dot product of two n-float rows in wick's order (src/kernels.rs:14-28 scalar,
 * :196-230 AVX2 + hsum). */
float wo_dot(const float *w, const float *x, int n, int order);

/* softmax in place (src/kernels.rs:359-371). */
void wo_softmax(float *x, int n);

/* rmsnorm (src/kernels.rs:343-349); out may not alias x. */
void wo_rmsnorm(const float *x, const float *w, float eps, float *out, int n);
/* rmsnorm_inplace (src/kernels.rs:351-357). */
void wo_rmsnorm_inplace(float *x, const float *w, float eps, int n);

/* rotary embedding of every head_dim-sized head in v (src/model.rs:404-414). */
void wo_rope(float *v, int n, int head_dim, int pos, const float *inv_freq);

/* Rotary inverse frequencies (src/config.rs:162-185).  theta is the f32 the
 * config holds; scaling_factor <= 0 means no Llama-3 scaling. */
void wo_rope_inv_freq(float theta, int head_dim, float scaling_factor, float low_freq_factor,
                      float high_freq_factor, int original_max_position, float *out);

/* Model::attention (src/model.rs:518-553).
 *   q      [t][heads*head_dim]
 *   keys   [>= start+t][kv_heads*head_dim]   (wick's per-layer cache slice)
 *   values same layout as keys
 *   att    [t][heads*head_dim] (fully overwritten)
 * Work items (token, head) are claimed from an atomic counter by `threads`
 * workers, as Pool::run does (src/pool.rs:67-120); the result does not depend
 * on the thread count. */
void wo_attention(const float *q, const float *keys, const float *values, float *att, int t, int start,
                  int heads, int kv_heads, int head_dim, int order, int threads);

/* One transformer layer set, f32 weights; NULL for absent optional tensors.
 * Row-major matrices as stored by Hugging Face: [out][in]. */
typedef struct {
    const float *attn_norm, *wq, *wk, *wv, *wo, *bq, *bk, *bv, *q_norm, *k_norm;
    const float *ffn_norm, *w_gate, *w_up, *w_down;
} wo_layer;

typedef struct {
    int hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
    float rms_eps;
    const float *inv_freq;  /* [head_dim/2] */
    const float *embed;     /* [vocab][hidden] */
    const float *lm_head;   /* [vocab][hidden], or NULL when tied to embed */
    const float *norm;      /* [hidden] */
    const wo_layer *layer;  /* [layers] */
} wo_model;

/* Model::forward (src/model.rs:420-516) over an f32 cache laid out as wick's
 * KvCache: cache_k/cache_v are [layers][capacity][kv_heads*head_dim].
 * Appends the t tokens at positions *cache_len.., advances *cache_len, and
 * writes the logits of the last token (all_logits == 0) or of every token
 * ([t][vocab]) to logits.  If att_trace is non-NULL it receives each layer's
 * attention output [layers][t][heads*head_dim] and q_trace the matching q.
 * Returns 0, or -1 when the tokens do not fit in the cache. */
int wo_forward(const wo_model *m, float *cache_k, float *cache_v, int capacity, int *cache_len,
               const uint32_t *tokens, int t, int all_logits, float *logits, int order, int threads,
               float *q_trace, float *att_trace);

/* sampler::argmax (src/sampler.rs:129-137): first index of the maximum. */
uint32_t wo_argmax(const float *x, int n);

/* ---- the sampler (/root/reference/src/sampler.rs), oracle/wick_sampler.c ---- */

/* SamplerConfig (src/sampler.rs:3-14). */
typedef struct {
    float temperature;
    uint32_t top_k;
    float top_p;
    float min_p;
    float repetition_penalty;
    uint64_t seed;
} wo_sampler_config;

/* Rng::new, next_u64, next_f32 (src/sampler.rs:33-60). */
void wo_rng_seed(uint64_t seed, uint64_t s[4]);
uint64_t wo_rng_next_u64(uint64_t s[4]);
float wo_rng_next_f32(uint64_t s[4]);

/* Sampler::sample (src/sampler.rs:73-127) with generator state rng[4]:
 * logits [n] are penalised in place; returns the drawn id.  Optionally the k
 * sorted candidates (ids_out, probs_out after normalisation, capacity n) and
 * the kept count; *k_out = *keep_out = 0 after a greedy draw. */
uint32_t wo_sample(const wo_sampler_config *cfg, uint64_t rng[4], float *logits, int n, const uint32_t *history,
                   int n_history, uint32_t *ids_out, float *probs_out, int *k_out, int *keep_out);

#ifdef __cplusplus
}
#endif
#endif
