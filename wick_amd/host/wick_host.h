/*
 * wick_host.h -- C++ host-side mirror of wick's Model::forward over the HIP attention ABI.
 *
 * wick's own host code is Rust (/root/reference/src/model.rs); Rust is not
 * available to this build, so this mirror stands in for it: the same f32
 * arithmetic for every non-attention step, with the KV cache and attention
 * routed through include/wick_hip.h exactly where the Rust code would call it
 * (the cache write at src/model.rs:481-483 and Model::attention at :485).
 * The C functions below exist so that tests and bench.py can drive it.
 */
#ifndef WICK_HOST_H
#define WICK_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
    float rms_eps;
} wick_host_config;

/* Per layer, in this order (NULL for an absent optional tensor):
 * attn_norm, wq, wk, wv, wo, bq, bk, bv, q_norm, k_norm, ffn_norm, w_gate, w_up, w_down. */
#define WICK_HOST_LAYER_TENSORS 14

typedef struct wick_host_model wick_host_model;
typedef struct wick_host_state wick_host_state;

/* Model::from_tensors (src/model.rs:178-235) for f32 weights.  All pointers are
 * borrowed and must outlive the model.  lm_head == NULL means tied to embed.
 * threads: size of the persistent worker pool (Pool::new, src/pool.rs:44). */
wick_host_model *wick_host_model_create(const wick_host_config *cfg, const float *inv_freq, const float *embed,
                                        const float *lm_head, const float *norm, const float *const *layer_tensors,
                                        int threads);
void wick_host_model_destroy(wick_host_model *m);

/* State::new (src/model.rs:300-302): a device-resident KV cache of `capacity` positions. */
wick_host_state *wick_host_state_create(wick_host_model *m, int capacity);
void wick_host_state_destroy(wick_host_state *s);
/* KvCache::len, read and truncated (prefix reuse, src/engine.rs:127-132). */
int wick_host_state_len(const wick_host_state *s);
int wick_host_state_set_len(wick_host_state *s, int len);
/* The device cache handle, for tests that read the cache back. */
void *wick_host_state_kv(wick_host_state *s);

/* Model::forward (src/model.rs:420-516): logits of the last token
 * ([vocab]) or of every token ([t][vocab]).  If att_trace is non-NULL it
 * receives each layer's attention output [layers][t][heads*head_dim].
 * Returns 0, or a negative status (see wick_host_last_error()). */
int wick_host_forward(wick_host_model *m, wick_host_state *s, const uint32_t *tokens, int t, int all_logits,
                      float *logits, float *att_trace);

const char *wick_host_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
