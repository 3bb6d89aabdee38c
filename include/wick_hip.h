/*
 * wick_hip.h -- C ABI of the MI355X attention path for wick.
 *
 * Replaces, behind a C boundary that a Rust `extern "C"` module can bind with
 * no new crates:
 *   - KvCache (/root/reference/src/model.rs:251-275), its allocation
 *     KvCache::new (:261-270) and per-layer slicing state_cache_layer (:556-559):
 *     the cache becomes device-resident, laid out [layer][kv_head][pos][head_dim].
 *   - the KV append in Model::forward (/root/reference/src/model.rs:481-483).
 *   - Model::attention (/root/reference/src/model.rs:518-553), called once per
 *     layer from Model::forward (/root/reference/src/model.rs:485).
 *
 * Conventions
 *   - Every function returning int returns WICK_HIP_OK (0) or a negative
 *     WICK_HIP_E* code; wick_hip_last_error() then describes the failure for
 *     the calling thread.  Nothing aborts or throws across this boundary.
 *   - Host pointers are borrowed for the duration of the call only.
 *   - A handle owns its device memory and one HIP stream.  Calls on one handle
 *     must be serialised by the caller (wick serialises sequences behind a
 *     Mutex<Session>, /root/reference/src/server.rs:143,180).
 *   - There is no CPU fallback: without a usable gfx950 device every call
 *     fails with WICK_HIP_EDEVICE.
 */
#ifndef WICK_HIP_H
#define WICK_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WICK_HIP_OK 0
#define WICK_HIP_EINVAL (-1)  /* bad argument or shape                          */
#define WICK_HIP_EHIP (-2)    /* a HIP runtime call failed                      */
#define WICK_HIP_ENOMEM (-3)  /* device allocation failed                       */
#define WICK_HIP_EDEVICE (-4) /* no usable GPU                                  */

typedef struct wick_hip_kv wick_hip_kv;

/* KvCache::new (src/model.rs:261-270): K and V for `layers` layers of
 * `capacity` positions, zero-filled, on the current HIP device.
 * head_dim must be 16, 32, 64 or 128. */
int wick_hip_kv_create(int layers, int capacity, int kv_heads, int head_dim, wick_hip_kv **out);

/* Drop of KvCache / State (src/model.rs:294-302).  NULL is a no-op. */
void wick_hip_kv_destroy(wick_hip_kv *kv);

/* The cache append of Model::forward (src/model.rs:481-483): rows k, v are
 * host arrays [t][kv_heads*head_dim] for positions start..start+t of `layer`.
 * Bit-exact copy.  Synchronous. */
int wick_hip_kv_append(wick_hip_kv *kv, int layer, int start, int t, const float *k, const float *v);

/* Read back positions pos0..pos0+n of `layer` in wick's host layout
 * [n][kv_heads*head_dim] (either pointer may be NULL).  Synchronous. */
int wick_hip_kv_read(const wick_hip_kv *kv, int layer, int pos0, int n, float *k, float *v);

/* Model::attention (src/model.rs:518-553) for `layer`: q and att are host
 * arrays [t][heads*head_dim]; token i attends to positions 0..=start+i, which
 * must already be in the cache.  heads must be a multiple of kv_heads.
 * att is fully overwritten.  Synchronous: att is valid on return. */
int wick_hip_attention(wick_hip_kv *kv, int layer, int heads, const float *q, int t, int start, float *att);

/* Message for the last failing call on this thread ("" if none). */
const char *wick_hip_last_error(void);

/* ---- device-resident variants (no counterpart in the reference: they let a
 *      caller whose q / k / v / att already live in HBM skip the host copies).
 *      Asynchronous on the handle's stream.  Device arrays must be 16-byte
 *      aligned (the kernels move them as float4); others give WICK_HIP_EINVAL. */

/* As wick_hip_kv_append, with k_dev / v_dev device arrays [t][kv_heads*head_dim]. */
int wick_hip_kv_append_device(wick_hip_kv *kv, int layer, int start, int t, const float *k_dev, const float *v_dev);

/* As wick_hip_attention, with q_dev / att_dev device arrays [t][heads*head_dim]. */
int wick_hip_attention_device(wick_hip_kv *kv, int layer, int heads, const float *q_dev, int t, int start,
                              float *att_dev);

/* As wick_hip_attention_device, but it allocates nothing: no hipMalloc, hipFree
 * or allocating library call on any call, the first included.  No counterpart
 * in the reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid it).
 * Single-token decode keeps its split-K partial states in a static 32 MiB
 * device array (one per GPU, held until the process ends) instead of the
 * handle's workspace: it needs kv_heads * ceil(group / 16) * 16 * 256 *
 * (head_dim + 2) floats, at most 8 Mi (e.g. up to 31 kv heads at head_dim 64
 * with group <= 16, or 15 at head_dim 128); a larger shape returns
 * WICK_HIP_EINVAL.  Prefill (t > 1) uses no workspace.  Every call on one GPU
 * shares that array, so calls that overlap on one GPU (other handles or
 * streams included) race: serialise them.  Asynchronous on the handle's
 * stream. */
int wick_hip_attention_device_noalloc(wick_hip_kv *kv, int layer, int heads, const float *q_dev, int t, int start,
                                      float *att_dev);

/* ---- input preparation on the device: the per-token part of Model::forward
 *      that produces what attention reads (src/model.rs:464-484): bias add,
 *      QK-norm, RoPE of q and k, and the cache append.  The prepared q and the
 *      appended k, v are bit-identical to wick's CPU arithmetic. */

/* RoPE table: (sin, cos) of the f32 angle pos * inv_freq[i] for every cache
 * position pos < capacity, computed on the host with the C library's sinf and
 * cosf (the calls f32::sin_cos makes in rope, src/model.rs:404-414) and kept
 * on the device.  inv_freq is a host array [head_dim/2]
 * (Config::rope_inv_freq, src/config.rs:153-185).  Synchronous. */
int wick_hip_kv_set_rope(wick_hip_kv *kv, const float *inv_freq);

/* Per-layer constants of the preparation (src/model.rs:470-478), host arrays
 * copied to the device: biases bq [heads*head_dim], bk and bv
 * [kv_heads*head_dim] (all three or none: wick adds them only when all three
 * exist), QK-norm weights q_norm and k_norm [head_dim] (both or none), and
 * the RMSNorm eps.  Call it for every layer that wick_hip_attend will see,
 * with NULLs for a model that has neither.  Synchronous. */
int wick_hip_kv_set_prep(wick_hip_kv *kv, int layer, int heads, const float *bq, const float *bk, const float *bv,
                         const float *q_norm, const float *k_norm, float eps);

/* src/model.rs:464-485 for one layer: q [t][heads*head_dim], k and v
 * [t][kv_heads*head_dim] are the raw projections (host arrays) of the tokens
 * at positions start..start+t.  Applies bias, QK-norm and RoPE to q and k as
 * the CPU does (bit-identical), appends k and v at start.., then runs
 * Model::attention; att [t][heads*head_dim] is fully overwritten.  q, k and v
 * are not modified.  Needs wick_hip_kv_set_rope and wick_hip_kv_set_prep
 * (same heads) first.  Synchronous. */
int wick_hip_attend(wick_hip_kv *kv, int layer, int heads, const float *q, const float *k, const float *v, int t,
                    int start, float *att);

/* As wick_hip_attend on device arrays (16-byte aligned).  For t > 1, q_dev is
 * rewritten in place with the prepared q; a single token (t = 1) is prepared
 * inside the decode kernel and q_dev is left as it is.  Asynchronous on the
 * handle's stream. */
int wick_hip_attend_device(wick_hip_kv *kv, int layer, int heads, float *q_dev, const float *k_dev,
                           const float *v_dev, int t, int start, float *att_dev);

/* Make the handle launch on `stream` (a hipStream_t; NULL = the handle's own
 * stream, not the legacy default stream).  Set it before the first call. */
int wick_hip_kv_set_stream(wick_hip_kv *kv, void *stream);

/* Wait for all work queued on the handle's stream. */
int wick_hip_kv_synchronize(wick_hip_kv *kv);

/* Tuning knobs. */
#define WICK_HIP_OPT_DECODE_CHUNK 1 /* positions per decode workgroup (a multiple of 16, at least 64; 0 = automatic) */
/* Split-K key order: 1 = automatic (the default: chunks of at least 256 keys at
 * head_dim 128, or 512 at head_dim 64 with more than 4 query heads per kv head,
 * are read as key groups dealt round-robin over the kv head's workgroups),
 * 0 = one contiguous chunk per workgroup. */
#define WICK_HIP_OPT_DECODE_ORDER 2
int wick_hip_kv_set_option(wick_hip_kv *kv, int option, int value);

/* Number of workgroups the last attention call launched (for measurement). */
int wick_hip_kv_last_grid(const wick_hip_kv *kv);

/* Bytes of staging and decode workspace the handle has allocated so far, beyond
 * its K/V cache and RoPE / preparation tables (device and pinned host memory;
 * grown on demand by the allocating entry points, never by
 * wick_hip_attention_device_noalloc).  No counterpart in the reference: for
 * tests and inspection. */
long long wick_hip_kv_scratch_bytes(const wick_hip_kv *kv);

#ifdef __cplusplus
}
#endif
#endif
