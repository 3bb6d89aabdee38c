/*
 * wick_sampler.c -- CPU restatement of wick's sampler (/root/reference/src/sampler.rs).
 *
 * TEST INFRASTRUCTURE ONLY: the checker the device sampler is compared
 * against.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.
 *
 * Each step follows the line of sampler.rs it cites, with wick's f32
 * operations (IEEE division, glibc expf as Rust's f32::exp calls it,
 * sequential sums).  wick's top-k uses an unstable select and sort, which
 * leave the order of equal logits unspecified; here equal logits are ordered
 * by token id, the order the device sampler uses.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "wick_oracle.h"

/* Rng::new (src/sampler.rs:33-43): splitmix64 from the seed, four outputs. */
void wo_rng_seed(uint64_t seed, uint64_t s[4]) {
    uint64_t z = seed;
    for (int i = 0; i < 4; i++) {
        z += 0x9E3779B97F4A7C15ull;
        uint64_t x = z;
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        s[i] = x ^ (x >> 31);
    }
}

static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

/* Rng::next_u64 (:45-55): xoshiro256**. */
uint64_t wo_rng_next_u64(uint64_t s[4]) {
    const uint64_t out = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return out;
}

/* Rng::next_f32 (:57-60). */
float wo_rng_next_f32(uint64_t s[4]) { return (float)(wo_rng_next_u64(s) >> 40) / (float)(1ull << 24); }

/* f32::total_cmp (Rust core): the bit pattern with the low 31 bits of
 * negative values flipped, compared as a signed integer. */
static int32_t total_key(float x) {
    int32_t b;
    memcpy(&b, &x, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

static const float *g_logits;

/* descending logit (total_cmp), then ascending id */
static int by_logit_desc(const void *pa, const void *pb) {
    const uint32_t a = *(const uint32_t *)pa, b = *(const uint32_t *)pb;
    const int32_t ka = total_key(g_logits[a]), kb = total_key(g_logits[b]);
    if (ka != kb) return ka > kb ? -1 : 1;
    return a < b ? -1 : (a > b);
}

uint32_t wo_sample(const wo_sampler_config *cfg, uint64_t rng[4], float *logits, int n, const uint32_t *history,
                   int n_history, uint32_t *ids_out, float *probs_out, int *k_out, int *keep_out) {
    if (k_out) *k_out = 0;
    if (keep_out) *keep_out = 0;
    /* :75-83 repetition penalty, once per distinct id below n */
    if (cfg->repetition_penalty != 1.0f) {
        unsigned char *seen = calloc((size_t)n, 1);
        for (int i = 0; i < n_history; i++) {
            const uint32_t t = history[i];
            if (t < (uint32_t)n && !seen[t]) {
                seen[t] = 1;
                const float l = logits[t];
                logits[t] = l > 0.0f ? l / cfg->repetition_penalty : l * cfg->repetition_penalty;
            }
        }
        free(seen);
    }
    /* :84-86 */
    if (cfg->temperature <= 0.0f) return wo_argmax(logits, n);
    /* :87-94 top-k, sorted */
    const int k = (cfg->top_k == 0 || cfg->top_k > (uint32_t)n) ? n : (int)cfg->top_k;
    uint32_t *idx = malloc((size_t)n * sizeof(uint32_t));
    for (int i = 0; i < n; i++) idx[i] = (uint32_t)i;
    g_logits = logits;
    qsort(idx, (size_t)n, sizeof(uint32_t), by_logit_desc);
    /* :95-98 softmax at the temperature */
    const float max = logits[idx[0]];
    float *probs = malloc((size_t)k * sizeof(float));
    for (int i = 0; i < k; i++) probs[i] = expf((logits[idx[i]] - max) / cfg->temperature);
    float sum = -0.0f;
    for (int i = 0; i < k; i++) sum += probs[i];
    for (int i = 0; i < k; i++) probs[i] /= sum;
    /* :99-104 min-p */
    int keep = k;
    if (cfg->min_p > 0.0f) {
        const float floor_p = probs[0] * cfg->min_p;
        for (int i = 0; i < k; i++)
            if (probs[i] < floor_p) {
                keep = i;
                break;
            }
        if (keep < 1) keep = 1;
    }
    /* :105-115 top-p */
    if (cfg->top_p < 1.0f) {
        float acc = 0.0f;
        for (int i = 0; i < keep; i++) {
            acc += probs[i];
            if (acc >= cfg->top_p) {
                keep = i + 1;
                break;
            }
        }
    }
    /* :116-125 the draw */
    float total = -0.0f;
    for (int i = 0; i < keep; i++) total += probs[i];
    float r = wo_rng_next_f32(rng) * total;
    uint32_t tok = idx[keep - 1];
    for (int i = 0; i < keep; i++) {
        r -= probs[i];
        if (r <= 0.0f) {
            tok = idx[i];
            break;
        }
    }
    if (ids_out) memcpy(ids_out, idx, (size_t)k * sizeof(uint32_t));
    if (probs_out) memcpy(probs_out, probs, (size_t)k * sizeof(float));
    if (k_out) *k_out = k;
    if (keep_out) *keep_out = keep;
    free(probs);
    free(idx);
    return tok;
}
