/* A C host driving the attention path through include/wick_hip.h only -- the
 * way wick's Rust side would through its extern "C" block: create a
 * device-resident cache, append rows, read them back bit-exact, and run
 * single-token decode (split-K at this length) and a prefill chunk, checked
 * against a double-precision softmax attention computed here.
 * Exit status 0 when every check passes. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "wick_hip.h"

enum { LAYERS = 2, CAP = 4200, KVH = 2, HEADS = 14, D = 64 };

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;

static float next_normalish(void) {
    /* xorshift64*, sum of four uniforms centred: plenty for test data */
    float acc = 0.f;
    for (int i = 0; i < 4; i++) {
        rng_state ^= rng_state >> 12;
        rng_state ^= rng_state << 25;
        rng_state ^= rng_state >> 27;
        const uint64_t r = rng_state * 0x2545F4914F6CDD1Dull;
        acc += (float)((r >> 40) * (1.0 / 16777216.0)) - 0.5f;
    }
    return acc * 1.7f;
}

static void fill(float *x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = next_normalish();
}

/* Model::attention in double: token i of the chunk attends to 0..start+i */
static void reference(const float *q, const float *k, const float *v, int t, int start, double *out) {
    const double scale = 1.0 / sqrt((double)D);
    const int group = HEADS / KVH;
    double *s = malloc(sizeof(double) * (size_t)(start + t));
    for (int i = 0; i < t; i++)
        for (int h = 0; h < HEADS; h++) {
            const int kvh = h / group, len = start + i + 1;
            const float *qr = q + ((size_t)i * HEADS + h) * D;
            double m = -INFINITY, sum = 0.0;
            for (int p = 0; p < len; p++) {
                const float *kr = k + ((size_t)p * KVH + kvh) * D;
                double dot = 0.0;
                for (int j = 0; j < D; j++) dot += (double)qr[j] * kr[j];
                s[p] = dot * scale;
                if (s[p] > m) m = s[p];
            }
            for (int p = 0; p < len; p++) {
                s[p] = exp(s[p] - m);
                sum += s[p];
            }
            double *o = out + ((size_t)i * HEADS + h) * D;
            for (int j = 0; j < D; j++) o[j] = 0.0;
            for (int p = 0; p < len; p++) {
                const float *vr = v + ((size_t)p * KVH + kvh) * D;
                for (int j = 0; j < D; j++) o[j] += s[p] / sum * vr[j];
            }
        }
    free(s);
}

static int check(const char *what, const float *got, const double *want, size_t n) {
    double worst = 0.0;
    int bad = 0;
    for (size_t i = 0; i < n; i++) {
        const double err = fabs((double)got[i] - want[i]);
        if (!(err <= 2e-5 + 1e-4 * fabs(want[i]))) bad++;
        if (err > worst) worst = err;
    }
    printf("%s: max abs err %.3e, %d outside 2e-5 + 1e-4|ref| -> %s\n", what, worst, bad, bad ? "FAIL" : "ok");
    return bad == 0;
}

#define TRY(call)                                                                  \
    do {                                                                           \
        if ((call) != WICK_HIP_OK) {                                               \
            fprintf(stderr, "%s failed: %s\n", #call, wick_hip_last_error());       \
            return 2;                                                              \
        }                                                                          \
    } while (0)

int main(void) {
    const int L = 4097, T = 37, S = 100;
    const size_t kvd = (size_t)KVH * D, qd = (size_t)HEADS * D;
    float *k = malloc(sizeof(float) * CAP * kvd), *v = malloc(sizeof(float) * CAP * kvd);
    float *kb = malloc(sizeof(float) * CAP * kvd), *vb = malloc(sizeof(float) * CAP * kvd);
    float *q = malloc(sizeof(float) * T * qd), *att = malloc(sizeof(float) * T * qd);
    double *want = malloc(sizeof(double) * T * qd);
    wick_hip_kv *kv = NULL;
    int ok = 1;

    fill(k, (size_t)L * kvd);
    fill(v, (size_t)L * kvd);
    TRY(wick_hip_kv_create(LAYERS, CAP, KVH, D, &kv));
    /* layer 1 only, in two appends; layer 0 stays zero */
    TRY(wick_hip_kv_append(kv, 1, 0, 1000, k, v));
    TRY(wick_hip_kv_append(kv, 1, 1000, L - 1000, k + 1000 * kvd, v + 1000 * kvd));
    TRY(wick_hip_kv_read(kv, 1, 0, L, kb, vb));
    const int same = memcmp(k, kb, sizeof(float) * L * kvd) == 0 && memcmp(v, vb, sizeof(float) * L * kvd) == 0;
    printf("append / read back %d rows: %s\n", L, same ? "bit-exact ok" : "FAIL");
    ok &= same;

    /* one token at position L-1 (split-K decode with the merge pass) */
    fill(q, qd);
    TRY(wick_hip_attention(kv, 1, HEADS, q, 1, L - 1, att));
    reference(q, k, v, 1, L - 1, want);
    ok &= check("decode, 4097 positions", att, want, qd);
    printf("decode workgroups: %d\n", wick_hip_kv_last_grid(kv));

    /* a prefill chunk of T tokens at start S (causal over the prefix) */
    fill(q, (size_t)T * qd);
    TRY(wick_hip_attention(kv, 1, HEADS, q, T, S, att));
    reference(q, k, v, T, S, want);
    ok &= check("prefill chunk, 37 tokens at 100", att, want, (size_t)T * qd);

    /* an error comes back as a status and a message, not an abort */
    const int rc = wick_hip_attention(kv, 1, HEADS + 1, q, 1, 10, att);
    printf("bad head count: status %d, \"%s\"\n", rc, wick_hip_last_error());
    ok &= rc == WICK_HIP_EINVAL;

    wick_hip_kv_destroy(kv);
    free(k), free(v), free(kb), free(vb), free(q), free(att), free(want);
    printf("%s\n", ok ? "all ok" : "FAILED");
    return ok ? 0 : 1;
}
