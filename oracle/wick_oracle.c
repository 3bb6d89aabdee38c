/*
 * wick_oracle.c -- CPU restatement of wick's attention path (test infrastructure).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never part of it.
 * Build flags matter: -O2 -mavx2 -mfma -ffp-contract=off, no -ffast-math, so
 * that every multiply and add rounds where Rust rounds (Rust never contracts
 * a*b+c into an FMA; the AVX2 kernels use explicit FMA intrinsics).
 *
 * Parity status of each function is recorded next to it ("pinned by ...").
 */
#include "wick_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- dot product */

/* src/kernels.rs:196-206 hsum: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). */
static inline float hsum256(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

/* src/kernels.rs:208-230 (avx2::dot_f32_n, one row).  Pinned by the tiny
 * fixtures' logits and greedy ids through wo_forward, and by test_oracle's
 * exact-product cases. */
static float dot_avx2(const float *w, const float *x, int n) {
    __m256 acc = _mm256_setzero_ps();
    int i = 0;
    for (; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(w + i), _mm256_loadu_ps(x + i), acc);
    float out = hsum256(acc);
    for (int j = i; j < n; j++) out += w[j] * x[j];
    return out;
}

/* src/kernels.rs:14-28 (scalar::dot_f32): eight unfused partial sums, summed in
 * order starting from -0.0 (Rust's f32 Sum), then the unfused tail. */
static float dot_scalar(const float *w, const float *x, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int nn = n / 8 * 8;
    for (int i = 0; i < nn; i += 8)
        for (int k = 0; k < 8; k++) acc[k] += w[i + k] * x[i + k];
    float s = -0.0f;
    for (int k = 0; k < 8; k++) s += acc[k];
    for (int i = nn; i < n; i++) s += w[i] * x[i];
    return s;
}

float wo_dot(const float *w, const float *x, int n, int order) {
    return order == WO_ORDER_SCALAR ? dot_scalar(w, x, n) : dot_avx2(w, x, n);
}

/* ---------------------------------------------------------------- small ops */

/* src/kernels.rs:359-371.  max = fold(-inf, f32::max); x = exp(x - max) with a
 * sequential f32 sum; x *= 1/sum.  Pinned: closed forms in test_oracle (one
 * element -> 1, equal scores -> 1/n, two scores -> logistic). */
void wo_softmax(float *x, int n) {
    float max = -INFINITY;
    for (int i = 0; i < n; i++) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* src/kernels.rs:343-349.  Pinned through the tiny fixtures (every layer). */
void wo_rmsnorm(const float *x, const float *w, float eps, float *out, int n) {
    float ss = -0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / (float)n;
    float scale = 1.0f / sqrtf(ss + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* src/kernels.rs:351-357.  Pinned through the qwen3-qknorm fixture. */
void wo_rmsnorm_inplace(float *x, const float *w, float eps, int n) {
    float ss = -0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / (float)n;
    float scale = 1.0f / sqrtf(ss + eps);
    for (int i = 0; i < n; i++) x[i] = x[i] * scale * w[i];
}

/* src/model.rs:404-414: rotate-half RoPE, (sin, cos) of the f32 angle
 * pos * inv_freq[i] from libm.  Pinned through the tiny fixtures (positions
 * 0..47) and the rotation-invariant check in test_oracle. */
void wo_rope(float *v, int n, int head_dim, int pos, const float *inv_freq) {
    int half = head_dim / 2;
    for (int h0 = 0; h0 + head_dim <= n; h0 += head_dim) {
        float *head = v + h0;
        for (int i = 0; i < half; i++) {
            float ang = (float)pos * inv_freq[i];
            float s = sinf(ang), c = cosf(ang);
            float a = head[i], b = head[i + half];
            head[i] = a * c - b * s;
            head[i + half] = b * c + a * s;
        }
    }
}

/* src/config.rs:162-185, computed in f64 then rounded to f32.  Pinned by the
 * llama3-scaled fixture (the scaled band) and closed forms in test_oracle. */
void wo_rope_inv_freq(float theta, int head_dim, float scaling_factor, float low_freq_factor,
                      float high_freq_factor, int original_max_position, float *out) {
    int d = head_dim;
    for (int i = 0; i < d / 2; i++) {
        double inv = 1.0 / pow((double)theta, 2.0 * (double)i / (double)d);
        if (scaling_factor <= 0.0f) {
            out[i] = (float)inv;
            continue;
        }
        double omp = (double)original_max_position;
        double low_wavelen = omp / (double)low_freq_factor;
        double high_wavelen = omp / (double)high_freq_factor;
        double wavelen = 2.0 * M_PI / inv;
        double scaled;
        if (wavelen < high_wavelen) {
            scaled = inv;
        } else if (wavelen > low_wavelen) {
            scaled = inv / (double)scaling_factor;
        } else {
            double smooth = (omp / wavelen - (double)low_freq_factor) /
                            ((double)high_freq_factor - (double)low_freq_factor);
            scaled = (1.0 - smooth) * inv / (double)scaling_factor + smooth * inv;
        }
        out[i] = (float)scaled;
    }
}

uint32_t wo_argmax(const float *x, int n) {
    int best = 0;
    for (int i = 0; i < n; i++)
        if (x[i] > x[best]) best = i;
    return (uint32_t)best;
}

/* ---------------------------------------------------------------- fork-join */

/* Dynamic scheduling of n items over `threads` workers through an atomic
 * counter, as src/pool.rs:110-120 (work_on) does.  Items are independent, so
 * the results do not depend on the schedule. */
typedef struct {
    atomic_int next;
    int n;
    void (*fn)(void *ctx, int item);
    void *ctx;
} par_job;

static void *par_worker(void *arg) {
    par_job *j = (par_job *)arg;
    for (;;) {
        int i = atomic_fetch_add(&j->next, 1);
        if (i >= j->n) break;
        j->fn(j->ctx, i);
    }
    return NULL;
}

static void par_run(int n, int threads, void (*fn)(void *, int), void *ctx) {
    par_job j;
    atomic_init(&j.next, 0);
    j.n = n;
    j.fn = fn;
    j.ctx = ctx;
    if (threads < 1) threads = 1;
    if (threads > n) threads = n;
    pthread_t tid[256];
    if (threads > 256) threads = 256;
    for (int i = 1; i < threads; i++) pthread_create(&tid[i], NULL, par_worker, &j);
    par_worker(&j); /* the caller takes part, as Pool::run's caller does */
    for (int i = 1; i < threads; i++) pthread_join(tid[i], NULL);
}

/* ---------------------------------------------------------------- attention */

typedef struct {
    const float *q, *keys, *values;
    float *att;
    int t, start, heads, kv_heads, head_dim, order;
    float scale;
} attn_ctx;

static void attn_item(void *vctx, int item) {
    const attn_ctx *c = (const attn_ctx *)vctx;
    int hd = c->head_dim, kvd = c->kv_heads * hd, qd = c->heads * hd;
    int group = c->heads / c->kv_heads;
    int i = item / c->heads, head = item % c->heads;
    int kvh = head / group;
    const float *qv = c->q + (size_t)i * qd + (size_t)head * hd;
    int len = c->start + i + 1;
    float *sc = (float *)malloc(sizeof(float) * (size_t)len);
    for (int p = 0; p < len; p++) {
        const float *kv = c->keys + (size_t)p * kvd + (size_t)kvh * hd;
        sc[p] = wo_dot(kv, qv, hd, c->order) * c->scale;
    }
    wo_softmax(sc, len);
    float *out = c->att + (size_t)i * qd + (size_t)head * hd;
    for (int k = 0; k < hd; k++) out[k] = 0.0f;
    for (int p = 0; p < len; p++) {
        const float *vv = c->values + (size_t)p * kvd + (size_t)kvh * hd;
        float w = sc[p];
        for (int k = 0; k < hd; k++) out[k] += w * vv[k];
    }
    free(sc);
}

/* src/model.rs:518-553.  Pinned: len = 1 gives V[0] bit-exact; constant keys
 * give the mean of V; an f64 brute force agrees on random shapes; causality
 * (output of token i independent of later tokens); the tiny fixtures'
 * chunked-vs-batch logits. */
void wo_attention(const float *q, const float *keys, const float *values, float *att, int t, int start,
                  int heads, int kv_heads, int head_dim, int order, int threads) {
    attn_ctx c = {q, keys, values, att, t, start, heads, kv_heads, head_dim, order,
                  1.0f / sqrtf((float)head_dim)};
    par_run(t * heads, threads, attn_item, &c);
}

/* ---------------------------------------------------------------- matmul */

typedef struct {
    const float *w; /* [rows][cols] */
    const float *x; /* [t][cols] */
    float *out;     /* [t][stride] */
    int rows, cols, t, stride, order;
} mm_ctx;

enum { MM_ROWS = 16 };

static void mm_item(void *vctx, int item) {
    const mm_ctx *c = (const mm_ctx *)vctx;
    int r0 = item * MM_ROWS, r1 = r0 + MM_ROWS < c->rows ? r0 + MM_ROWS : c->rows;
    for (int r = r0; r < r1; r++) {
        const float *row = c->w + (size_t)r * c->cols;
        for (int tt = 0; tt < c->t; tt++)
            c->out[(size_t)tt * c->stride + r] = wo_dot(row, c->x + (size_t)tt * c->cols, c->cols, c->order);
    }
}

/* matmul_into for one f32 job (src/model.rs:306-383): out[tt][r] = row_r . x[tt].
 * dot_f32_n<4> computes each of its four rows exactly as the one-row kernel
 * does, so grouping tokens by four does not change any bit. */
static void matmul(const float *w, int rows, int cols, const float *x, int t, float *out, int stride, int order,
                   int threads) {
    mm_ctx c = {w, x, out, rows, cols, t, stride, order};
    par_run((rows + MM_ROWS - 1) / MM_ROWS, threads, mm_item, &c);
}

/* ---------------------------------------------------------------- forward */

int wo_forward(const wo_model *m, float *cache_k, float *cache_v, int capacity, int *cache_len,
               const uint32_t *tokens, int t, int all_logits, float *logits, int order, int threads,
               float *q_trace, float *att_trace) {
    int h = m->hidden, hd = m->head_dim, qd = m->heads * hd, kvd = m->kv_heads * hd, ff = m->intermediate;
    int start = *cache_len;
    if (t <= 0 || start + t > capacity) return -1;
    size_t layer_stride = (size_t)capacity * kvd;
    int xn_w = h > qd ? h : qd;
    float *x = calloc((size_t)t * h, 4), *xn = calloc((size_t)t * xn_w, 4);
    float *q = calloc((size_t)t * qd, 4), *k = calloc((size_t)t * kvd, 4), *v = calloc((size_t)t * kvd, 4);
    float *att = calloc((size_t)t * qd, 4), *o = calloc((size_t)t * h, 4);
    float *gate = calloc((size_t)t * ff, 4), *up = calloc((size_t)t * ff, 4);

    for (int i = 0; i < t; i++) memcpy(x + (size_t)i * h, m->embed + (size_t)tokens[i] * h, sizeof(float) * h);

    for (int li = 0; li < m->layers; li++) {
        const wo_layer *l = &m->layer[li];
        for (int i = 0; i < t; i++) wo_rmsnorm(x + (size_t)i * h, l->attn_norm, m->rms_eps, xn + (size_t)i * h, h);
        matmul(l->wq, qd, h, xn, t, q, qd, order, threads);
        matmul(l->wk, kvd, h, xn, t, k, kvd, order, threads);
        matmul(l->wv, kvd, h, xn, t, v, kvd, order, threads);
        for (int i = 0; i < t; i++) {
            float *qi = q + (size_t)i * qd, *ki = k + (size_t)i * kvd, *vi = v + (size_t)i * kvd;
            if (l->bq && l->bk && l->bv) {
                for (int j = 0; j < qd; j++) qi[j] += l->bq[j];
                for (int j = 0; j < kvd; j++) ki[j] += l->bk[j];
                for (int j = 0; j < kvd; j++) vi[j] += l->bv[j];
            }
            if (l->q_norm && l->k_norm) {
                for (int j = 0; j < qd; j += hd) wo_rmsnorm_inplace(qi + j, l->q_norm, m->rms_eps, hd);
                for (int j = 0; j < kvd; j += hd) wo_rmsnorm_inplace(ki + j, l->k_norm, m->rms_eps, hd);
            }
            wo_rope(qi, qd, hd, start + i, m->inv_freq);
            wo_rope(ki, kvd, hd, start + i, m->inv_freq);
            size_t base = (size_t)li * layer_stride + (size_t)(start + i) * kvd;
            memcpy(cache_k + base, ki, sizeof(float) * kvd);
            memcpy(cache_v + base, vi, sizeof(float) * kvd);
        }
        wo_attention(q, cache_k + (size_t)li * layer_stride, cache_v + (size_t)li * layer_stride, att, t, start,
                     m->heads, m->kv_heads, hd, order, threads);
        if (q_trace) memcpy(q_trace + (size_t)li * t * qd, q, sizeof(float) * (size_t)t * qd);
        if (att_trace) memcpy(att_trace + (size_t)li * t * qd, att, sizeof(float) * (size_t)t * qd);
        matmul(l->wo, h, qd, att, t, o, h, order, threads);
        for (size_t j = 0; j < (size_t)t * h; j++) x[j] += o[j];

        for (int i = 0; i < t; i++) wo_rmsnorm(x + (size_t)i * h, l->ffn_norm, m->rms_eps, xn + (size_t)i * h, h);
        matmul(l->w_gate, ff, h, xn, t, gate, ff, order, threads);
        matmul(l->w_up, ff, h, xn, t, up, ff, order, threads);
        for (size_t j = 0; j < (size_t)t * ff; j++) gate[j] = gate[j] / (1.0f + expf(-gate[j])) * up[j];
        matmul(l->w_down, h, ff, gate, t, o, h, order, threads);
        for (size_t j = 0; j < (size_t)t * h; j++) x[j] += o[j];
    }
    *cache_len = start + t;

    int n = all_logits ? t : 1, first = all_logits ? 0 : t - 1;
    for (int j = 0; j < n; j++) wo_rmsnorm(x + (size_t)(first + j) * h, m->norm, m->rms_eps, xn + (size_t)j * h, h);
    const float *head = m->lm_head ? m->lm_head : m->embed;
    matmul(head, m->vocab, h, xn, n, logits, m->vocab, order, threads);

    free(x); free(xn); free(q); free(k); free(v); free(att); free(o); free(gate); free(up);
    return 0;
}
