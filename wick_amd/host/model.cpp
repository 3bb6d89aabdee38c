// model.cpp -- f32 Model::forward mirror whose KV cache and attention run on the GPU.
//
// Mirrors /root/reference/src/model.rs:420-516 step by step.  Every host step
// keeps wick's f32 operation order (AVX2 dot product with FMA and wick's
// horizontal sum, src/kernels.rs:196-230; rmsnorm :343-349; silu_mul
// src/kernels.rs:373-378).  The per-token preparation (bias, QK-norm, RoPE;
// src/model.rs:464-480), the cache write and the attention run on the GPU
// through wick_hip_attend; the preparation there is bit-identical to the CPU's,
// so the only numerical difference from an all-CPU run is the attention itself.
// Build with -mavx2 -mfma -ffp-contract=off.
#include "wick_host.h"

#include <immintrin.h>

#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "wick_hip.h"

namespace {

thread_local std::string g_err;

// ------------------------------------------------------------------ pool
// Persistent fork-join workers claiming items from an atomic counter, the
// scheme of src/pool.rs:44-154 (the caller works too).
class Pool {
  public:
    explicit Pool(int threads) {
        if (threads < 1) threads = 1;
        for (int i = 1; i < threads; i++) workers_.emplace_back([this] { loop(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
            epoch_++;
        }
        cv_.notify_all();
        for (auto &w : workers_) w.join();
    }
    void run(int n, const std::function<void(int)> &fn) {
        if (n <= 0) return;
        if (workers_.empty() || n == 1) {
            for (int i = 0; i < n; i++) fn(i);
            return;
        }
        {
            std::lock_guard<std::mutex> g(mu_);
            fn_ = &fn;
            n_ = n;
            next_.store(0);
            active_.store((int)workers_.size());
            epoch_++;
        }
        cv_.notify_all();
        work();
        while (active_.load(std::memory_order_acquire) != 0) std::this_thread::yield();
        fn_ = nullptr;
    }

  private:
    void work() {
        for (;;) {
            int i = next_.fetch_add(1);
            if (i >= n_) break;
            (*fn_)(i);
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return epoch_ != seen; });
                seen = epoch_;
                if (stop_) return;
            }
            work();
            active_.fetch_sub(1, std::memory_order_release);
        }
    }
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable cv_;
    uint64_t epoch_ = 0;
    bool stop_ = false;
    const std::function<void(int)> *fn_ = nullptr;
    int n_ = 0;
    std::atomic<int> next_{0}, active_{0};
};

// ------------------------------------------------------------------ kernels

// src/kernels.rs:196-206
inline float hsum(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

// dot_f32_n<R> (src/kernels.rs:208-230): R <= 4 dot products of one weight row;
// each result is computed exactly as the one-row kernel computes it.
template <int R>
inline void dot_rows(const float *w, const float *const *xs, int n, float *out) {
    __m256 acc[R];
    for (int r = 0; r < R; r++) acc[r] = _mm256_setzero_ps();
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        __m256 wv = _mm256_loadu_ps(w + i);
        for (int r = 0; r < R; r++) acc[r] = _mm256_fmadd_ps(wv, _mm256_loadu_ps(xs[r] + i), acc[r]);
    }
    for (int r = 0; r < R; r++) {
        float s = hsum(acc[r]);
        for (int j = i; j < n; j++) s += w[j] * xs[r][j];
        out[r] = s;
    }
}

struct Job {
    const float *w;  // [rows][cols]
    int rows;
    float *out;      // [t][stride]
    int stride;
};

// matmul_into (src/model.rs:306-383) for f32 jobs sharing the input x [t][cols]:
// items are (job, 16-row chunk); tokens go four at a time through one row pass.
void matmul(Pool &pool, const std::vector<Job> &jobs, const float *x, int t, int cols) {
    constexpr int ROWS = 16;
    std::vector<std::pair<int, int>> items;
    for (int j = 0; j < (int)jobs.size(); j++)
        for (int r = 0; r < jobs[j].rows; r += ROWS) items.emplace_back(j, r);
    pool.run((int)items.size(), [&](int it) {
        const Job &jb = jobs[items[it].first];
        const int r0 = items[it].second, r1 = std::min(r0 + ROWS, jb.rows);
        for (int r = r0; r < r1; r++) {
            const float *row = jb.w + (size_t)r * cols;
            for (int tt = 0; tt < t; tt += 4) {
                const int n = std::min(4, t - tt);
                const float *xs[4];
                for (int k = 0; k < n; k++) xs[k] = x + (size_t)(tt + k) * cols;
                float res[4];
                if (n == 4) dot_rows<4>(row, xs, cols, res);
                else
                    for (int k = 0; k < n; k++) dot_rows<1>(row, xs + k, cols, res + k);
                for (int k = 0; k < n; k++) jb.out[(size_t)(tt + k) * jb.stride + r] = res[k];
            }
        }
    });
}

// src/kernels.rs:343-349 and :351-357 (the Rust f32 sum starts from -0.0)
void rmsnorm(const float *x, const float *w, float eps, float *out, int n) {
    float ss = -0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / (float)n;
    const float scale = 1.0f / std::sqrt(ss + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

enum { T_ATTN_NORM, T_WQ, T_WK, T_WV, T_WO, T_BQ, T_BK, T_BV, T_QN, T_KN, T_FFN_NORM, T_GATE, T_UP, T_DOWN };

}  // namespace

struct wick_host_model {
    wick_host_config c;
    const float *inv_freq, *embed, *lm_head, *norm;
    std::vector<const float *> t;  // layers * 14
    Pool pool;
    wick_host_model(int threads) : pool(threads) {}
    const float *L(int layer, int which) const { return t[(size_t)layer * WICK_HOST_LAYER_TENSORS + which]; }
};

struct wick_host_state {
    wick_hip_kv *kv = nullptr;
    int capacity = 0, len = 0;
    // scratch (src/model.rs:277-291)
    std::vector<float> x, xn, q, k, v, att, o, gate, up;
};

extern "C" {

const char *wick_host_last_error(void) { return g_err.c_str(); }

wick_host_model *wick_host_model_create(const wick_host_config *cfg, const float *inv_freq, const float *embed,
                                        const float *lm_head, const float *norm, const float *const *layer_tensors,
                                        int threads) {
    if (!cfg || !inv_freq || !embed || !norm || !layer_tensors) {
        g_err = "null argument";
        return nullptr;
    }
    if (cfg->heads % cfg->kv_heads != 0 || cfg->head_dim % 2 != 0) {
        g_err = "heads must be a multiple of kv_heads and head_dim even";
        return nullptr;
    }
    auto *m = new wick_host_model(threads);
    m->c = *cfg;
    m->inv_freq = inv_freq;
    m->embed = embed;
    m->lm_head = lm_head;
    m->norm = norm;
    m->t.assign(layer_tensors, layer_tensors + (size_t)cfg->layers * WICK_HOST_LAYER_TENSORS);
    return m;
}

void wick_host_model_destroy(wick_host_model *m) { delete m; }

wick_host_state *wick_host_state_create(wick_host_model *m, int capacity) {
    if (!m || capacity < 1) {
        g_err = "bad state arguments";
        return nullptr;
    }
    auto *s = new wick_host_state();
    int rc = wick_hip_kv_create(m->c.layers, capacity, m->c.kv_heads, m->c.head_dim, &s->kv);
    if (rc != WICK_HIP_OK) {
        g_err = std::string("wick_hip_kv_create: ") + wick_hip_last_error();
        delete s;
        return nullptr;
    }
    // constants of the device-side input preparation: the RoPE table and, per
    // layer, the optional biases and QK-norm weights
    rc = wick_hip_kv_set_rope(s->kv, m->inv_freq);
    for (int li = 0; rc == WICK_HIP_OK && li < m->c.layers; li++)
        rc = wick_hip_kv_set_prep(s->kv, li, m->c.heads, m->L(li, T_BQ), m->L(li, T_BK), m->L(li, T_BV), m->L(li, T_QN),
                                  m->L(li, T_KN), m->c.rms_eps);
    if (rc != WICK_HIP_OK) {
        g_err = std::string("wick_hip_kv_set_rope/set_prep: ") + wick_hip_last_error();
        wick_hip_kv_destroy(s->kv);
        delete s;
        return nullptr;
    }
    s->capacity = capacity;
    return s;
}

void wick_host_state_destroy(wick_host_state *s) {
    if (!s) return;
    wick_hip_kv_destroy(s->kv);
    delete s;
}

int wick_host_state_len(const wick_host_state *s) { return s ? s->len : -1; }

int wick_host_state_set_len(wick_host_state *s, int len) {
    if (!s || len < 0 || len > s->capacity) return -1;
    s->len = len;
    return 0;
}

void *wick_host_state_kv(wick_host_state *s) { return s ? s->kv : nullptr; }

int wick_host_forward(wick_host_model *m, wick_host_state *s, const uint32_t *tokens, int t, int all_logits,
                      float *logits, float *att_trace) {
    if (!m || !s || !tokens || !logits || t <= 0) {
        g_err = "bad forward arguments";
        return -1;
    }
    const wick_host_config &c = m->c;
    // src/model.rs:423-424
    if (s->len + t > s->capacity) {
        g_err = "context length exceeded";
        return -1;
    }
    const int h = c.hidden, hd = c.head_dim, qd = c.heads * hd, kvd = c.kv_heads * hd, ff = c.intermediate;
    const int start = s->len;
    auto fit = [](std::vector<float> &v, size_t n) {
        if (v.size() < n) v.assign(n, 0.f);
    };
    fit(s->x, (size_t)t * h);
    fit(s->xn, (size_t)t * std::max(h, qd));
    fit(s->q, (size_t)t * qd);
    fit(s->k, (size_t)t * kvd);
    fit(s->v, (size_t)t * kvd);
    fit(s->att, (size_t)t * qd);
    fit(s->o, (size_t)t * h);
    fit(s->gate, (size_t)t * ff);
    fit(s->up, (size_t)t * ff);
    float *x = s->x.data(), *xn = s->xn.data(), *q = s->q.data(), *k = s->k.data(), *v = s->v.data();
    float *att = s->att.data(), *o = s->o.data(), *gate = s->gate.data(), *up = s->up.data();

    for (int i = 0; i < t; i++) std::memcpy(x + (size_t)i * h, m->embed + (size_t)tokens[i] * h, sizeof(float) * h);

    for (int li = 0; li < c.layers; li++) {
        for (int i = 0; i < t; i++) rmsnorm(x + (size_t)i * h, m->L(li, T_ATTN_NORM), c.rms_eps, xn + (size_t)i * h, h);
        matmul(m->pool, {{m->L(li, T_WQ), qd, q, qd}, {m->L(li, T_WK), kvd, k, kvd}, {m->L(li, T_WV), kvd, v, kvd}}, xn, t,
               h);
        // src/model.rs:464-485 on the GPU: bias, QK-norm, RoPE, the cache write and Model::attention
        int rc = wick_hip_attend(s->kv, li, c.heads, q, k, v, t, start, att);
        if (rc != WICK_HIP_OK) {
            g_err = std::string("attention: ") + wick_hip_last_error();
            return rc;
        }
        if (att_trace) std::memcpy(att_trace + (size_t)li * t * qd, att, sizeof(float) * (size_t)t * qd);
        matmul(m->pool, {{m->L(li, T_WO), h, o, h}}, att, t, qd);
        for (size_t j = 0; j < (size_t)t * h; j++) x[j] += o[j];

        for (int i = 0; i < t; i++) rmsnorm(x + (size_t)i * h, m->L(li, T_FFN_NORM), c.rms_eps, xn + (size_t)i * h, h);
        matmul(m->pool, {{m->L(li, T_GATE), ff, gate, ff}, {m->L(li, T_UP), ff, up, ff}}, xn, t, h);
        for (size_t j = 0; j < (size_t)t * ff; j++) gate[j] = gate[j] / (1.0f + expf(-gate[j])) * up[j];
        matmul(m->pool, {{m->L(li, T_DOWN), h, o, h}}, gate, t, ff);
        for (size_t j = 0; j < (size_t)t * h; j++) x[j] += o[j];
    }
    s->len = start + t;

    const int n = all_logits ? t : 1, first = all_logits ? 0 : t - 1;
    for (int j = 0; j < n; j++) rmsnorm(x + (size_t)(first + j) * h, m->norm, c.rms_eps, xn + (size_t)j * h, h);
    matmul(m->pool, {{m->lm_head ? m->lm_head : m->embed, c.vocab, logits, c.vocab}}, xn, n, h);
    return 0;
}

}  // extern "C"
