// sampler_api.cpp -- the C ABI of include/wick_hip_sampler.h: wick's Sampler
// (/root/reference/src/sampler.rs:62-127) with its generator state and scratch
// resident on the GPU.
#include "wick_hip_sampler.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "attn_kernels.h"
#include "sampler_kernels.h"
#include "wick_hip.h"

struct wick_hip_sampler {
    wick_hip_sampler_config cfg{};
    int vocab = 0;
    hipStream_t stream = nullptr;
    uint32_t *flags = nullptr;
    uint64_t *rng = nullptr;
    uint32_t *key0 = nullptr, *key1 = nullptr, *idx1 = nullptr, *res_idx = nullptr;
    float *res_prob = nullptr;
    int *meta = nullptr;
    int parts = 1, slice = 32;
    float *part_val = nullptr;
    uint32_t *part_id = nullptr;
    unsigned long long *part_cand = nullptr;
    int *part_count = nullptr;
    // staging for the host-array entry point
    float *logits = nullptr;
    uint32_t *out = nullptr;
    uint32_t *history = nullptr;
    int cap_history = 0;
};

namespace {

using wick::set_error;

int hip_fail(hipError_t e, const char *what) {
    return set_error(e == hipErrorOutOfMemory ? WICK_HIP_ENOMEM : WICK_HIP_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr)                                     \
    do {                                                  \
        hipError_t e_ = (expr);                           \
        if (e_ != hipSuccess) return hip_fail(e_, #expr); \
    } while (0)

// Rng::new (src/sampler.rs:33-43): four outputs of splitmix64 from the seed.
void seed_rng(uint64_t seed, uint64_t out[4]) {
    uint64_t z = seed;
    for (int i = 0; i < 4; i++) {
        z += 0x9E3779B97F4A7C15ull;
        uint64_t x = z;
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        out[i] = x ^ (x >> 31);
    }
}

void release(wick_hip_sampler *s) {
    void *bufs[] = {s->flags, s->rng,      s->key0,     s->key1,      s->idx1,       s->res_idx, s->res_prob, s->meta,
                    s->part_val, s->part_id, s->part_cand, s->part_count, s->logits, s->out,     s->history};
    for (void *b : bufs)
        if (b) (void)hipFree(b);
}

int check_draw(const wick_hip_sampler *s, const float *logits, const uint32_t *history, int n_history,
               const uint32_t *out) {
    if (!s || !logits || !out) return set_error(WICK_HIP_EINVAL, "null argument");
    if (n_history < 0) return set_error(WICK_HIP_EINVAL, "n_history must be >= 0 (got %d)", n_history);
    if (n_history > 0 && !history) return set_error(WICK_HIP_EINVAL, "null history with n_history %d", n_history);
    return WICK_HIP_OK;
}

}  // namespace

namespace wick {

int sampler_enqueue(wick_hip_sampler *s, float *logits, const uint32_t *history, int n_history, uint32_t *out) {
    if (int rc = check_draw(s, logits, history, n_history, out)) return rc;
    if (reinterpret_cast<uintptr_t>(logits) & 15u)
        return set_error(WICK_HIP_EINVAL, "logits must be 16-byte aligned");
    SampleArgs a{};
    a.logits = logits;
    a.vocab = s->vocab;
    a.history = history;
    a.n_history = s->cfg.repetition_penalty != 1.0f ? n_history : 0;
    a.flags = s->flags;
    a.rng = s->rng;
    a.out = out;
    a.temperature = s->cfg.temperature;
    a.top_p = s->cfg.top_p;
    a.min_p = s->cfg.min_p;
    a.penalty = s->cfg.repetition_penalty;
    a.top_k = s->cfg.top_k;
    a.key0 = s->key0;
    a.key1 = s->key1;
    a.idx1 = s->idx1;
    a.res_idx = s->res_idx;
    a.res_prob = s->res_prob;
    a.res_meta = s->meta;
    a.parts = s->parts;
    a.slice = s->slice;
    a.split_top_k = s->slice <= kSliceMax;
    a.part_val = s->part_val;
    a.part_id = s->part_id;
    a.part_cand = s->part_cand;
    a.part_count = s->part_count;
    hipError_t e = launch_sample(a, s->stream);
    if (e != hipSuccess) return hip_fail(e, "sample launch");
    return WICK_HIP_OK;
}

hipStream_t sampler_stream(const wick_hip_sampler *s) { return s->stream; }
int sampler_vocab(const wick_hip_sampler *s) { return s->vocab; }
bool sampler_reads_history(const wick_hip_sampler *s) { return s->cfg.repetition_penalty != 1.0f; }

}  // namespace wick

extern "C" {

int wick_hip_sampler_create(const wick_hip_sampler_config *cfg, int vocab, void *stream, wick_hip_sampler **out) {
    if (!cfg || !out) return set_error(WICK_HIP_EINVAL, "null argument");
    *out = nullptr;
    if (vocab < 1) return set_error(WICK_HIP_EINVAL, "vocab must be >= 1 (got %d)", vocab);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) return set_error(WICK_HIP_EDEVICE, "no HIP device");
    wick_hip_sampler *s = new (std::nothrow) wick_hip_sampler;
    if (!s) return set_error(WICK_HIP_ENOMEM, "out of host memory");
    s->cfg = *cfg;
    s->vocab = vocab;
    s->stream = static_cast<hipStream_t>(stream);
    // slices of the split kernel: whole bitset words, about 4096 ids or more each
    s->parts = std::min(wick::kSampleParts, (vocab + 4095) / 4096);
    s->slice = ((vocab + s->parts - 1) / s->parts + 31) / 32 * 32;
    s->parts = (vocab + s->slice - 1) / s->slice;
    const size_t n = (size_t)vocab, words = (n + 31) / 32, np = wick::kSampleParts;
    struct {
        void **p;
        size_t bytes;
    } want[] = {{(void **)&s->flags, words * 4},   {(void **)&s->rng, 32},        {(void **)&s->key0, n * 4},
                {(void **)&s->key1, n * 4},        {(void **)&s->idx1, n * 4},    {(void **)&s->res_idx, n * 4},
                {(void **)&s->res_prob, n * 4},    {(void **)&s->meta, 16},       {(void **)&s->logits, n * 4},
                {(void **)&s->out, 16},            {(void **)&s->part_val, np * 4},
                {(void **)&s->part_id, np * 4},    {(void **)&s->part_cand, np * wick::kFastK * 8},
                {(void **)&s->part_count, np * 4}};
    int rc = WICK_HIP_OK;
    for (auto &w : want) {
        hipError_t e = hipMalloc(w.p, w.bytes);
        if (e != hipSuccess) {
            rc = hip_fail(e, "hipMalloc(sampler)");
            break;
        }
    }
    uint64_t st[4];
    seed_rng(cfg->seed, st);
    if (!rc) {
        hipError_t e = hipMemsetAsync(s->flags, 0, words * 4, s->stream);
        if (e == hipSuccess) e = hipMemsetAsync(s->meta, 0, 16, s->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(s->rng, st, sizeof st, hipMemcpyHostToDevice, s->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
        if (e != hipSuccess) rc = hip_fail(e, "sampler set-up");
    }
    if (rc) {
        release(s);
        delete s;
        return rc;
    }
    *out = s;
    return WICK_HIP_OK;
}

void wick_hip_sampler_destroy(wick_hip_sampler *s) {
    if (!s) return;
    (void)hipStreamSynchronize(s->stream);
    release(s);
    delete s;
}

int wick_hip_sampler_sample_device(wick_hip_sampler *s, float *logits_dev, const uint32_t *history_dev,
                                   int n_history, uint32_t *out_dev) {
    return wick::sampler_enqueue(s, logits_dev, history_dev, n_history, out_dev);
}

int wick_hip_sampler_sample(wick_hip_sampler *s, float *logits, const uint32_t *history, int n_history,
                            uint32_t *out) {
    if (int rc = check_draw(s, logits, history, n_history, out)) return rc;
    const bool reads = s->cfg.repetition_penalty != 1.0f && n_history > 0;
    if (reads && n_history > s->cap_history) {
        HIP_TRY(hipStreamSynchronize(s->stream));
        if (s->history) (void)hipFree(s->history);
        s->history = nullptr;
        s->cap_history = 0;
        HIP_TRY(hipMalloc(&s->history, (size_t)n_history * sizeof(uint32_t)));
        s->cap_history = n_history;
    }
    const size_t bytes = (size_t)s->vocab * sizeof(float);
    HIP_TRY(hipMemcpyAsync(s->logits, logits, bytes, hipMemcpyHostToDevice, s->stream));
    if (reads)
        HIP_TRY(hipMemcpyAsync(s->history, history, (size_t)n_history * sizeof(uint32_t), hipMemcpyHostToDevice,
                               s->stream));
    if (int rc = wick::sampler_enqueue(s, s->logits, reads ? s->history : nullptr, reads ? n_history : 0, s->out))
        return rc;
    HIP_TRY(hipMemcpyAsync(logits, s->logits, bytes, hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipMemcpyAsync(out, s->out, sizeof(uint32_t), hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return WICK_HIP_OK;
}

int wick_hip_sampler_rng_state(wick_hip_sampler *s, uint64_t state[4]) {
    if (!s || !state) return set_error(WICK_HIP_EINVAL, "null argument");
    HIP_TRY(hipMemcpyAsync(state, s->rng, 4 * sizeof(uint64_t), hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return WICK_HIP_OK;
}

int wick_hip_sampler_last_candidates(wick_hip_sampler *s, int *k, int *keep, uint32_t *ids, float *probs, int cap) {
    if (!s || !k || !keep) return set_error(WICK_HIP_EINVAL, "null argument");
    int meta[4];
    HIP_TRY(hipMemcpyAsync(meta, s->meta, sizeof meta, hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    if (meta[2] != 0) return set_error(WICK_HIP_EDEVICE, "sampler candidate count check failed (%d)", meta[2]);
    *k = meta[0];
    *keep = meta[1];
    const int n = meta[0] < cap ? meta[0] : cap;
    if (n > 0 && ids)
        HIP_TRY(hipMemcpyAsync(ids, s->res_idx, (size_t)n * sizeof(uint32_t), hipMemcpyDeviceToHost, s->stream));
    if (n > 0 && probs)
        HIP_TRY(hipMemcpyAsync(probs, s->res_prob, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return WICK_HIP_OK;
}

}  // extern "C"
