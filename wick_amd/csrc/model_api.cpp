// model_api.cpp -- the C ABI of include/wick_hip_model.h: a device-resident
// Model::forward (/root/reference/src/model.rs:420-516) built from the
// kernels of model.hip and the attention path of wick_hip.h.
//
// Per layer and chunk of t tokens the stream runs:
//   gemv  attn_norm + [wq; wk; wv]   -> q, k, v       (src/model.rs:449-462)
//   attend_model: bias, QK-norm, RoPE, cache append, attention (:464-485); for
//                 one token the preparation is the decode kernel's prologue
//   gemv  wo, residual add into x                      (:486-487)
//   gemv  ffn_norm + w_gate, w_up, silu_mul -> h       (:490-501)
//   gemv  w_down, residual add into x                  (:502-503)
// For one token over a short cache (one decode chunk per unit, head_dim 64 or
// 128, small GQA groups) the attention and the wo product are one launch that
// writes each unit's partial product, and the gate/up product adds those to
// the residual as its prologue: four launches per layer instead of five.
// then the final norm + LM head (:507-515) and, for the greedy entry points,
// sampler::argmax (src/sampler.rs:129-137), all on the model's stream.
#include "wick_hip_model.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "attn_kernels.h"
#include "model_kernels.h"
#include "sampler_kernels.h"

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

#define RC_TRY(expr)          \
    do {                      \
        int rc_ = (expr);     \
        if (rc_) return rc_;  \
    } while (0)

enum { T_ATTN_NORM, T_WQ, T_WK, T_WV, T_WO, T_BQ, T_BK, T_BV, T_QN, T_KN, T_FFN_NORM, T_GATE, T_UP, T_DOWN };

constexpr int kPrefillChunk = 256;  // Session::prefill's CHUNK (src/engine.rs:107)

}  // namespace

struct wick_hip_model {
    wick_hip_model_config c{};
    int qd = 0, kvd = 0;
    hipStream_t stream = nullptr;
    std::vector<float> inv_freq;
    // host copies of the per-layer preparation constants, registered on every cache
    struct Prep {
        std::vector<float> bq, bk, bv, qn, kn;
    };
    std::vector<Prep> prep;
    // device weights
    struct Layer {
        float *attn_norm = nullptr, *wqkv = nullptr, *wo = nullptr, *ffn_norm = nullptr;
        float *w_gate = nullptr, *w_up = nullptr, *w_down = nullptr;
    };
    std::vector<Layer> layers;
    float *embed = nullptr, *lm_head = nullptr, *norm = nullptr;
    std::vector<void *> allocs;
    // activations, sized for `cap_t` tokens
    int cap_t = 0;
    float *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *h = nullptr;
    // one token with the output projection fused into the decode kernel: the
    // per-unit partial products [units][hidden] and the residual after them
    float *oparts = nullptr, *xr = nullptr;
    int cap_logits = 0;  // rows of logits
    float *logits = nullptr;
    float *argparts = nullptr;  // the LM head's argmax pairs for the last token (argmax_parts(vocab) of them)
    int cap_ids = 0;
    uint32_t *ids = nullptr;  // token ids on the device (prompt, or the greedy chain)
    uint32_t *pinned_id = nullptr;  // page-locked slot the generate loop reads ids through
    int *counters = nullptr;        // [step, cache length] read by a replayed decode step
};

namespace {

int upload(wick_hip_model *m, float **dst, const float *src, size_t n, const char *what) {
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, n * sizeof(float));
    if (e != hipSuccess) return hip_fail(e, what);
    m->allocs.push_back(p);
    *dst = (float *)p;
    if (src) HIP_TRY(hipMemcpy(p, src, n * sizeof(float), hipMemcpyHostToDevice));
    return WICK_HIP_OK;
}

void free_activations(wick_hip_model *m) {
    void *bufs[] = {m->x, m->xn, m->q, m->k, m->v, m->att, m->h, m->oparts, m->xr};
    for (void *b : bufs)
        if (b) (void)hipFree(b);
    m->x = m->xn = m->q = m->k = m->v = m->att = m->h = m->oparts = m->xr = nullptr;
    m->cap_t = 0;
}

int ensure_activations(wick_hip_model *m, int t) {
    if (t <= m->cap_t) return WICK_HIP_OK;
    HIP_TRY(hipStreamSynchronize(m->stream));  // nothing queued may still use the old buffers
    free_activations(m);
    const wick_hip_model_config &c = m->c;
    struct {
        float **p;
        size_t n;
    } want[] = {{&m->x, (size_t)c.hidden},  {&m->xn, (size_t)c.hidden}, {&m->q, (size_t)m->qd},
                {&m->k, (size_t)m->kvd},    {&m->v, (size_t)m->kvd},    {&m->att, (size_t)m->qd},
                {&m->h, (size_t)c.intermediate}};
    for (auto &w : want) {
        hipError_t e = hipMalloc(w.p, (size_t)t * w.n * sizeof(float));
        if (e != hipSuccess) {
            free_activations(m);
            return hip_fail(e, "hipMalloc(activations)");
        }
    }
    const int group = c.heads / c.kv_heads;
    const size_t units = (size_t)c.kv_heads * ((group + wick::kTileRows - 1) / wick::kTileRows);
    struct {
        float **p;
        size_t n;
    } one[] = {{&m->oparts, units * c.hidden}, {&m->xr, (size_t)c.hidden}};
    for (auto &w : one) {
        hipError_t e = hipMalloc(w.p, w.n * sizeof(float));
        if (e != hipSuccess) {
            free_activations(m);
            return hip_fail(e, "hipMalloc(activations)");
        }
    }
    m->cap_t = t;
    return WICK_HIP_OK;
}

int ensure_logits(wick_hip_model *m, int rows) {
    if (!m->argparts)
        HIP_TRY(hipMalloc(&m->argparts, (size_t)2 * wick::argmax_parts(m->c.vocab) * sizeof(float)));
    if (rows <= m->cap_logits) return WICK_HIP_OK;
    HIP_TRY(hipStreamSynchronize(m->stream));
    if (m->logits) (void)hipFree(m->logits);
    m->logits = nullptr;
    m->cap_logits = 0;
    HIP_TRY(hipMalloc(&m->logits, (size_t)rows * m->c.vocab * sizeof(float)));
    m->cap_logits = rows;
    return WICK_HIP_OK;
}

int ensure_ids(wick_hip_model *m, int n) {
    if (n <= m->cap_ids) return WICK_HIP_OK;
    HIP_TRY(hipStreamSynchronize(m->stream));
    if (m->ids) (void)hipFree(m->ids);
    m->ids = nullptr;
    m->cap_ids = 0;
    HIP_TRY(hipMalloc(&m->ids, (size_t)n * sizeof(uint32_t)));
    m->cap_ids = n;
    return WICK_HIP_OK;
}

int check_cache(const wick_hip_model *m, const wick_hip_kv *kv, int start, int t) {
    wick::KvInfo ki;
    if (!wick::kv_info(kv, &ki)) return set_error(WICK_HIP_EINVAL, "null cache handle");
    if (ki.layers != m->c.layers || ki.kv_heads != m->c.kv_heads || ki.head_dim != m->c.head_dim)
        return set_error(WICK_HIP_EINVAL, "cache shape (%d layers, %d kv heads, head_dim %d) does not match the model",
                         ki.layers, ki.kv_heads, ki.head_dim);
    if (ki.stream != m->stream)
        return set_error(WICK_HIP_EINVAL, "cache launches on another stream (make it with wick_hip_model_new_cache)");
    if (t < 1) return set_error(WICK_HIP_EINVAL, "t must be >= 1 (got %d)", t);
    if (start < 0 || (long long)start + t > ki.capacity)
        return set_error(WICK_HIP_EINVAL, "positions %d..%lld exceed the cache capacity %d (context length exceeded)",
                         start, (long long)start + t, ki.capacity);
    return WICK_HIP_OK;
}

// Prompt chunks of at least this many tokens run their products on the matrix
// cores (gemm_kernel, after a separate RMSNorm pass); shorter ones stream the
// weights through gemv_kernel, 4 tokens per pass.
constexpr int kGemmMinTokens = 16;

// One product with a fused epilogue.  g.norm (optional) is the RMSNorm applied
// to each input row: fused into the GEMV, or a separate pass into m->xn first.
int product(wick_hip_model *m, int epi, wick::GemvArgs g, const char *what) {
    hipError_t e;
    if (g.t >= kGemmMinTokens && g.cols % 16 == 0) {
        if (g.norm) {
            if ((e = wick::launch_rmsnorm(g.x, g.norm, g.eps, m->xn, g.t, g.cols, m->stream)) != hipSuccess)
                return hip_fail(e, "rmsnorm launch");
            g.x = m->xn;
            g.norm = nullptr;
        }
        e = wick::launch_gemm(epi, g, m->stream);
    } else {
        e = wick::launch_gemv(epi, g, m->stream);
    }
    if (e != hipSuccess) return hip_fail(e, what);
    return WICK_HIP_OK;
}

// Model::forward for t tokens whose ids are on the device; logits of the last
// token (or of all t when all_logits) go to m->logits.  Queued on m->stream.
// With counters (t = 1, a step captured for replay) the token is
// tok_dev[counters[0]] and the cache length counters[1]; start only picks the
// decode plan, and no buffer may need to grow.  embedded (t = 1): m->x already
// holds the token's embedding row (the previous greedy step's argmax wrote it).
int forward_device(wick_hip_model *m, wick_hip_kv *kv, const uint32_t *tok_dev, int t, int start, bool all_logits,
                   int *counters = nullptr, bool embedded = false) {
    const wick_hip_model_config &c = m->c;
    const hipStream_t s = m->stream;
    RC_TRY(ensure_activations(m, t));
    RC_TRY(ensure_logits(m, all_logits ? t : 1));
    if (!embedded) {
        hipError_t e = wick::launch_embed(m->embed, tok_dev, m->x, t, c.hidden, s, counters);
        if (e != hipSuccess) return hip_fail(e, "embed kernel launch");
    }
    // the gate/up product takes at most kMaxParts partial vectors of up to
    // 2048 floats (its input row in one pass)
    const int group = c.heads / c.kv_heads;
    const bool fusable = t == 1 && c.kv_heads * ((group + wick::kTileRows - 1) / wick::kTileRows) <= wick::kMaxParts &&
                         c.hidden <= 2048;
    for (int li = 0; li < c.layers; li++) {
        const wick_hip_model::Layer &L = m->layers[li];
        wick::GemvArgs g{};
        g.x = m->x;
        g.norm = L.attn_norm;
        g.eps = c.rms_eps;
        g.w = L.wqkv;
        g.out0 = m->q;
        g.out1 = m->k;
        g.out2 = m->v;
        g.ld0 = m->qd;
        g.ld1 = g.ld2 = m->kvd;
        g.split0 = m->qd;
        g.split1 = m->qd + m->kvd;
        g.rows = m->qd + 2 * m->kvd;
        g.cols = c.hidden;
        g.t = t;
        RC_TRY(product(m, wick::kEpiQkv, g, "qkv product launch"));

        // One token: attention and the output projection in one launch
        // (per-unit partial products), added to the residual by the gate/up
        // product's prologue; the down product then adds to that sum.
        int units = 0;
        const int fused = fusable ? wick::attend_model_oproj(kv, li, c.heads, m->q, m->k, m->v, start, L.wo, c.hidden,
                                                             m->oparts, &units, counters ? counters + 1 : nullptr)
                                  : 1;
        if (fused < 0) return fused;
        if (fused == 0) {
            g = wick::GemvArgs{};
            g.x = m->x;
            g.parts = m->oparts;
            g.nparts = units;
            g.xout = m->xr;
            g.norm = L.ffn_norm;
            g.eps = c.rms_eps;
            g.w = L.w_gate;
            g.w2 = L.w_up;
            g.out0 = m->h;
            g.ld0 = c.intermediate;
            g.rows = c.intermediate;
            g.cols = c.hidden;
            g.t = 1;
            RC_TRY(product(m, wick::kEpiSwiglu, g, "residual + gate/up product launch"));

            g = wick::GemvArgs{};
            g.x = m->h;
            g.w = L.w_down;
            g.resid = m->xr;
            g.out0 = m->x;
            g.ld0 = c.hidden;
            g.rows = c.hidden;
            g.cols = c.intermediate;
            g.t = 1;
            RC_TRY(product(m, wick::kEpiResid, g, "down product launch"));
            continue;
        }

        RC_TRY(wick::attend_model(kv, li, c.heads, m->q, m->k, m->v, t, start, m->att, counters ? counters + 1 : nullptr));

        g = wick::GemvArgs{};
        g.x = m->att;
        g.w = L.wo;
        g.out0 = m->x;
        g.ld0 = c.hidden;
        g.rows = c.hidden;
        g.cols = m->qd;
        g.t = t;
        RC_TRY(product(m, wick::kEpiResid, g, "o product launch"));

        g = wick::GemvArgs{};
        g.x = m->x;
        g.norm = L.ffn_norm;
        g.eps = c.rms_eps;
        g.w = L.w_gate;
        g.w2 = L.w_up;
        g.out0 = m->h;
        g.ld0 = c.intermediate;
        g.rows = c.intermediate;
        g.cols = c.hidden;
        g.t = t;
        RC_TRY(product(m, wick::kEpiSwiglu, g, "gate/up product launch"));

        g = wick::GemvArgs{};
        g.x = m->h;
        g.w = L.w_down;
        g.out0 = m->x;
        g.ld0 = c.hidden;
        g.rows = c.hidden;
        g.cols = c.intermediate;
        g.t = t;
        RC_TRY(product(m, wick::kEpiResid, g, "down product launch"));
    }
    wick::GemvArgs g{};
    g.x = all_logits ? m->x : m->x + (size_t)(t - 1) * c.hidden;
    g.norm = m->norm;
    g.eps = c.rms_eps;
    g.w = m->lm_head;
    g.out0 = m->logits;
    g.ld0 = c.vocab;
    g.rows = c.vocab;
    g.cols = c.hidden;
    g.t = all_logits ? t : 1;
    if (all_logits) {
        RC_TRY(product(m, wick::kEpiStore, g, "lm head product launch"));
    } else {
        g.out1 = m->argparts;  // the first greedy step rides along with the product
        RC_TRY(product(m, wick::kEpiArgmax, g, "lm head product launch"));
    }
    return WICK_HIP_OK;
}

// Host ids -> m->ids[0..n).  Waits for the copy, so the host array may go
// away on any later error return.
int upload_ids(wick_hip_model *m, const uint32_t *ids, int n) {
    HIP_TRY(hipMemcpyAsync(m->ids, ids, (size_t)n * sizeof(uint32_t), hipMemcpyHostToDevice, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return WICK_HIP_OK;
}

// Fewest steps worth replaying from a captured graph.  A run of equal-plan
// steps launches its first step directly (it makes any allocation the step
// needs, and the capture is taken from the same launch code); the remaining
// steps are replayed when there are at least this many of them, else they
// launch directly too (capture and instantiation cost about as much as ~20
// steps' worth of launch gaps save).
constexpr int kGraphMinSteps = 24;

// Greedy step i of a decode loop, launched directly: forward of ids[i] at
// position start + i (its embedding row already in m->x when `embedded`),
// argmax into ids[i + 1], whose embedding row the argmax leaves in m->x for
// the next step.
int decode_step(wick_hip_model *m, wick_hip_kv *kv, int start, int i, bool embedded) {
    RC_TRY(forward_device(m, kv, m->ids + i, 1, start + i, false, nullptr, embedded));
    hipError_t e = wick::launch_argmax(m->logits, m->c.vocab, m->ids + i + 1, m->stream, nullptr, nullptr, m->argparts,
                                       m->embed, m->x, m->c.hidden);
    if (e != hipSuccess) return hip_fail(e, "argmax launch");
    return WICK_HIP_OK;
}

// Steps i0..i1-1 (one decode plan) from one captured step replayed as a HIP
// graph: each replay reads its token index and cache length from
// m->counters, which its argmax advances; m->x holds ids[i0]'s embedding row
// (the previous step's argmax wrote it) and each replay's argmax writes the
// next one.  The graph holds no memset node and is destroyed before returning
// (it bakes in this call's buffers).
int decode_replayed(wick_hip_model *m, wick_hip_kv *kv, int start, int i0, int i1) {
    if (!m->counters) HIP_TRY(hipMalloc(&m->counters, 2 * sizeof(int)));
    hipGraph_t graph = nullptr;
    HIP_TRY(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    int rc = forward_device(m, kv, m->ids, 1, start + i0, false, m->counters, true);
    if (!rc) {
        hipError_t e = wick::launch_argmax(m->logits, m->c.vocab, m->ids, m->stream, m->counters, m->counters + 1,
                                           m->argparts, m->embed, m->x, m->c.hidden);
        if (e != hipSuccess) rc = hip_fail(e, "argmax launch");
    }
    hipError_t e = hipStreamEndCapture(m->stream, &graph);
    if (rc) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    e = wick::launch_set_step(m->counters, i0, start + i0 + 1, m->stream);
    for (int k = i0; k < i1 && e == hipSuccess; k++) e = hipGraphLaunch(exec, m->stream);
    // the replays must finish before the graph goes
    const hipError_t es = hipStreamSynchronize(m->stream);
    (void)hipGraphExecDestroy(exec);
    if (e != hipSuccess) return hip_fail(e, "decode step replay");
    if (es != hipSuccess) return hip_fail(es, "hipStreamSynchronize");
    return WICK_HIP_OK;
}

int check_tokens(const wick_hip_model *m, const uint32_t *tokens, int n) {
    for (int i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)m->c.vocab)
            return set_error(WICK_HIP_EINVAL, "token %u at %d is outside the vocabulary (%d)", tokens[i], i, m->c.vocab);
    return WICK_HIP_OK;
}

}  // namespace

extern "C" {

int wick_hip_model_create(const wick_hip_model_config *cfg, const float *inv_freq, const float *embed,
                          const float *lm_head, const float *norm, const float *const *layer_tensors,
                          wick_hip_model **out) {
    if (!out) return set_error(WICK_HIP_EINVAL, "null output pointer");
    *out = nullptr;
    if (!cfg || !inv_freq || !embed || !norm || !layer_tensors) return set_error(WICK_HIP_EINVAL, "null argument");
    const wick_hip_model_config c = *cfg;
    if (c.hidden < 4 || c.layers < 1 || c.heads < 1 || c.kv_heads < 1 || c.intermediate < 4 || c.vocab < 1)
        return set_error(WICK_HIP_EINVAL, "non-positive model dimension");
    if (c.heads % c.kv_heads != 0)
        return set_error(WICK_HIP_EINVAL, "heads (%d) must be a multiple of kv_heads (%d)", c.heads, c.kv_heads);
    if (c.head_dim != 16 && c.head_dim != 32 && c.head_dim != 64 && c.head_dim != 128)
        return set_error(WICK_HIP_EINVAL, "head_dim %d not supported (16, 32, 64, 128)", c.head_dim);
    if (c.hidden % 4 || c.intermediate % 4)
        return set_error(WICK_HIP_EINVAL, "hidden and intermediate must be multiples of 4");
    if (!(c.rms_eps >= 0.0f)) return set_error(WICK_HIP_EINVAL, "rms_eps must be >= 0");
    for (int li = 0; li < c.layers; li++) {
        const float *const *t = layer_tensors + (size_t)li * WICK_HIP_MODEL_LAYER_TENSORS;
        const int required[] = {T_ATTN_NORM, T_WQ, T_WK, T_WV, T_WO, T_FFN_NORM, T_GATE, T_UP, T_DOWN};
        for (int r : required)
            if (!t[r]) return set_error(WICK_HIP_EINVAL, "layer %d: required tensor %d is null", li, r);
        const int nb = (t[T_BQ] != nullptr) + (t[T_BK] != nullptr) + (t[T_BV] != nullptr);
        if (nb != 0 && nb != 3) return set_error(WICK_HIP_EINVAL, "layer %d: give all of bq, bk, bv or none", li);
        if ((t[T_QN] != nullptr) != (t[T_KN] != nullptr))
            return set_error(WICK_HIP_EINVAL, "layer %d: give both q_norm and k_norm or neither", li);
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) return set_error(WICK_HIP_EDEVICE, "no HIP device");

    auto *m = new wick_hip_model();
    m->c = c;
    m->qd = c.heads * c.head_dim;
    m->kvd = c.kv_heads * c.head_dim;
    m->inv_freq.assign(inv_freq, inv_freq + c.head_dim / 2);
    int rc = WICK_HIP_OK;
    do {
        hipError_t e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            rc = hip_fail(e, "hipStreamCreate");
            break;
        }
        const size_t h = c.hidden, qd = m->qd, kvd = m->kvd, ff = c.intermediate;
        if ((rc = upload(m, &m->embed, embed, (size_t)c.vocab * h, "embed"))) break;
        if ((rc = upload(m, &m->norm, norm, h, "norm"))) break;
        if (lm_head) {
            if ((rc = upload(m, &m->lm_head, lm_head, (size_t)c.vocab * h, "lm_head"))) break;
        } else {
            m->lm_head = m->embed;  // tied (src/model.rs:190-192)
        }
        m->layers.resize(c.layers);
        m->prep.resize(c.layers);
        for (int li = 0; li < c.layers && rc == WICK_HIP_OK; li++) {
            const float *const *t = layer_tensors + (size_t)li * WICK_HIP_MODEL_LAYER_TENSORS;
            wick_hip_model::Layer &L = m->layers[li];
            if ((rc = upload(m, &L.attn_norm, t[T_ATTN_NORM], h, "attn_norm"))) break;
            // [wq; wk; wv] as one [qd + 2 kvd][hidden] matrix: one pass over xn
            if ((rc = upload(m, &L.wqkv, nullptr, (qd + 2 * kvd) * h, "wqkv"))) break;
            if ((e = hipMemcpy(L.wqkv, t[T_WQ], qd * h * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess ||
                (e = hipMemcpy(L.wqkv + qd * h, t[T_WK], kvd * h * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess ||
                (e = hipMemcpy(L.wqkv + (qd + kvd) * h, t[T_WV], kvd * h * sizeof(float), hipMemcpyHostToDevice)) !=
                    hipSuccess) {
                rc = hip_fail(e, "hipMemcpy(wqkv)");
                break;
            }
            if ((rc = upload(m, &L.wo, t[T_WO], h * qd, "wo"))) break;
            if ((rc = upload(m, &L.ffn_norm, t[T_FFN_NORM], h, "ffn_norm"))) break;
            if ((rc = upload(m, &L.w_gate, t[T_GATE], ff * h, "w_gate"))) break;
            if ((rc = upload(m, &L.w_up, t[T_UP], ff * h, "w_up"))) break;
            if ((rc = upload(m, &L.w_down, t[T_DOWN], h * ff, "w_down"))) break;
            wick_hip_model::Prep &p = m->prep[li];
            if (t[T_BQ]) {
                p.bq.assign(t[T_BQ], t[T_BQ] + qd);
                p.bk.assign(t[T_BK], t[T_BK] + kvd);
                p.bv.assign(t[T_BV], t[T_BV] + kvd);
            }
            if (t[T_QN]) {
                p.qn.assign(t[T_QN], t[T_QN] + c.head_dim);
                p.kn.assign(t[T_KN], t[T_KN] + c.head_dim);
            }
        }
    } while (0);
    if (rc != WICK_HIP_OK) {
        wick_hip_model_destroy(m);
        return rc;
    }
    *out = m;
    return WICK_HIP_OK;
}

void wick_hip_model_destroy(wick_hip_model *m) {
    if (!m) return;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    free_activations(m);
    if (m->logits) (void)hipFree(m->logits);
    if (m->argparts) (void)hipFree(m->argparts);
    if (m->ids) (void)hipFree(m->ids);
    if (m->pinned_id) (void)hipHostFree(m->pinned_id);
    if (m->counters) (void)hipFree(m->counters);
    for (void *p : m->allocs) (void)hipFree(p);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

int wick_hip_model_new_cache(wick_hip_model *m, int capacity, wick_hip_kv **out) {
    if (!m || !out) return set_error(WICK_HIP_EINVAL, "null argument");
    *out = nullptr;
    wick_hip_kv *kv = nullptr;
    RC_TRY(wick_hip_kv_create(m->c.layers, capacity, m->c.kv_heads, m->c.head_dim, &kv));
    int rc = wick_hip_kv_set_stream(kv, m->stream);
    if (!rc) rc = wick_hip_kv_set_rope(kv, m->inv_freq.data());
    for (int li = 0; !rc && li < m->c.layers; li++) {
        const wick_hip_model::Prep &p = m->prep[li];
        auto ptr = [](const std::vector<float> &v) { return v.empty() ? nullptr : v.data(); };
        rc = wick_hip_kv_set_prep(kv, li, m->c.heads, ptr(p.bq), ptr(p.bk), ptr(p.bv), ptr(p.qn), ptr(p.kn),
                                  m->c.rms_eps);
    }
    if (rc) {
        wick_hip_kv_destroy(kv);
        return rc;
    }
    *out = kv;
    return WICK_HIP_OK;
}

int wick_hip_model_forward(wick_hip_model *m, wick_hip_kv *kv, const uint32_t *tokens, int t, int start,
                           int all_logits, float *logits) {
    if (!m || !tokens || !logits) return set_error(WICK_HIP_EINVAL, "null argument");
    RC_TRY(check_cache(m, kv, start, t));
    RC_TRY(check_tokens(m, tokens, t));
    RC_TRY(ensure_ids(m, t));
    RC_TRY(upload_ids(m, tokens, t));
    RC_TRY(forward_device(m, kv, m->ids, t, start, all_logits != 0));
    const size_t n = (size_t)(all_logits ? t : 1) * m->c.vocab;
    HIP_TRY(hipMemcpyAsync(logits, m->logits, n * sizeof(float), hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return WICK_HIP_OK;
}

int wick_hip_model_prefill(wick_hip_model *m, wick_hip_kv *kv, const uint32_t *prompt, int n, int start,
                           uint32_t *next) {
    if (!m || !prompt || !next) return set_error(WICK_HIP_EINVAL, "null argument");
    RC_TRY(check_cache(m, kv, start, n));
    RC_TRY(check_tokens(m, prompt, n));
    RC_TRY(ensure_ids(m, n + 1));
    RC_TRY(upload_ids(m, prompt, n));
    for (int off = 0; off < n; off += kPrefillChunk) {
        const int t = std::min(kPrefillChunk, n - off);
        RC_TRY(forward_device(m, kv, m->ids + off, t, start + off, false));
    }
    hipError_t e = wick::launch_argmax(m->logits, m->c.vocab, m->ids + n, m->stream, nullptr, nullptr, m->argparts);
    if (e != hipSuccess) return hip_fail(e, "argmax launch");
    HIP_TRY(hipMemcpyAsync(next, m->ids + n, sizeof(uint32_t), hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return WICK_HIP_OK;
}

int wick_hip_model_decode(wick_hip_model *m, wick_hip_kv *kv, uint32_t first, int start, int steps, uint32_t *out) {
    if (!m || !out) return set_error(WICK_HIP_EINVAL, "null argument");
    if (steps < 1) return set_error(WICK_HIP_EINVAL, "steps must be >= 1");
    RC_TRY(check_cache(m, kv, start, steps));
    RC_TRY(check_tokens(m, &first, 1));
    RC_TRY(ensure_ids(m, steps + 1));
    RC_TRY(upload_ids(m, &first, 1));
    int i = 0;
    while (i < steps) {
        // steps i..j-1 share the decode plan: all but the first run from one
        // captured step (the first, launched directly, makes any allocation
        // the step needs)
        const long long plan = wick::decode_plan_key(kv, m->c.heads, start + i + 1);
        int j = i + 1;
        while (j < steps && wick::decode_plan_key(kv, m->c.heads, start + j + 1) == plan) j++;
        // the loop's first step embeds its token; every argmax leaves the next
        // token's embedding row in m->x
        RC_TRY(decode_step(m, kv, start, i, i > 0));
        if (j - (i + 1) >= kGraphMinSteps) {
            RC_TRY(decode_replayed(m, kv, start, i + 1, j));
        } else {
            for (int k = i + 1; k < j; k++) RC_TRY(decode_step(m, kv, start, k, true));
        }
        i = j;
    }
    HIP_TRY(hipMemcpyAsync(out, m->ids + 1, (size_t)steps * sizeof(uint32_t), hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return WICK_HIP_OK;
}

int wick_hip_model_new_sampler(wick_hip_model *m, const wick_hip_sampler_config *cfg, wick_hip_sampler **out) {
    if (!m) return set_error(WICK_HIP_EINVAL, "null argument");
    return wick_hip_sampler_create(cfg, m->c.vocab, m->stream, out);
}

int wick_hip_model_generate(wick_hip_model *m, wick_hip_kv *kv, wick_hip_sampler *s, const uint32_t *tokens, int n,
                            int start, int max_tokens, const uint32_t *stops, int n_stops, uint32_t *out, int *n_out,
                            int *cache_len) {
    if (!m || !s || !tokens || !n_out || !cache_len || (max_tokens > 0 && !out))
        return set_error(WICK_HIP_EINVAL, "null argument");
    if (max_tokens < 0) return set_error(WICK_HIP_EINVAL, "max_tokens must be >= 0 (got %d)", max_tokens);
    if (n_stops < 0 || (n_stops > 0 && !stops)) return set_error(WICK_HIP_EINVAL, "bad stop list");
    if (wick::sampler_stream(s) != m->stream)
        return set_error(WICK_HIP_EINVAL, "sampler launches on another stream (make it with wick_hip_model_new_sampler)");
    if (wick::sampler_vocab(s) != m->c.vocab)
        return set_error(WICK_HIP_EINVAL, "sampler vocabulary %d != model vocabulary %d", wick::sampler_vocab(s),
                         m->c.vocab);
    if (start < 0 || start >= n)
        return set_error(WICK_HIP_EINVAL, "start %d must be in [0, n = %d): the last token is run for its logits",
                         start, n);
    RC_TRY(check_cache(m, kv, start, n - start));
    RC_TRY(check_tokens(m, tokens, n));
    wick::KvInfo ki;
    wick::kv_info(kv, &ki);
    max_tokens = std::min(max_tokens, ki.capacity - n);  // room (src/engine.rs:167-168)
    *n_out = 0;
    *cache_len = n;
    RC_TRY(ensure_ids(m, n + std::max(max_tokens, 1)));
    RC_TRY(upload_ids(m, tokens, n));
    for (int off = start; off < n; off += kPrefillChunk) {
        const int t = std::min(kPrefillChunk, n - off);
        RC_TRY(forward_device(m, kv, m->ids + off, t, off, false));
    }
    const bool history = wick::sampler_reads_history(s);
    auto step = [&](int j) -> int {
        RC_TRY(wick::sampler_enqueue(s, m->logits, m->ids, history ? n + j : 0, m->ids + n + j));
        if (n_stops > 0) {
            HIP_TRY(hipMemcpyAsync(m->pinned_id, m->ids + n + j, sizeof(uint32_t), hipMemcpyDeviceToHost, m->stream));
        }
        return WICK_HIP_OK;
    };
    if (n_stops == 0) {
        for (int j = 0; j < max_tokens; j++) {
            RC_TRY(step(j));
            if (j + 1 < max_tokens) RC_TRY(forward_device(m, kv, m->ids + n + j, 1, n + j, false));
        }
        if (max_tokens > 0)
            HIP_TRY(hipMemcpyAsync(out, m->ids + n, (size_t)max_tokens * sizeof(uint32_t), hipMemcpyDeviceToHost,
                                   m->stream));
        HIP_TRY(hipStreamSynchronize(m->stream));
        *n_out = max_tokens;
        *cache_len = n + std::max(max_tokens - 1, 0);
        return WICK_HIP_OK;
    }
    if (!m->pinned_id) HIP_TRY(hipHostMalloc((void **)&m->pinned_id, 64, hipHostMallocDefault));
    hipEvent_t ev = nullptr;
    HIP_TRY(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    int rc = WICK_HIP_OK;
    for (int j = 0; j < max_tokens && !rc; j++) {
        if ((rc = step(j))) break;
        hipError_t e = hipEventRecord(ev, m->stream);
        // queue the next forward before reading the id, so the GPU keeps working
        if (e == hipSuccess && j + 1 < max_tokens) rc = forward_device(m, kv, m->ids + n + j, 1, n + j, false);
        if (e == hipSuccess && !rc) e = hipEventSynchronize(ev);
        if (e != hipSuccess) {
            rc = hip_fail(e, "generate: reading the drawn id");
            break;
        }
        if (rc) break;
        const uint32_t tok = *m->pinned_id;
        if (std::find(stops, stops + n_stops, tok) != stops + n_stops) break;
        out[j] = tok;
        *n_out = j + 1;
        *cache_len = n + (j + 1 < max_tokens ? j + 1 : j);
    }
    hipError_t e = hipStreamSynchronize(m->stream);
    (void)hipEventDestroy(ev);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "generate");
    return rc;
}

}  // extern "C"
