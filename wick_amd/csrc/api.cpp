// api.cpp -- the C ABI of include/wick_hip.h over the HIP kernels.
//
// Every entry point validates its arguments on the host before anything is
// launched (a kernel never sees a shape it was not written for), turns HIP
// failures into status codes, and records a message for wick_hip_last_error().
#include "wick_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <cmath>
#include <string>
#include <vector>

#include "attn_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(e == hipErrorOutOfMemory ? WICK_HIP_ENOMEM : WICK_HIP_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr)                                   \
    do {                                                \
        hipError_t e_ = (expr);                         \
        if (e_ != hipSuccess) return hip_fail(e_, #expr); \
    } while (0)

bool supported_head_dim(int d) { return d == 16 || d == 32 || d == 64 || d == 128; }

}  // namespace

struct wick_hip_kv {
    int layers = 0, capacity = 0, kv_heads = 0, head_dim = 0;
    int device = 0, num_cus = 256;
    float *k = nullptr, *v = nullptr;  // [layers][kv_heads][capacity][head_dim]
    hipStream_t own_stream = nullptr, stream = nullptr;
    // staging for the host-pointer entry points
    float *q_dev = nullptr, *att_dev = nullptr, *kst_dev = nullptr, *vst_dev = nullptr;
    size_t q_cap = 0, att_cap = 0, kst_cap = 0;
    // wick_hip_attention / wick_hip_attend: the call's inputs and output in one
    // pinned host block and one device block, so each call makes one copy
    // each way, both DMA from pinned memory
    float *io_dev = nullptr, *io_host = nullptr;
    size_t io_cap = 0, io_host_cap = 0;
    // decode split-K workspace (partial softmax states of the chunks)
    float *part = nullptr;
    int ws_units = 0;
    // whether the static workspace's address was found on this device
    hipError_t static_rc = hipErrorNotInitialized;
    // options
    int decode_chunk = 0, decode_interleave = 1, last_grid = 0;
    int decode_blocks_per_cu = 1, prefill_blocks_per_cu = 1, prefill2_blocks_per_cu = 1;
    // input preparation (wick_hip_kv_set_rope / wick_hip_kv_set_prep)
    float *rope_cos = nullptr, *rope_sin = nullptr;  // [capacity][head_dim/2]
    struct LayerPrep {
        float *buf = nullptr;  // bq [heads*D] | bk [kvd] | bv [kvd] | q_norm [D] | k_norm [D]
        int heads = 0;
        bool set = false, bias = false, norm = false;
        float eps = 0.0f;
    };
    std::vector<LayerPrep> prep;

    size_t layer_floats() const { return (size_t)kv_heads * capacity * head_dim; }
    float *k_layer(int l) const { return k + (size_t)l * layer_floats(); }
    float *v_layer(int l) const { return v + (size_t)l * layer_floats(); }
};

namespace {

int grow(hipStream_t stream, float **buf, size_t *cap, size_t need, const char *what) {
    if (need <= *cap) return WICK_HIP_OK;
    // work queued earlier on the handle's stream may still read the old buffer
    if (*buf) {
        hipError_t e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        (void)hipFree(*buf);
    }
    *buf = nullptr;
    *cap = 0;
    hipError_t e = hipMalloc(buf, need * sizeof(float));
    if (e != hipSuccess) return hip_fail(e, what);
    *cap = need;
    return WICK_HIP_OK;
}

// The pinned host block and the device block of the host-pointer calls, at
// least `need` floats each.
int ensure_io(wick_hip_kv *kv, size_t need) {
    int rc = grow(kv->stream, &kv->io_dev, &kv->io_cap, need, "hipMalloc(io staging)");
    if (rc || need <= kv->io_host_cap) return rc;
    if (kv->io_host) {
        HIP_TRY(hipStreamSynchronize(kv->stream));  // an earlier copy may still read it
        (void)hipHostFree(kv->io_host);
    }
    kv->io_host = nullptr;
    kv->io_host_cap = 0;
    HIP_TRY(hipHostMalloc(reinterpret_cast<void **>(&kv->io_host), need * sizeof(float), hipHostMallocDefault));
    kv->io_host_cap = need;
    return WICK_HIP_OK;
}

// Decode workspace for `units` (kv head, 16-head slice) pairs.  Grown on
// demand; a decode launch rewrites every state it later reads.
int ensure_workspace(wick_hip_kv *kv, int units) {
    if (units <= kv->ws_units) return WICK_HIP_OK;
    if (kv->part) {
        HIP_TRY(hipStreamSynchronize(kv->stream));  // an earlier decode may still use it
        (void)hipFree(kv->part);
    }
    kv->part = nullptr;
    kv->ws_units = 0;
    HIP_TRY(hipMalloc(&kv->part, wick::decode_workspace_floats(units, kv->head_dim) * sizeof(float)));
    kv->ws_units = units;
    return WICK_HIP_OK;
}

int check_kv(const wick_hip_kv *kv, int layer) {
    if (!kv) return fail(WICK_HIP_EINVAL, "null cache handle");
    if (layer < 0 || layer >= kv->layers) return fail(WICK_HIP_EINVAL, "layer %d out of range [0, %d)", layer, kv->layers);
    return WICK_HIP_OK;
}

// Device arrays handed in by the caller are read and written as float4.
int check_aligned(const void *p, const char *what) {
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return fail(WICK_HIP_EINVAL, "%s is not 16-byte aligned", what);
    return WICK_HIP_OK;
}

int check_span(const wick_hip_kv *kv, int start, int t) {
    if (t < 1) return fail(WICK_HIP_EINVAL, "t must be >= 1 (got %d)", t);
    if (start < 0 || (long long)start + t > kv->capacity)
        return fail(WICK_HIP_EINVAL, "positions %d..%lld exceed the cache capacity %d", start, (long long)start + t,
                    kv->capacity);
    return WICK_HIP_OK;
}

// Chunk size and count of a decode call over len positions for `units`
// (kv head x 16-head slice) workgroup rows.
void plan_chunks(const wick_hip_kv *kv, int units, int len, int *chunk_out, int *nchunks_out) {
    int chunk = kv->decode_chunk, quantum = 16;
    if (chunk <= 0 && len <= wick::kDecodeSingleChunkMax) {
        // Short context: one workgroup per unit and no merge pass.  Its
        // waves (8 at head_dim <= 64, else 4) take at most two tile groups
        // each, which costs less than the second launch a split needs.
        // Whole 64-key chunks, so that a decode loop keeps one launch plan
        // (and one captured graph) over 64 consecutive lengths.
        chunk = len;
        quantum = 64;
    } else if (chunk <= 0) {
        // One resident round: as many chunks as the GPU holds decode
        // workgroups at once, each streaming one long contiguous range.
        // Chunks in 16-key steps let the grid fill the round: the
        // Llama-3-8B shape at 32768 positions takes 94 chunks of 352 keys
        // (752 of 768 resident workgroups) where 64-key steps gave 86 of 384
        // (688).
        const int resident = kv->num_cus * kv->decode_blocks_per_cu;
        const int target = std::max(1, resident / units);
        chunk = (len + target - 1) / target;
    }
    chunk = std::max(64, (chunk + quantum - 1) / quantum * quantum);
    const int min_chunk = (len + wick::kDecodeMaxChunks - 1) / wick::kDecodeMaxChunks;
    if (chunk < min_chunk) chunk = (min_chunk + 15) / 16 * 16;
    *chunk_out = chunk;
    *nchunks_out = (len + chunk - 1) / chunk;
}

// Split-K schedule of one decode call over len positions: fills the shape
// fields of *a and kv->last_grid.
// static_part: the partial states go to the static workspace (no allocation)
// instead of the handle's own.
int plan_decode(wick_hip_kv *kv, int layer, int group, int len, const float *q_dev, float *att_dev,
                wick::DecodeArgs *a, float *static_part = nullptr) {
    const int hslices = (group + wick::kTileRows - 1) / wick::kTileRows;
    const int units = kv->kv_heads * hslices;
    if (static_part) {
        const size_t need = wick::decode_workspace_floats(units, kv->head_dim);
        if (need > wick::kStaticScratchFloats)
            return fail(WICK_HIP_EINVAL,
                        "decode needs %zu floats of workspace for %d kv heads x %d head slices at head_dim %d; the "
                        "static workspace holds %zu",
                        need, kv->kv_heads, hslices, kv->head_dim, wick::kStaticScratchFloats);
    } else {
        int rc = ensure_workspace(kv, units);
        if (rc) return rc;
    }
    int chunk, nchunks;
    plan_chunks(kv, units, len, &chunk, &nchunks);
    a->q = q_dev;
    a->k = kv->k_layer(layer);
    a->v = kv->v_layer(layer);
    a->att = att_dev;
    a->part = static_part ? static_part : kv->part;
    a->capacity = kv->capacity;
    a->len = len;
    a->kv_heads = kv->kv_heads;
    a->group = group;
    a->hslices = hslices;
    a->chunk = chunk;
    a->nchunks = nchunks;
    a->stagger = nchunks > 1 && (long long)units * nchunks >= 2LL * kv->num_cus ? 1 : 0;
    a->interleave = kv->decode_interleave && wick::decode_interleaves(kv->head_dim, group, nchunks, chunk) ? 1 : 0;
    kv->last_grid = units * nchunks;
    return WICK_HIP_OK;
}

int run_attention(wick_hip_kv *kv, int layer, int heads, const float *q_dev, int t, int start, float *att_dev,
                  float *static_part = nullptr) {
    const int D = kv->head_dim;
    if (heads < 1 || heads % kv->kv_heads != 0)
        return fail(WICK_HIP_EINVAL, "heads (%d) must be a positive multiple of kv_heads (%d)", heads, kv->kv_heads);
    const int group = heads / kv->kv_heads;
    const float scale = 1.0f / sqrtf((float)D);  // src/model.rs:527

    if (t == 1) {
        wick::DecodeArgs a{};
        int rc = plan_decode(kv, layer, group, start + 1, q_dev, att_dev, &a, static_part);
        if (rc) return rc;
        a.scale = scale;
        hipError_t e = wick::launch_decode(D, a, kv->last_grid, kv->stream);
        if (e != hipSuccess) return hip_fail(e, "decode kernel launch");
        return WICK_HIP_OK;
    }

    wick::PrefillArgs a{};
    a.q = q_dev;
    a.k = kv->k_layer(layer);
    a.v = kv->v_layer(layer);
    a.att = att_dev;
    a.capacity = kv->capacity;
    a.t = t;
    a.start = start;
    a.kv_heads = kv->kv_heads;
    a.group = group;
    a.nblocks = (t * group + wick::kTileRows - 1) / wick::kTileRows;
    // Two row blocks per workgroup share each loaded tile, where that grid
    // still gives every CU two workgroups; zigzag pairing where the launched
    // grid is resident at once.
    const long long grid1 = (long long)a.kv_heads * a.nblocks, grid2 = (long long)a.kv_heads * ((a.nblocks + 1) / 2);
    a.rows32 = wick::prefill_has_rows32(D, kv->capacity) && grid2 >= 2LL * kv->num_cus ? 1 : 0;
    a.zigzag = (a.rows32 ? grid2 : grid1) <=
                       (long long)kv->num_cus * (a.rows32 ? kv->prefill2_blocks_per_cu : kv->prefill_blocks_per_cu)
                   ? 1
                   : 0;
    a.scale = scale;
    kv->last_grid = wick::prefill_grid(D, a);
    hipError_t e = wick::launch_prefill(D, a, kv->stream);
    if (e != hipSuccess) return hip_fail(e, "prefill kernel launch");
    return WICK_HIP_OK;
}

// Bias, QK-norm and RoPE of q (in place) and k, and the append of k and v
// (src/model.rs:464-484), for tokens at start..start+t of `layer`.
// The registered preparation constants of `layer`, checked against `heads`.
struct PrepConsts {
    const float *bq = nullptr, *bk = nullptr, *bv = nullptr, *qn = nullptr, *kn = nullptr;
    float eps = 0.0f;
};

int prep_consts(const wick_hip_kv *kv, int layer, int heads, PrepConsts *c) {
    if (!kv->rope_cos) return fail(WICK_HIP_EINVAL, "no RoPE table (call wick_hip_kv_set_rope first)");
    const wick_hip_kv::LayerPrep &p = kv->prep[layer];
    if (!p.set) return fail(WICK_HIP_EINVAL, "layer %d has no preparation constants (call wick_hip_kv_set_prep)", layer);
    if (heads != p.heads)
        return fail(WICK_HIP_EINVAL, "heads %d differs from the %d given to wick_hip_kv_set_prep", heads, p.heads);
    const int D = kv->head_dim, kvd = kv->kv_heads * D;
    if (p.bias) {
        c->bq = p.buf;
        c->bk = p.buf + (size_t)heads * D;
        c->bv = c->bk + kvd;
    }
    if (p.norm) {
        c->qn = p.buf + (size_t)heads * D + 2 * kvd;
        c->kn = c->qn + D;
    }
    c->eps = p.eps;
    return WICK_HIP_OK;
}

int run_prep(wick_hip_kv *kv, int layer, int heads, float *q_dev, const float *k_dev, const float *v_dev, int t,
             int start) {
    PrepConsts c;
    int rc = prep_consts(kv, layer, heads, &c);
    if (rc) return rc;
    const int D = kv->head_dim;
    wick::PrepArgs a{};
    a.q = q_dev;
    a.ksrc = k_dev;
    a.vsrc = v_dev;
    a.k = kv->k_layer(layer);
    a.v = kv->v_layer(layer);
    a.bq = c.bq;
    a.bk = c.bk;
    a.bv = c.bv;
    a.qn = c.qn;
    a.kn = c.kn;
    a.rope_cos = kv->rope_cos;
    a.rope_sin = kv->rope_sin;
    a.capacity = kv->capacity;
    a.start = start;
    a.t = t;
    a.heads = heads;
    a.kv_heads = kv->kv_heads;
    a.eps = c.eps;
    hipError_t e = wick::launch_prep(D, a, kv->stream);
    if (e != hipSuccess) return hip_fail(e, "prep kernel launch");
    return WICK_HIP_OK;
}

// One token: the preparation fused into the decode kernel's prologue (q from
// the raw projections, k and v appended at position start), then attention.
int run_decode_fused(wick_hip_kv *kv, int layer, int heads, const float *q_raw, const float *k_raw,
                     const float *v_raw, int start, float *att_dev, const int *len_dev) {
    PrepConsts c;
    int rc = prep_consts(kv, layer, heads, &c);
    if (rc) return rc;
    wick::DecodeArgs a{};
    if ((rc = plan_decode(kv, layer, heads / kv->kv_heads, start + 1, q_raw, att_dev, &a))) return rc;
    a.scale = 1.0f / sqrtf((float)kv->head_dim);  // src/model.rs:527
    a.prep = 1;
    a.kraw = k_raw;
    a.vraw = v_raw;
    a.bq = c.bq;
    a.bk = c.bk;
    a.bv = c.bv;
    a.qn = c.qn;
    a.kn = c.kn;
    a.rope_cos = kv->rope_cos;
    a.rope_sin = kv->rope_sin;
    a.eps = c.eps;
    a.len_dev = len_dev;
    hipError_t e = wick::launch_decode(kv->head_dim, a, kv->last_grid, kv->stream);
    if (e != hipSuccess) return hip_fail(e, "decode kernel launch");
    return WICK_HIP_OK;
}

}  // namespace

namespace wick {

int set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int attend_model(wick_hip_kv *kv, int layer, int heads, float *q_dev, const float *k_dev, const float *v_dev, int t,
                 int start, float *att_dev, const int *len_dev) {
    int rc = check_kv(kv, layer);
    if (rc) return rc;
    if ((rc = check_span(kv, start, t))) return rc;
    if (!q_dev || !k_dev || !v_dev || !att_dev) return fail(WICK_HIP_EINVAL, "null q, k, v or att");
    if ((rc = check_aligned(q_dev, "q_dev")) || (rc = check_aligned(k_dev, "k_dev")) ||
        (rc = check_aligned(v_dev, "v_dev")) || (rc = check_aligned(att_dev, "att_dev")))
        return rc;
    if (heads < 1 || heads % kv->kv_heads != 0)
        return fail(WICK_HIP_EINVAL, "heads (%d) must be a positive multiple of kv_heads (%d)", heads, kv->kv_heads);
    if (t == 1) return run_decode_fused(kv, layer, heads, q_dev, k_dev, v_dev, start, att_dev, len_dev);
    if (len_dev) return fail(WICK_HIP_EINVAL, "a device cache length needs t = 1");
    if ((rc = run_prep(kv, layer, heads, q_dev, k_dev, v_dev, t, start))) return rc;
    return run_attention(kv, layer, heads, q_dev, t, start, att_dev);
}

int attend_model_oproj(wick_hip_kv *kv, int layer, int heads, float *q_dev, const float *k_dev, const float *v_dev,
                       int start, const float *wo, int hidden, float *oparts, int *units_out, const int *len_dev) {
    int rc = check_kv(kv, layer);
    if (rc) return rc;
    if ((rc = check_span(kv, start, 1))) return rc;
    if (!q_dev || !k_dev || !v_dev || !wo || !oparts || !units_out) return fail(WICK_HIP_EINVAL, "null argument");
    if ((rc = check_aligned(q_dev, "q_dev")) || (rc = check_aligned(k_dev, "k_dev")) ||
        (rc = check_aligned(v_dev, "v_dev")))
        return rc;
    if (heads < 1 || heads % kv->kv_heads != 0)
        return fail(WICK_HIP_EINVAL, "heads (%d) must be a positive multiple of kv_heads (%d)", heads, kv->kv_heads);
    if (hidden < 1) return fail(WICK_HIP_EINVAL, "hidden must be >= 1");
    const int group = heads / kv->kv_heads;
    const int hslices = (group + wick::kTileRows - 1) / wick::kTileRows;
    int chunk, nchunks;
    plan_chunks(kv, kv->kv_heads * hslices, start + 1, &chunk, &nchunks);
    if (!wick::decode_oproj_supported(kv->head_dim, group, nchunks, chunk)) return 1;
    PrepConsts c;
    if ((rc = prep_consts(kv, layer, heads, &c))) return rc;
    wick::DecodeArgs a{};
    if ((rc = plan_decode(kv, layer, group, start + 1, q_dev, nullptr, &a))) return rc;
    a.scale = 1.0f / sqrtf((float)kv->head_dim);  // src/model.rs:527
    a.prep = 1;
    a.kraw = k_dev;
    a.vraw = v_dev;
    a.bq = c.bq;
    a.bk = c.bk;
    a.bv = c.bv;
    a.qn = c.qn;
    a.kn = c.kn;
    a.rope_cos = kv->rope_cos;
    a.rope_sin = kv->rope_sin;
    a.eps = c.eps;
    a.len_dev = len_dev;
    a.wo = wo;
    a.oparts = oparts;
    a.hidden = hidden;
    a.wo_ld = heads * kv->head_dim;
    hipError_t e = wick::launch_decode_oproj(kv->head_dim, a, kv->stream);
    if (e != hipSuccess) return hip_fail(e, "decode + output projection launch");
    *units_out = kv->kv_heads * hslices;
    return WICK_HIP_OK;
}

long long decode_plan_key(const wick_hip_kv *kv, int heads, int len) {
    const int group = heads / kv->kv_heads;
    const int hslices = (group + wick::kTileRows - 1) / wick::kTileRows;
    int chunk, nchunks;
    plan_chunks(kv, kv->kv_heads * hslices, len, &chunk, &nchunks);
    return ((long long)chunk << 32) | (unsigned)nchunks;
}

bool kv_info(const wick_hip_kv *kv, KvInfo *out) {
    if (!kv || !out) return false;
    *out = KvInfo{kv->layers, kv->capacity, kv->kv_heads, kv->head_dim, kv->stream};
    return true;
}

}  // namespace wick

extern "C" {

const char *wick_hip_last_error(void) { return g_last_error.c_str(); }

int wick_hip_kv_create(int layers, int capacity, int kv_heads, int head_dim, wick_hip_kv **out) {
    if (!out) return fail(WICK_HIP_EINVAL, "null output pointer");
    *out = nullptr;
    if (layers < 1 || capacity < 1 || kv_heads < 1)
        return fail(WICK_HIP_EINVAL, "layers, capacity and kv_heads must be >= 1");
    if (!supported_head_dim(head_dim)) return fail(WICK_HIP_EINVAL, "head_dim %d not supported (16, 32, 64, 128)", head_dim);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) return fail(WICK_HIP_EDEVICE, "no HIP device");
    wick_hip_kv *kv = new wick_hip_kv();
    kv->layers = layers;
    kv->capacity = capacity;
    kv->kv_heads = kv_heads;
    kv->head_dim = head_dim;
    int rc = WICK_HIP_OK;
    hipError_t e;
    do {
        if ((e = hipGetDevice(&kv->device)) != hipSuccess) { rc = hip_fail(e, "hipGetDevice"); break; }
        hipDeviceProp_t prop;
        if ((e = hipGetDeviceProperties(&prop, kv->device)) != hipSuccess) { rc = hip_fail(e, "hipGetDeviceProperties"); break; }
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
            rc = fail(WICK_HIP_EDEVICE, "device %d is %s; this library is built for gfx950", kv->device, prop.gcnArchName);
            break;
        }
        kv->num_cus = prop.multiProcessorCount;
        // the no-allocation entry point's workspace on this device (resolved once)
        kv->static_rc = wick::static_scratch_init(kv->device);
        kv->prep.resize(layers);
        kv->decode_blocks_per_cu = wick::decode_blocks_per_cu(head_dim);
        kv->prefill_blocks_per_cu = wick::prefill_blocks_per_cu(head_dim, 0);
        kv->prefill2_blocks_per_cu = wick::prefill_blocks_per_cu(head_dim, 1);
        if ((e = hipStreamCreateWithFlags(&kv->own_stream, hipStreamNonBlocking)) != hipSuccess) { rc = hip_fail(e, "hipStreamCreate"); break; }
        kv->stream = kv->own_stream;
        const size_t bytes = (size_t)layers * kv->layer_floats() * sizeof(float);
        if ((e = hipMalloc(&kv->k, bytes)) != hipSuccess) { rc = hip_fail(e, "hipMalloc(K cache)"); break; }
        if ((e = hipMalloc(&kv->v, bytes)) != hipSuccess) { rc = hip_fail(e, "hipMalloc(V cache)"); break; }
        // KvCache::new zero-fills (src/model.rs:265-266)
        if ((e = hipMemsetAsync(kv->k, 0, bytes, kv->stream)) != hipSuccess) { rc = hip_fail(e, "hipMemset(K)"); break; }
        if ((e = hipMemsetAsync(kv->v, 0, bytes, kv->stream)) != hipSuccess) { rc = hip_fail(e, "hipMemset(V)"); break; }
        if ((e = hipStreamSynchronize(kv->stream)) != hipSuccess) { rc = hip_fail(e, "hipStreamSynchronize"); break; }
    } while (0);
    if (rc != WICK_HIP_OK) {
        wick_hip_kv_destroy(kv);
        return rc;
    }
    *out = kv;
    return WICK_HIP_OK;
}

void wick_hip_kv_destroy(wick_hip_kv *kv) {
    if (!kv) return;
    if (kv->stream) (void)hipStreamSynchronize(kv->stream);
    float *bufs[] = {kv->k, kv->v, kv->q_dev, kv->att_dev, kv->kst_dev, kv->vst_dev, kv->part, kv->io_dev};
    for (float *b : bufs)
        if (b) (void)hipFree(b);
    if (kv->io_host) (void)hipHostFree(kv->io_host);
    if (kv->rope_cos) (void)hipFree(kv->rope_cos);
    if (kv->rope_sin) (void)hipFree(kv->rope_sin);
    for (auto &p : kv->prep)
        if (p.buf) (void)hipFree(p.buf);
    if (kv->own_stream) (void)hipStreamDestroy(kv->own_stream);
    delete kv;
}

int wick_hip_kv_set_stream(wick_hip_kv *kv, void *stream) {
    if (!kv) return fail(WICK_HIP_EINVAL, "null cache handle");
    kv->stream = stream ? (hipStream_t)stream : kv->own_stream;
    return WICK_HIP_OK;
}

int wick_hip_kv_synchronize(wick_hip_kv *kv) {
    if (!kv) return fail(WICK_HIP_EINVAL, "null cache handle");
    HIP_TRY(hipStreamSynchronize(kv->stream));
    return WICK_HIP_OK;
}

int wick_hip_kv_set_option(wick_hip_kv *kv, int option, int value) {
    if (!kv) return fail(WICK_HIP_EINVAL, "null cache handle");
    switch (option) {
    case WICK_HIP_OPT_DECODE_CHUNK:
        if (value != 0 && (value < 64 || value % 16 != 0))
            return fail(WICK_HIP_EINVAL, "decode chunk must be 0 or a multiple of 16 of at least 64 (got %d)", value);
        kv->decode_chunk = value;
        return WICK_HIP_OK;
    case WICK_HIP_OPT_DECODE_ORDER:
        if (value != 0 && value != 1)
            return fail(WICK_HIP_EINVAL, "decode order must be 0 (contiguous chunks) or 1 (automatic) (got %d)",
                        value);
        kv->decode_interleave = value;
        return WICK_HIP_OK;
    default:
        return fail(WICK_HIP_EINVAL, "unknown option %d", option);
    }
}

int wick_hip_kv_last_grid(const wick_hip_kv *kv) { return kv ? kv->last_grid : 0; }

long long wick_hip_kv_scratch_bytes(const wick_hip_kv *kv) {
    if (!kv) return 0;
    size_t floats = kv->q_cap + kv->att_cap + 2 * kv->kst_cap + kv->io_cap + kv->io_host_cap;
    if (kv->part) floats += wick::decode_workspace_floats(kv->ws_units, kv->head_dim);
    return (long long)(floats * sizeof(float));
}

int wick_hip_kv_append_device(wick_hip_kv *kv, int layer, int start, int t, const float *k_dev, const float *v_dev) {
    int rc = check_kv(kv, layer);
    if (rc) return rc;
    if ((rc = check_span(kv, start, t))) return rc;
    if (!k_dev || !v_dev) return fail(WICK_HIP_EINVAL, "null k or v");
    if ((rc = check_aligned(k_dev, "k_dev")) || (rc = check_aligned(v_dev, "v_dev"))) return rc;
    wick::AppendArgs a{k_dev, v_dev, kv->k_layer(layer), kv->v_layer(layer), kv->capacity, start, t, kv->kv_heads};
    hipError_t e = wick::launch_append(kv->head_dim, a, kv->stream);
    if (e != hipSuccess) return hip_fail(e, "append kernel launch");
    return WICK_HIP_OK;
}

int wick_hip_kv_append(wick_hip_kv *kv, int layer, int start, int t, const float *k, const float *v) {
    int rc = check_kv(kv, layer);
    if (rc) return rc;
    if ((rc = check_span(kv, start, t))) return rc;
    if (!k || !v) return fail(WICK_HIP_EINVAL, "null k or v");
    const size_t n = (size_t)t * kv->kv_heads * kv->head_dim;
    if (n > kv->kst_cap) {
        size_t ck = kv->kst_cap, cv = kv->kst_cap;
        kv->kst_cap = 0;
        if ((rc = grow(kv->stream, &kv->kst_dev, &ck, n, "hipMalloc(k staging)"))) return rc;
        if ((rc = grow(kv->stream, &kv->vst_dev, &cv, n, "hipMalloc(v staging)"))) return rc;
        kv->kst_cap = n;
    }
    HIP_TRY(hipMemcpyAsync(kv->kst_dev, k, n * sizeof(float), hipMemcpyHostToDevice, kv->stream));
    HIP_TRY(hipMemcpyAsync(kv->vst_dev, v, n * sizeof(float), hipMemcpyHostToDevice, kv->stream));
    if ((rc = wick_hip_kv_append_device(kv, layer, start, t, kv->kst_dev, kv->vst_dev))) return rc;
    HIP_TRY(hipStreamSynchronize(kv->stream));
    return WICK_HIP_OK;
}

int wick_hip_kv_read(const wick_hip_kv *kv, int layer, int pos0, int n, float *k, float *v) {
    int rc = check_kv(kv, layer);
    if (rc) return rc;
    if ((rc = check_span(kv, pos0, n))) return rc;
    const int D = kv->head_dim, kvd = kv->kv_heads * D;
    for (int h = 0; h < kv->kv_heads; h++) {
        const size_t off = ((size_t)h * kv->capacity + pos0) * D;
        if (k)
            HIP_TRY(hipMemcpy2DAsync(k + (size_t)h * D, kvd * sizeof(float), kv->k_layer(layer) + off, D * sizeof(float),
                                     D * sizeof(float), n, hipMemcpyDeviceToHost, kv->stream));
        if (v)
            HIP_TRY(hipMemcpy2DAsync(v + (size_t)h * D, kvd * sizeof(float), kv->v_layer(layer) + off, D * sizeof(float),
                                     D * sizeof(float), n, hipMemcpyDeviceToHost, kv->stream));
    }
    HIP_TRY(hipStreamSynchronize(kv->stream));
    return WICK_HIP_OK;
}

int wick_hip_attention_device(wick_hip_kv *kv, int layer, int heads, const float *q_dev, int t, int start,
                              float *att_dev) {
    int rc = check_kv(kv, layer);
    if (rc) return rc;
    if ((rc = check_span(kv, start, t))) return rc;
    if (!q_dev || !att_dev) return fail(WICK_HIP_EINVAL, "null q or att");
    if ((rc = check_aligned(q_dev, "q_dev")) || (rc = check_aligned(att_dev, "att_dev"))) return rc;
    return run_attention(kv, layer, heads, q_dev, t, start, att_dev);
}

int wick_hip_attention_device_noalloc(wick_hip_kv *kv, int layer, int heads, const float *q_dev, int t, int start,
                                      float *att_dev) {
    int rc = check_kv(kv, layer);
    if (rc) return rc;
    if ((rc = check_span(kv, start, t))) return rc;
    if (!q_dev || !att_dev) return fail(WICK_HIP_EINVAL, "null q or att");
    if ((rc = check_aligned(q_dev, "q_dev")) || (rc = check_aligned(att_dev, "att_dev"))) return rc;
    if (kv->static_rc != hipSuccess) return hip_fail(kv->static_rc, "hipGetSymbolAddress(static decode workspace)");
    float *part = wick::static_scratch(kv->device);
    if (!part) return fail(WICK_HIP_EHIP, "no static decode workspace on device %d", kv->device);
    return run_attention(kv, layer, heads, q_dev, t, start, att_dev, part);
}

int wick_hip_attention(wick_hip_kv *kv, int layer, int heads, const float *q, int t, int start, float *att) {
    int rc = check_kv(kv, layer);
    if (rc) return rc;
    if ((rc = check_span(kv, start, t))) return rc;
    if (!q || !att) return fail(WICK_HIP_EINVAL, "null q or att");
    if (heads < 1) return fail(WICK_HIP_EINVAL, "heads must be >= 1");
    // io blocks: q [n] | att [n]
    const size_t n = (size_t)t * heads * kv->head_dim;
    if ((rc = ensure_io(kv, 2 * n))) return rc;
    memcpy(kv->io_host, q, n * sizeof(float));
    HIP_TRY(hipMemcpyAsync(kv->io_dev, kv->io_host, n * sizeof(float), hipMemcpyHostToDevice, kv->stream));
    // one token: att straight into the pinned block; a chunk: copied back
    float *att_out = t == 1 ? kv->io_host + n : kv->io_dev + n;
    if ((rc = run_attention(kv, layer, heads, kv->io_dev, t, start, att_out))) return rc;
    if (t > 1)
        HIP_TRY(hipMemcpyAsync(kv->io_host + n, att_out, n * sizeof(float), hipMemcpyDeviceToHost, kv->stream));
    HIP_TRY(hipStreamSynchronize(kv->stream));
    memcpy(att, kv->io_host + n, n * sizeof(float));
    return WICK_HIP_OK;
}

}  // extern "C"

extern "C" {

int wick_hip_kv_set_rope(wick_hip_kv *kv, const float *inv_freq) {
    if (!kv) return fail(WICK_HIP_EINVAL, "null cache handle");
    if (!inv_freq) return fail(WICK_HIP_EINVAL, "null inv_freq");
    const int H = kv->head_dim / 2;
    const size_t n = (size_t)kv->capacity * H;
    std::vector<float> c(n), s(n);
    for (int pos = 0; pos < kv->capacity; pos++)
        for (int i = 0; i < H; i++) {
            // rope (src/model.rs:408): (pos as f32 * inv_freq[i]).sin_cos()
            const float ang = (float)pos * inv_freq[i];
            s[(size_t)pos * H + i] = sinf(ang);
            c[(size_t)pos * H + i] = cosf(ang);
        }
    if (!kv->rope_cos) HIP_TRY(hipMalloc(&kv->rope_cos, n * sizeof(float)));
    if (!kv->rope_sin) HIP_TRY(hipMalloc(&kv->rope_sin, n * sizeof(float)));
    HIP_TRY(hipMemcpyAsync(kv->rope_cos, c.data(), n * sizeof(float), hipMemcpyHostToDevice, kv->stream));
    HIP_TRY(hipMemcpyAsync(kv->rope_sin, s.data(), n * sizeof(float), hipMemcpyHostToDevice, kv->stream));
    HIP_TRY(hipStreamSynchronize(kv->stream));
    return WICK_HIP_OK;
}

int wick_hip_kv_set_prep(wick_hip_kv *kv, int layer, int heads, const float *bq, const float *bk, const float *bv,
                         const float *q_norm, const float *k_norm, float eps) {
    int rc = check_kv(kv, layer);
    if (rc) return rc;
    if (heads < 1 || heads % kv->kv_heads != 0)
        return fail(WICK_HIP_EINVAL, "heads (%d) must be a positive multiple of kv_heads (%d)", heads, kv->kv_heads);
    const int nb = (bq != nullptr) + (bk != nullptr) + (bv != nullptr);
    if (nb != 0 && nb != 3) return fail(WICK_HIP_EINVAL, "give all three of bq, bk, bv or none");
    if ((q_norm != nullptr) != (k_norm != nullptr)) return fail(WICK_HIP_EINVAL, "give both q_norm and k_norm or neither");
    if (!(eps >= 0.0f)) return fail(WICK_HIP_EINVAL, "eps must be >= 0");
    const int D = kv->head_dim, kvd = kv->kv_heads * D;
    wick_hip_kv::LayerPrep &p = kv->prep[layer];
    const size_t need = (size_t)heads * D + 2 * (size_t)kvd + 2 * (size_t)D;
    if (p.buf && p.heads != heads) {
        HIP_TRY(hipStreamSynchronize(kv->stream));
        (void)hipFree(p.buf);
        p.buf = nullptr;
    }
    p.set = false;
    if (!p.buf) HIP_TRY(hipMalloc(&p.buf, need * sizeof(float)));
    p.heads = heads;
    p.bias = nb == 3;
    p.norm = q_norm != nullptr;
    p.eps = eps;
    if (p.bias) {
        HIP_TRY(hipMemcpyAsync(p.buf, bq, (size_t)heads * D * sizeof(float), hipMemcpyHostToDevice, kv->stream));
        HIP_TRY(hipMemcpyAsync(p.buf + (size_t)heads * D, bk, kvd * sizeof(float), hipMemcpyHostToDevice, kv->stream));
        HIP_TRY(hipMemcpyAsync(p.buf + (size_t)heads * D + kvd, bv, kvd * sizeof(float), hipMemcpyHostToDevice,
                               kv->stream));
    }
    if (p.norm) {
        float *qn = p.buf + (size_t)heads * D + 2 * kvd;
        HIP_TRY(hipMemcpyAsync(qn, q_norm, D * sizeof(float), hipMemcpyHostToDevice, kv->stream));
        HIP_TRY(hipMemcpyAsync(qn + D, k_norm, D * sizeof(float), hipMemcpyHostToDevice, kv->stream));
    }
    HIP_TRY(hipStreamSynchronize(kv->stream));
    p.set = true;
    return WICK_HIP_OK;
}

int wick_hip_attend_device(wick_hip_kv *kv, int layer, int heads, float *q_dev, const float *k_dev,
                           const float *v_dev, int t, int start, float *att_dev) {
    // one token: preparation and append in the decode kernel's prologue (one
    // launch, q_dev untouched); a chunk: the preparation kernel (q in place),
    // then attention
    return wick::attend_model(kv, layer, heads, q_dev, k_dev, v_dev, t, start, att_dev, nullptr);
}

int wick_hip_attend(wick_hip_kv *kv, int layer, int heads, const float *q, const float *k, const float *v, int t,
                    int start, float *att) {
    int rc = check_kv(kv, layer);
    if (rc) return rc;
    if ((rc = check_span(kv, start, t))) return rc;
    if (!q || !k || !v || !att) return fail(WICK_HIP_EINVAL, "null q, k, v or att");
    if (heads < 1 || heads % kv->kv_heads != 0)
        return fail(WICK_HIP_EINVAL, "heads (%d) must be a positive multiple of kv_heads (%d)", heads, kv->kv_heads);
    // io blocks: q [nq] | k [nk] | v [nk] | att [nq] (each a multiple of head_dim
    // floats, so every part stays 16-byte aligned)
    const size_t nq = (size_t)t * heads * kv->head_dim, nk = (size_t)t * kv->kv_heads * kv->head_dim;
    if ((rc = ensure_io(kv, 2 * nq + 2 * nk))) return rc;
    float *h = kv->io_host, *d = kv->io_dev;
    memcpy(h, q, nq * sizeof(float));
    memcpy(h + nq, k, nk * sizeof(float));
    memcpy(h + nq + nk, v, nk * sizeof(float));
    HIP_TRY(hipMemcpyAsync(d, h, (nq + 2 * nk) * sizeof(float), hipMemcpyHostToDevice, kv->stream));
    // one token: the kernel writes att straight into the pinned block (a few KB
    // over the bus, one copy less); a chunk: a device block and one copy back
    float *att_out = t == 1 ? h + nq + 2 * nk : d + nq + 2 * nk;
    if ((rc = wick::attend_model(kv, layer, heads, d, d + nq, d + nq + nk, t, start, att_out))) return rc;
    if (t > 1)
        HIP_TRY(hipMemcpyAsync(h + nq + 2 * nk, att_out, nq * sizeof(float), hipMemcpyDeviceToHost, kv->stream));
    HIP_TRY(hipStreamSynchronize(kv->stream));
    memcpy(att, h + nq + 2 * nk, nq * sizeof(float));
    return WICK_HIP_OK;
}

}  // extern "C"
