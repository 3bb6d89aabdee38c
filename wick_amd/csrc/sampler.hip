// sampler.hip -- Sampler::sample (/root/reference/src/sampler.rs:73-127) as one
// single-workgroup kernel per draw, next to the logits the LM head wrote.
//
// Phases (every branch that encloses a barrier depends only on kernel
// arguments or on LDS values read after a barrier, so all threads take it):
//   1. repetition penalty (:75-83) through a device bitset of seen ids;
//   2. temperature <= 0: argmax (:84-86, :129-137);
//   3. top-k (:87-94): keys in f32::total_cmp order; an 11/11/10-bit radix
//      select finds the smallest key bound whose candidate set holds the k best
//      logits (the set ends at a bin boundary, so it can hold more);
//   4. sort of the set by (key, id): bitonic in LDS up to kList entries, else
//      a stable LSD radix sort of the whole vocabulary in global memory; the
//      first k entries are the candidates, equal logits ordered by id;
//   5. softmax at the temperature (:95-98), min-p (:99-104), top-p (:105-115),
//      the draw (:116-125): f32 operations in wick's order, the running sums
//      walked one element at a time by one wave.
// The sums stop early once the next term is below a quarter ulp of the sum:
// the terms only shrink (the list is sorted), so no later term can change it.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>

#include "sampler_kernels.h"

namespace wick {
namespace {

constexpr int kT = 1024, kW = kT / 64;
constexpr int kCopies = 16;     // histogram copies, indexed by lane % 16
constexpr int kMaxBins = 2048;  // 11-bit digits
constexpr int kList = 4096;     // largest candidate set sorted in LDS

typedef float f4 __attribute__((ext_vector_type(4)));

struct SampleLds {
    union {
        uint32_t hist[kMaxBins * kCopies];  // 128 KiB: radix select and sort histograms
        struct {
            unsigned long long cand[kList];  // (key << 32) | id
            float prob[kList];
        } l;
        uint32_t wcnt[kW * 256];  // global sort: per-wave digit counts, then offsets
    };
    uint32_t run[256];  // global sort: next free slot per digit
    uint32_t wsum[kW];
    uint32_t sel_bin, sel_before, sel_count, count, min_pos;
    int any_nan, bad;
    float fv[kW];
    int fi[kW];
    float sum;
};

// f32::total_cmp order as an unsigned key, complemented so that ascending keys
// are descending logits.
__device__ __forceinline__ uint32_t desc_key(float x) {
    const uint32_t u = __float_as_uint(x);
    return ~((u & 0x80000000u) ? ~u : (u | 0x80000000u));
}

// acc + p == acc for every 0 <= p' <= p (round to nearest): p is at most a
// quarter of the spacing above acc (a margin of 2x over the exact half).
__device__ __forceinline__ bool negligible(float acc, float p) {
    const uint32_t e = (__float_as_uint(acc) >> 23) & 0xffu;
    if ((__float_as_uint(acc) >> 31) || e <= 25u || e == 255u) return false;
    return p <= __uint_as_float((e - 25u) << 23);
}

// f32::exp as exp() in double rounded once to f32.
__device__ __forceinline__ float exp_f32(float y) { return (float)exp((double)y); }

__device__ __forceinline__ void arg_better(float v, int i, float &bv, int &bi) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// f(i, x[i]) for every i < n, by every thread of the block; 16 floats per
// thread in flight per pass.
template <class F>
__device__ __forceinline__ void for_each_logit(const float *__restrict__ x, int n, F &&f) {
    constexpr int U = 4;
    const int n4 = n >> 2;
    const f4 *x4 = reinterpret_cast<const f4 *>(x);
    for (int base = threadIdx.x; base < n4; base += U * kT) {
        f4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = base + u * kT;
            v[u] = c < n4 ? x4[c] : f4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = base + u * kT;
            if (c < n4) {
                f(4 * c, v[u].x);
                f(4 * c + 1, v[u].y);
                f(4 * c + 2, v[u].z);
                f(4 * c + 3, v[u].w);
            }
        }
    }
    for (int i = 4 * n4 + (int)threadIdx.x; i < n; i += kT) f(i, x[i]);
}

// Exclusive prefix over the block of one value per thread; *total = the sum.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, SampleLds &s, uint32_t *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
    }
    if (lane == 63) s.wsum[w] = inc;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int j = 0; j < kW; j++) {
        const uint32_t t = s.wsum[j];
        before += j < w ? t : 0u;
        all += t;
    }
    __syncthreads();
    *total = all;
    return before + inc - v;
}

// p[0..n) in order, one element at a time in every lane of the calling wave
// (values broadcast with readlane, so the lanes stay uniform), until f returns
// false.
template <class F>
__device__ __forceinline__ void walk(const float *p, int n, F &&f) {
    const int lane = threadIdx.x & 63;
    for (int base = 0; base < n; base += 64) {
        const float v = base + lane < n ? p[base + lane] : 0.f;
        const int m = min(64, n - base);
        for (int j = 0; j < m; j++) {
            const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
            if (!f(base + j, pj)) return;
        }
    }
}

// Rng::next_u64 (src/sampler.rs:45-55), xoshiro256**.
__device__ __forceinline__ uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
__device__ __forceinline__ uint64_t next_u64(uint64_t (&s)[4]) {
    const uint64_t out = rotl64(s[1] * 5u, 7) * 9u;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return out;
}

// Radix select: the candidate set {i : key_i <= *bound} of the k best logits;
// returns its size (>= k; > kList only after the last digit).
__device__ uint32_t select_bound(const float *__restrict__ x, int vocab, uint32_t k, SampleLds &s, uint32_t *bound) {
    const int lane = threadIdx.x & 63;
    const int shifts[3] = {21, 10, 0}, widths[3] = {11, 11, 10};
    uint32_t prefix = 0, pmask = 0, need = k, below = 0;
    for (int pass = 0; pass < 3; pass++) {
        const int shift = shifts[pass], nb = 1 << widths[pass];
        for (int i = threadIdx.x; i < nb * kCopies; i += kT) s.hist[i] = 0u;
        __syncthreads();
        const uint32_t dmask = (uint32_t)nb - 1u;
        for_each_logit(x, vocab, [&](int, float v) {
            const uint32_t key = desc_key(v);
            if ((key & pmask) == prefix) atomicAdd(&s.hist[((key >> shift) & dmask) * kCopies + (lane & 15)], 1u);
        });
        __syncthreads();
        // thread t owns bins [t * per, (t + 1) * per)
        const int per = nb / kT;
        uint32_t c[2] = {0u, 0u}, mine = 0u;
        for (int j = 0; j < per; j++) {
            const uint32_t *h = &s.hist[(threadIdx.x * per + j) * kCopies];
#pragma unroll
            for (int r = 0; r < kCopies; r++) c[j] += h[r];
            mine += c[j];
        }
        uint32_t total;
        const uint32_t before = block_exclusive_scan(mine, s, &total);
        if (before < need && need <= before + mine) {
            uint32_t acc = before;
            for (int j = 0; j < per; j++) {
                if (need <= acc + c[j]) {
                    s.sel_bin = (uint32_t)(threadIdx.x * per + j);
                    s.sel_before = acc;
                    s.sel_count = c[j];
                    break;
                }
                acc += c[j];
            }
        }
        __syncthreads();
        const uint32_t bin = s.sel_bin, sb = s.sel_before, sc = s.sel_count;
        __syncthreads();
        const uint32_t le = below + sb + sc;
        if (le <= (uint32_t)kList || pass == 2) {
            *bound = prefix | (bin << shift) | ((1u << shift) - 1u);
            return le;
        }
        prefix |= bin << shift;
        pmask |= dmask << shift;
        need -= sb;
        below += sb;
    }
    return 0;  // not reached
}

// Stable LSD radix sort of (key0, idx0) over n entries, 8 bits per pass; the
// result ends in (key0, idx0).
__device__ void global_sort(uint32_t *key0, uint32_t *idx0, uint32_t *key1, uint32_t *idx1, int n, SampleLds &s) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const unsigned long long below_me = (1ull << lane) - 1ull;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 8 * pass;
        const uint32_t *sk = (pass & 1) ? key1 : key0, *si = (pass & 1) ? idx1 : idx0;
        uint32_t *dk = (pass & 1) ? key0 : key1, *di = (pass & 1) ? idx0 : idx1;
        for (int i = threadIdx.x; i < 256 * kCopies; i += kT) s.hist[i] = 0u;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += kT) atomicAdd(&s.hist[((sk[i] >> shift) & 255u) * kCopies + (lane & 15)], 1u);
        __syncthreads();
        uint32_t cnt = 0u;
        if (threadIdx.x < 256) {
#pragma unroll
            for (int r = 0; r < kCopies; r++) cnt += s.hist[threadIdx.x * kCopies + r];
        }
        uint32_t total;
        const uint32_t base = block_exclusive_scan(cnt, s, &total);
        if (threadIdx.x < 256) s.run[threadIdx.x] = base;
        for (int i = threadIdx.x; i < kW * 256; i += kT) s.wcnt[i] = 0u;
        __syncthreads();
        for (int tile = 0; tile < n; tile += kT) {
            const int i = tile + (int)threadIdx.x;
            const bool valid = i < n;
            const uint32_t key = valid ? sk[i] : 0u, id = valid ? si[i] : 0u;
            const uint32_t d = (key >> shift) & 255u;
            // lanes of this wave holding the same digit
            unsigned long long peers = __ballot(valid);
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const bool bit = (d >> b) & 1u;
                const unsigned long long m = __ballot(bit);
                peers &= bit ? m : ~m;
            }
            const uint32_t rank = (uint32_t)__popcll(peers & below_me);
            if (valid && rank == 0u) s.wcnt[w * 256 + d] = (uint32_t)__popcll(peers);
            __syncthreads();
            if (threadIdx.x < 256) {
                uint32_t off = s.run[threadIdx.x];
#pragma unroll
                for (int ww = 0; ww < kW; ww++) {
                    const uint32_t c = s.wcnt[ww * 256 + threadIdx.x];
                    s.wcnt[ww * 256 + threadIdx.x] = off;
                    off += c;
                }
                s.run[threadIdx.x] = off;
            }
            __syncthreads();
            if (valid) {
                const uint32_t pos = s.wcnt[w * 256 + d] + rank;
                if (pos < (uint32_t)n) {
                    dk[pos] = key;
                    di[pos] = id;
                } else {
                    s.bad = 2;
                }
            }
            __syncthreads();
            for (int j = threadIdx.x; j < kW * 256; j += kT) s.wcnt[j] = 0u;
            __syncthreads();
        }
    }
}

__global__ __launch_bounds__(kT) void sample_kernel(SampleArgs a) {
    __shared__ SampleLds s;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float *__restrict__ x = a.logits;
    const int vocab = a.vocab;

    // 1. repetition penalty: each distinct id below vocab once (src/sampler.rs:75-83)
    if (a.penalty != 1.0f) {
        for (int i = tid; i < a.n_history; i += kT) {
            const uint32_t t = a.history[i];
            if (t < (uint32_t)vocab) {
                const uint32_t bit = 1u << (t & 31u);
                if (!(atomicOr(&a.flags[t >> 5], bit) & bit)) {
                    const float l = x[t];
                    x[t] = l > 0.0f ? l / a.penalty : l * a.penalty;
                }
            }
        }
        __syncthreads();
        for (int i = tid; i < a.n_history; i += kT) {
            const uint32_t t = a.history[i];
            if (t < (uint32_t)vocab) a.flags[t >> 5] = 0u;
        }
        __syncthreads();
    }

    // 2. greedy (src/sampler.rs:84-86): the first index of the maximum; a NaN
    // at index 0 (or no value above NaN) keeps index 0, as argmax (:129-137)
    if (a.temperature <= 0.0f) {
        float bv = -INFINITY;
        int bi = INT_MAX;
        for_each_logit(x, vocab, [&](int i, float v) { arg_better(v, i, bv, bi); });
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            arg_better(ov, oi, bv, bi);
        }
        if (lane == 0) {
            s.fv[w] = bv;
            s.fi[w] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int j = 1; j < kW; j++) arg_better(s.fv[j], s.fi[j], bv, bi);
            if (bi == INT_MAX || isnan(x[0])) bi = 0;
            *a.out = (uint32_t)bi;
            a.res_meta[0] = 0;
            a.res_meta[1] = 0;
            a.res_meta[2] = 0;
        }
        return;
    }

    // 3./4. the k best logits, sorted (src/sampler.rs:87-94)
    const uint32_t k = (a.top_k == 0u || a.top_k > (uint32_t)vocab) ? (uint32_t)vocab : a.top_k;
    uint32_t bound = 0xffffffffu, nset = (uint32_t)vocab;
    if (k < (uint32_t)vocab) nset = select_bound(x, vocab, k, s, &bound);
    const bool in_lds = nset <= (uint32_t)kList;
    if (tid == 0) {
        s.count = 0u;
        s.bad = 0;
    }
    __syncthreads();
    if (in_lds) {
        for_each_logit(x, vocab, [&](int i, float v) {
            const uint32_t key = desc_key(v);
            if (key <= bound) {
                const uint32_t pos = atomicAdd(&s.count, 1u);
                if (pos < (uint32_t)kList) s.l.cand[pos] = ((unsigned long long)key << 32) | (uint32_t)i;
            }
        });
        __syncthreads();
        const uint32_t got = s.count;
        if (got != nset && tid == 0) s.bad = 1;
        const int n = (int)min(got, (uint32_t)kList);
        int n2 = 2;
        while (n2 < n) n2 <<= 1;
        for (int i = n + tid; i < n2; i += kT) s.l.cand[i] = ~0ull;
        __syncthreads();
        for (int size = 2; size <= n2; size <<= 1) {
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                for (int t = tid; t < (n2 >> 1); t += kT) {
                    const int lo = 2 * t - (t & (stride - 1)), hi = lo + stride;
                    const unsigned long long p = s.l.cand[lo], q = s.l.cand[hi];
                    if ((p > q) == ((lo & size) == 0)) {
                        s.l.cand[lo] = q;
                        s.l.cand[hi] = p;
                    }
                }
                __syncthreads();
            }
        }
        for (int i = tid; i < (int)k; i += kT) a.res_idx[i] = (uint32_t)s.l.cand[i];
    } else {
        for (int i = tid; i < vocab; i += kT) {
            a.key0[i] = desc_key(x[i]);
            a.res_idx[i] = (uint32_t)i;
        }
        __syncthreads();
        global_sort(a.key0, a.res_idx, a.key1, a.idx1, vocab, s);
    }
    __syncthreads();

    // 5. probabilities (src/sampler.rs:95-98).  An id outside the vocabulary
    // would be a bookkeeping error: it is read as id 0 and reported.
    float *prob = in_lds ? s.l.prob : a.res_prob;
    const float mx = x[min(a.res_idx[0], (uint32_t)vocab - 1u)];
    if (tid == 0) s.any_nan = 0;
    __syncthreads();
    for (int i = tid; i < (int)k; i += kT) {
        uint32_t id = a.res_idx[i];
        if (id >= (uint32_t)vocab) {
            id = 0u;
            s.bad = 3;
        }
        const float p = exp_f32((x[id] - mx) / a.temperature);
        prob[i] = p;
        if (isnan(p)) s.any_nan = 1;
    }
    __syncthreads();
    const bool any_nan = s.any_nan != 0;
    if (w == 0) {
        float sum = -0.0f;
        walk(prob, (int)k, [&](int, float p) {
            if (!any_nan && negligible(sum, p)) return false;
            sum += p;
            return true;
        });
        if (lane == 0) s.sum = sum;
    }
    if (tid == 0) s.min_pos = k;
    __syncthreads();
    const float sum = s.sum;
    for (int i = tid; i < (int)k; i += kT) {
        const float p = prob[i] / sum;
        prob[i] = p;
        if (in_lds) a.res_prob[i] = p;
    }
    __syncthreads();
    // min-p (src/sampler.rs:99-104): the first position below probs[0] * min_p
    if (a.min_p > 0.0f) {
        const float floor_p = prob[0] * a.min_p;
        for (int i = tid; i < (int)k; i += kT)
            if (prob[i] < floor_p) atomicMin(&s.min_pos, (uint32_t)i);
        __syncthreads();
    }
    if (w == 0) {
        int keep = max((int)s.min_pos, 1);
        // top-p (:105-115); total (:116) is the same running sum over the kept prefix
        float acc = 0.0f;
        const bool top_p = a.top_p < 1.0f;
        walk(prob, keep, [&](int i, float p) {
            if (!any_nan && negligible(acc, p)) return false;
            acc += p;
            if (top_p && acc >= a.top_p) {
                keep = i + 1;
                return false;
            }
            return true;
        });
        const float total = acc;
        uint64_t st[4] = {a.rng[0], a.rng[1], a.rng[2], a.rng[3]};
        const uint64_t u = next_u64(st);
        float r = (float)(uint32_t)(u >> 40) / 16777216.0f * total;
        int pick = keep - 1;
        walk(prob, keep, [&](int i, float p) {
            r -= p;
            if (r <= 0.0f) {
                pick = i;
                return false;
            }
            return true;
        });
        if (lane == 0) {
            a.rng[0] = st[0];
            a.rng[1] = st[1];
            a.rng[2] = st[2];
            a.rng[3] = st[3];
            *a.out = min(a.res_idx[pick], (uint32_t)vocab - 1u);
            a.res_meta[0] = (int)k;
            a.res_meta[1] = keep;
            a.res_meta[2] = s.bad;
        }
    }
}

}  // namespace

hipError_t launch_sample(const SampleArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kT), 0, s, a);
    return hipGetLastError();
}

}  // namespace wick
