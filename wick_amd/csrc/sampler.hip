// sampler.hip -- Sampler::sample (/root/reference/src/sampler.rs:73-127) as two
// kernels per draw, next to the logits the LM head wrote: a split kernel over
// up to kSampleParts slices of the vocabulary (one workgroup streams only a
// few tens of GB/s, so passes over the whole vocabulary are shared out), then
// one workgroup that finishes the draw.
//
// Phases (every branch that encloses a barrier depends only on kernel
// arguments or on LDS values read after a barrier, so all threads take it):
//   1. repetition penalty (:75-83) through a device bitset of seen ids, each
//      slice's ids by its workgroup;
//   2. temperature <= 0: argmax (:84-86, :129-137) per slice, then merged;
//   3. top-k (:87-94) on keys in f32::total_cmp order.  For k <= kFastK each
//      slice keeps its k best (key, id) pairs and the final kernel merges them
//      by rank.  Otherwise (or when a slice holds too many ties) an
//      11/11/10-bit radix select over the whole vocabulary finds the smallest
//      key bound whose candidate set holds the k best logits (the set ends at
//      a bin boundary, so it can hold more);
//   4. sort of that set by (key, id): bitonic in LDS up to kList entries, else
//      a stable LSD radix sort of the whole vocabulary in global memory; the
//      first k entries are the candidates, equal logits ordered by id;
//   5. softmax at the temperature (:95-98), min-p (:99-104), top-p (:105-115),
//      the draw (:116-125): f32 operations in wick's order (exp with the bits
//      of the C library's expf, exp_f32.h), the running sums and the draw
//      walked one element at a time by one wave.
// The sums stop early once the next term is at most a quarter ulp of the sum:
// the terms only shrink (the list is sorted), so no later term can change it.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>

#include "exp_f32.h"
#include "sampler_kernels.h"

namespace wick {
namespace {

constexpr int kT = 1024, kW = kT / 64;
constexpr int kCopies = 16;            // histogram copies, indexed by lane % 16
constexpr int kStride = kCopies + 1;   // words per bin: odd, so a bin per lane reads 32 banks
constexpr int kMaxBins = 2048;         // 11-bit digits
constexpr int kList = 4096;            // largest candidate set sorted in LDS
constexpr int kSlicePer = kSliceMax / kT;  // slice entries per thread in the split kernel
constexpr int kPartCand = 1024;        // candidates one slice may hold at its k-th key

typedef float f4 __attribute__((ext_vector_type(4)));

struct SampleLds {
    union {
        uint32_t hist[kMaxBins * kStride];  // 136 KiB: radix select and sort histograms
        struct {
            unsigned long long cand[kList];  // (key << 32) | id
            float prob[kList];
        } l;
        uint32_t wcnt[kW * 256];  // global sort: per-wave digit counts, then offsets
    };
    uint32_t tot[kMaxBins];  // per-bin totals of the copies
    uint32_t run[256];       // global sort: next free slot per digit
    uint32_t wsum[kW];
    uint32_t sel_bin, sel_before, sel_count, count, min_pos;
    int any_nan, bad, fast;
    int pcount[kSampleParts];
    unsigned long long top[kFastK];  // the merged list of the split path
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

// The logit a desc_key came from (the key is a bijection of the bits).
__device__ __forceinline__ float key_value(uint32_t key) {
    const uint32_t ord = ~key;
    return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
}

__device__ __forceinline__ void arg_better(float v, int i, float &bv, int &bi) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// f(i, x[i]) for every i < n, by every thread of the block; 32 floats per
// thread in flight per pass.
template <class F>
__device__ __forceinline__ void for_each_logit(const float *__restrict__ x, int n, F &&f) {
    constexpr int U = 8;
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

// The walks below run in one whole wave with wave-uniform arguments.  A chunk
// of 64 terms is loaded one per lane and the running f32 value takes term j
// (broadcast by readlane) in order, the same in every lane.  The running sum
// only grows and the draw's remainder only shrinks (the terms are >= 0), so
// without NaNs a crossing shows in the chunk's last value; only that chunk is
// walked again keeping the value after term j in lane j, and one ballot finds
// the first term where the condition holds (with NaNs every chunk is, and the
// last chunk is walked that way directly).  Early
// exits of the sums are tested once per chunk: terms past the exit point are
// at most a quarter ulp of the running sum and would leave it unchanged.
__device__ __forceinline__ float lane_value(float v, int j) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

// The first m (<= 64) terms of a chunk: all 64 unrolled, or in steps of 8 for
// a partial chunk (lanes past the valid terms hold zeros, which leave the
// value unchanged).
template <bool SUB>
__device__ __forceinline__ float chunk_end(float v, float acc, int m) {
    if (m == 64) {
#pragma unroll
        for (int j = 0; j < 64; j++) acc = SUB ? acc - lane_value(v, j) : acc + lane_value(v, j);
        return acc;
    }
    for (int j0 = 0; j0 < m; j0 += 8) {
#pragma unroll
        for (int j = j0; j < j0 + 8; j++) acc = SUB ? acc - lane_value(v, j) : acc + lane_value(v, j);
    }
    return acc;
}

template <bool SUB>
__device__ __forceinline__ float chunk_record(float v, float acc, int m) {
    const int lane = threadIdx.x & 63;
    float rec = 0.0f;
    if (m == 64) {
#pragma unroll
        for (int j = 0; j < 64; j++) {
            acc = SUB ? acc - lane_value(v, j) : acc + lane_value(v, j);
            rec = lane == j ? acc : rec;
        }
        return rec;
    }
    for (int j0 = 0; j0 < m; j0 += 8) {
#pragma unroll
        for (int j = j0; j < j0 + 8; j++) {
            acc = SUB ? acc - lane_value(v, j) : acc + lane_value(v, j);
            rec = lane == j ? acc : rec;
        }
    }
    return rec;
}

// The running f32 sum of p[0..n) in order, from acc.
__device__ __forceinline__ float sequential_sum(const float *p, int n, float acc, bool no_nan) {
    const int lane = threadIdx.x & 63;
    for (int base = 0; base < n; base += 64) {
        const float v = base + lane < n ? p[base + lane] : 0.0f;
        if (no_nan && negligible(acc, lane_value(v, 0))) break;
        acc = chunk_end<false>(v, acc, min(64, n - base));
    }
    return acc;
}

// top-p (src/sampler.rs:105-115): the running sum over p[0..*keep) from 0.0;
// *keep becomes i + 1 for the first i where it reaches top_p.  Returns the sum
// over the kept prefix (the total of :116).
__device__ __forceinline__ float top_p_cut(const float *p, int *keep, float top_p, bool no_nan) {
    const int lane = threadIdx.x & 63, n = *keep;
    float acc = 0.0f;
    for (int base = 0; base < n; base += 64) {
        const float v = base + lane < n ? p[base + lane] : 0.0f;
        if (no_nan && negligible(acc, lane_value(v, 0))) break;
        const int m = min(64, n - base);
        // the last chunk (or any, with NaNs) is walked keeping every value
        const bool last = base + 64 >= n;
        const float end = last || !no_nan ? 0.0f : chunk_end<false>(v, acc, m);
        if (last || !no_nan || end >= top_p) {
            const float run = chunk_record<false>(v, acc, m);
            const unsigned long long hit = __ballot(run >= top_p && base + lane < n);
            if (hit) {
                const int j = __builtin_ctzll(hit);
                *keep = base + j + 1;
                return lane_value(run, j);
            }
            acc = lane_value(run, m - 1);
        } else {
            acc = end;
        }
    }
    return acc;
}

// The draw (src/sampler.rs:118-125): r -= p[i] in order until r <= 0.
__device__ __forceinline__ int draw_index(const float *p, int keep, float r, bool no_nan) {
    const int lane = threadIdx.x & 63;
    for (int base = 0; base < keep; base += 64) {
        const float v = base + lane < keep ? p[base + lane] : 0.0f;
        const int m = min(64, keep - base);
        const bool last = base + 64 >= keep;
        const float end = last || !no_nan ? 0.0f : chunk_end<true>(v, r, m);
        if (last || !no_nan || end <= 0.0f) {
            const float run = chunk_record<true>(v, r, m);
            const unsigned long long hit = __ballot(run <= 0.0f && base + lane < keep);
            if (hit) return base + __builtin_ctzll(hit);
            r = lane_value(run, m - 1);
        } else {
            r = end;
        }
    }
    return keep - 1;
}

// Bitonic sort of one key per lane, ascending with the lane index.
__device__ __forceinline__ unsigned long long wave_sort(unsigned long long v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)v, stride, 64), hi = __shfl_xor((uint32_t)(v >> 32), stride, 64);
            const unsigned long long o = ((unsigned long long)hi << 32) | lo;
            const bool keep_min = ((lane & stride) == 0) == ((lane & size) == 0);
            v = keep_min ? (v < o ? v : o) : (v < o ? o : v);
        }
    }
    return v;
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

// Radix select over the keys each(f) visits (f(key) once per element, by every
// thread of the block), most significant digit first with the digit widths
// WIDTHS (summing to 32, each at most 11): the candidate set {key <= *bound}
// of the k smallest keys; returns its size (>= k; above `limit` only after the
// last digit).
template <int... WIDTHS, class Each>
__device__ __forceinline__ uint32_t select_bound(Each &&each, uint32_t k, uint32_t limit, SampleLds &s, uint32_t *bound) {
    const int lane = threadIdx.x & 63;
    constexpr int NP = sizeof...(WIDTHS);
    const int widths[NP] = {WIDTHS...};
    uint32_t prefix = 0, pmask = 0, need = k, below = 0;
    int shift = 32;
    for (int pass = 0; pass < NP; pass++) {
        shift -= widths[pass];
        const int nb = 1 << widths[pass];
        for (int i = threadIdx.x; i < nb * kStride; i += kT) s.hist[i] = 0u;
        __syncthreads();
        const uint32_t dmask = (uint32_t)nb - 1u;
        each([&](uint32_t key) {
            if ((key & pmask) == prefix) atomicAdd(&s.hist[((key >> shift) & dmask) * kStride + (lane & 15)], 1u);
        });
        __syncthreads();
        // fold the copies (bin b by thread b % kT), then thread t owns bins
        // [t * per, (t + 1) * per) for the scan
        for (int b = threadIdx.x; b < nb; b += kT) {
            uint32_t c = 0u;
#pragma unroll
            for (int r = 0; r < kCopies; r++) c += s.hist[b * kStride + r];
            s.tot[b] = c;
        }
        __syncthreads();
        const int per = nb >= kT ? nb / kT : 1;
        uint32_t c[2] = {0u, 0u}, mine = 0u;
        if ((int)threadIdx.x * per < nb) {
            for (int j = 0; j < per; j++) {
                c[j] = s.tot[threadIdx.x * per + j];
                mine += c[j];
            }
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
        if (le <= limit || pass == NP - 1) {
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
        for (int i = threadIdx.x; i < 256 * kStride; i += kT) s.hist[i] = 0u;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += kT) atomicAdd(&s.hist[((sk[i] >> shift) & 255u) * kStride + (lane & 15)], 1u);
        __syncthreads();
        uint32_t cnt = 0u;
        if (threadIdx.x < 256) {
#pragma unroll
            for (int r = 0; r < kCopies; r++) cnt += s.hist[threadIdx.x * kStride + r];
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

// Block-wide reduction of (bv, bi) with arg_better; the result in thread 0.
__device__ __forceinline__ void block_argmax(float &bv, int &bi, SampleLds &s) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
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
    if (threadIdx.x == 0)
        for (int j = 1; j < kW; j++) arg_better(s.fv[j], s.fi[j], bv, bi);
}

// The number of keys[0..n) below c (the keys are distinct); the reads are
// broadcasts, eight in flight.
__device__ __forceinline__ int rank_of(unsigned long long c, const unsigned long long *keys, int n) {
    int r = 0, j = 0;
    for (; j + 8 <= n; j += 8) {
        unsigned long long v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = keys[j + u];
#pragma unroll
        for (int u = 0; u < 8; u++) r += v[u] < c ? 1 : 0;
    }
    for (; j < n; j++) r += keys[j] < c ? 1 : 0;
    return r;
}

__host__ __device__ inline uint32_t top_k_of(const SampleArgs &a) {
    return (a.top_k == 0u || a.top_k > (uint32_t)a.vocab) ? (uint32_t)a.vocab : a.top_k;
}

// The first kernel of a draw: workgroup g owns the slice [g * slice, +slice)
// of the vocabulary (slices are whole bitset words).  It applies the
// repetition penalty to its ids (src/sampler.rs:75-83, each distinct id once),
// then writes its slice's argmax (greedy) or, for k <= kFastK, its k best
// (key, id) pairs in order: the k best of the vocabulary are among these.
__global__ __launch_bounds__(kT) void sample_split_kernel(SampleArgs a) {
    __shared__ SampleLds s;
    const int g = blockIdx.x, tid = threadIdx.x;
    float *__restrict__ x = a.logits;
    const int lo = g * a.slice, hi = max(lo, min(a.vocab, lo + a.slice));
    if (a.penalty != 1.0f) {
        for (int i = tid; i < a.n_history; i += kT) {
            const uint32_t t = a.history[i];
            if (t >= (uint32_t)lo && t < (uint32_t)hi) {
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
            if (t >= (uint32_t)lo && t < (uint32_t)hi) a.flags[t >> 5] = 0u;
        }
        __syncthreads();
    }
    if (a.temperature <= 0.0f) {
        float bv = -INFINITY;
        int bi = INT_MAX;
        for_each_logit(x + lo, hi - lo, [&](int i, float v) { arg_better(v, lo + i, bv, bi); });
        block_argmax(bv, bi, s);
        if (tid == 0) {
            a.part_val[g] = bv;
            a.part_id[g] = (uint32_t)bi;
        }
        return;
    }
    const uint32_t k = top_k_of(a);
    if (!a.split_top_k || k > (uint32_t)kFastK) return;
    uint32_t key[kSlicePer];
#pragma unroll
    for (int j = 0; j < kSlicePer; j++) {
        const int i = lo + j * kT + tid;
        key[j] = i < hi ? desc_key(x[i]) : 0u;
    }
    uint32_t bound = 0xffffffffu, nset = (uint32_t)(hi - lo);
    if (k < nset)
        nset = select_bound<8, 8, 8, 8>(
            [&](auto &&f) {
#pragma unroll
                for (int j = 0; j < kSlicePer; j++)
                    if (lo + j * kT + tid < hi) f(key[j]);
            },
            k, 64u, s, &bound);
    if (tid == 0) s.count = 0u;
    __syncthreads();
    if (nset > (uint32_t)kPartCand) {  // too many ties: the final kernel takes the whole vocabulary
        if (tid == 0) a.part_count[g] = -1;
        return;
    }
#pragma unroll
    for (int j = 0; j < kSlicePer; j++) {
        const int i = lo + j * kT + tid;
        if (i < hi && key[j] <= bound) {
            const uint32_t pos = atomicAdd(&s.count, 1u);
            if (pos < (uint32_t)kPartCand) s.l.cand[pos] = ((unsigned long long)key[j] << 32) | (uint32_t)i;
        }
    }
    __syncthreads();
    const int n = (int)min(s.count, (uint32_t)kPartCand);
    if (n <= 64) {  // one wave sorts them
        if (tid < 64) {
            const unsigned long long c = wave_sort(tid < n ? s.l.cand[tid] : ~0ull);
            if (tid < min(n, (int)k)) a.part_cand[g * kFastK + tid] = c;
        }
    } else if (tid < n) {
        const unsigned long long c = s.l.cand[tid];
        const int r = rank_of(c, s.l.cand, n);
        if (r < (int)k) a.part_cand[g * kFastK + r] = c;
    }
    if (tid == 0) a.part_count[g] = s.count == nset ? min(n, (int)k) : -1;
}

// The second kernel: one workgroup finishes the draw.
__global__ __launch_bounds__(kT) void sample_kernel(SampleArgs a) {
    __shared__ SampleLds s;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    float *__restrict__ x = a.logits;
    const int vocab = a.vocab;

    // 2. greedy (src/sampler.rs:84-86): the first index of the maximum over the
    // slices' results; a NaN at index 0 (or no value above NaN) keeps index 0,
    // as argmax (:129-137)
    if (a.temperature <= 0.0f) {
        if (tid == 0) {
            float bv = -INFINITY;
            int bi = INT_MAX;
            for (int g = 0; g < a.parts; g++) arg_better(a.part_val[g], (int)a.part_id[g], bv, bi);
            if (bi == INT_MAX || isnan(x[0])) bi = 0;
            *a.out = (uint32_t)bi;
            a.res_meta[0] = 0;
            a.res_meta[1] = 0;
            a.res_meta[2] = 0;
        }
        return;
    }

    // 3./4. the k best logits, sorted (src/sampler.rs:87-94)
    const uint32_t k = top_k_of(a);
    const bool try_fast = a.split_top_k && k <= (uint32_t)kFastK;
    if (tid == 0) {
        s.count = 0u;
        s.bad = 0;
        s.fast = try_fast ? 1 : 0;
    }
    __syncthreads();
    if (try_fast && tid < a.parts) {
        const int c = a.part_count[tid];
        s.pcount[tid] = c;
        if (c < 0) s.fast = 0;
    }
    __syncthreads();
    const bool fast = s.fast != 0;
    bool in_lds = true;
    if (fast) {
        // Each thread holds at most one of the slices' pairs; a radix select on
        // their keys bounds the k best, and one wave sorts the (usually few)
        // pairs up to that bound -- more are placed by rank.
        const int slots = a.parts * kFastK;
        unsigned long long mine = ~0ull;
        bool have = false;
        if (tid < slots) {
            const int g = tid / kFastK;
            have = tid - g * kFastK < min(s.pcount[g], kFastK);
            if (have) mine = a.part_cand[tid];
        }
        const uint32_t total = (uint32_t)__syncthreads_count(have);
        uint32_t bound = 0xffffffffu;
        if (k < total)
            select_bound<8, 8, 8, 8>([&](auto &&f) { if (have) f((uint32_t)(mine >> 32)); }, k, 64u, s, &bound);
        if (have && (uint32_t)(mine >> 32) <= bound) s.l.cand[atomicAdd(&s.count, 1u)] = mine;
        __syncthreads();
        const int n = (int)s.count;
        if (n < (int)k && tid == 0) s.bad = 4;
        if (n <= 64) {
            if (w == 0) s.top[lane] = wave_sort(lane < n ? s.l.cand[lane] : ~0ull);
        } else {
            for (int t = tid; t < n; t += kT) {
                const unsigned long long c = s.l.cand[t];
                const int r = rank_of(c, s.l.cand, n);
                if (r < (int)k) s.top[r] = c;
            }
        }
        __syncthreads();
        for (int i = tid; i < (int)k; i += kT) a.res_idx[i] = (uint32_t)s.top[i];
    } else {
        uint32_t bound = 0xffffffffu, nset = (uint32_t)vocab;
        if (k < (uint32_t)vocab)
            nset = select_bound<11, 11, 10>(
                [&](auto &&f) { for_each_logit(x, vocab, [&](int, float v) { f(desc_key(v)); }); }, k,
                (uint32_t)kList, s, &bound);
        in_lds = nset <= (uint32_t)kList;
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
            if (n2 <= 64) {
                if (w == 0) s.l.cand[lane] = wave_sort(lane < n ? s.l.cand[lane] : ~0ull);
                __syncthreads();
            } else {
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
    }
    __syncthreads();

    // 5. probabilities (src/sampler.rs:95-98); the logits are read back from
    // the sorted keys
    float *prob = in_lds ? s.l.prob : a.res_prob;
    const unsigned long long *sorted = fast ? s.top : s.l.cand;
    auto logit = [&](int i) { return key_value(in_lds ? (uint32_t)(sorted[i] >> 32) : a.key0[i]); };
    const float mx = logit(0);
    if (tid == 0) s.any_nan = 0;
    __syncthreads();
    for (int i = tid; i < (int)k; i += kT) {
        const float p = exp_f32((logit(i) - mx) / a.temperature);
        prob[i] = p;
        if (isnan(p)) s.any_nan = 1;
    }
    __syncthreads();
    const bool any_nan = s.any_nan != 0;
    if (w == 0) {
        const float sum = sequential_sum(prob, (int)k, -0.0f, !any_nan);
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
        // top-p (:105-115); the total (:116) is the same running sum over the kept prefix
        const float total = a.top_p < 1.0f ? top_p_cut(prob, &keep, a.top_p, !any_nan)
                                           : sequential_sum(prob, keep, 0.0f, !any_nan);
        uint64_t st[4] = {a.rng[0], a.rng[1], a.rng[2], a.rng[3]};
        const uint64_t u = next_u64(st);
        const float r = (float)(uint32_t)(u >> 40) / 16777216.0f * total;
        const int pick = draw_index(prob, keep, r, !any_nan);
        if (lane == 0) {
            a.rng[0] = st[0];
            a.rng[1] = st[1];
            a.rng[2] = st[2];
            a.rng[3] = st[3];
            const uint32_t id = in_lds ? (uint32_t)sorted[pick] : a.res_idx[pick];
            *a.out = min(id, (uint32_t)vocab - 1u);
            a.res_meta[0] = (int)k;
            a.res_meta[1] = keep;
            a.res_meta[2] = s.bad;
        }
    }
}

}  // namespace

hipError_t launch_sample(const SampleArgs &a, hipStream_t s) {
    // the split kernel is needed for the penalty, greedy, and the split top-k
    if (a.penalty != 1.0f || a.temperature <= 0.0f || (a.split_top_k && top_k_of(a) <= (uint32_t)kFastK)) {
        hipLaunchKernelGGL(sample_split_kernel, dim3(a.parts), dim3(kT), 0, s, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kT), 0, s, a);
    return hipGetLastError();
}

}  // namespace wick
