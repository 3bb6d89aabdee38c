// attention.hip -- causal GQA attention over a device-resident KV cache, gfx950.
//
// Replaces Model::attention (/root/reference/src/model.rs:518-553): for every
// (token i, query head h) of a chunk of t tokens at positions start..start+t,
//   att[i,h,:] = sum_{p <= start+i} softmax_p(q[i,h] . K[p, h/group] * scale) V[p, h/group, :]
// with scale = 1/sqrt(head_dim) (src/model.rs:527) and kv head h/group
// (src/model.rs:526,532).
//
// All kernels share one wave-level layout: a wave owns 16 "columns" -- 16
// query heads of one kv head (decode) or 16 flattened (token, head) rows of
// one kv head (prefill; the two-block prefill kernels run two such sets of
// columns against every tile) -- and streams 16-key tiles of K and V through
// two f32 MFMAs (the lean core lean_load/lean_step at head_dim 64 and 128, the older
// attend_range core at head_dim 16 and 32):
//   S^T[16 keys x 16 cols] = K_tile[16 x D] . Q^T[D x 16]       (v_mfma_f32_16x16x4_f32)
//   O^T[D x 16 cols]      += V_tile^T[D x 16] . P^T[16 x 16]     (same instruction)
// so each lane owns one column: the online-softmax max/sum of a column needs
// only an in-lane reduction over 4 scores and two cross-lane steps, and P never
// leaves registers (the S^T accumulator layout is exactly the B-operand layout
// the PV product needs).  gfx950 has no xf32 MFMA, so both products run at the
// full-precision f32 matrix rate.
//
// MFMA 16x16x4 f32 lane layout (checked on the device): lane l supplies
// A[l%16][l/16] and B[l/16][l%16] and receives D[4*(l/16)+r][l%16], r = 0..3.
// The contraction index may be permuted freely, which is used to make every
// lane load contiguous float4s:
//   QK: MFMA m = 4j+e contracts head dim c(m, g) = 16j + 4g + e, g = l/16, so
//       lane (row i, g) loads K[p0+i][16j+4g .. +3] as one float4 per j.
//   PV: MFMA (m, db) contracts key 4g+m of the tile (exactly the key whose
//       score lane (col, g) holds in S^T register m) and produces head dims
//       dmap(row, db) = 64*(db/4) + W*row + db%4 (W = min(D/16, 4)), so lane
//       (i, g) loads V[p0+4g+m][64*seg + W*i .. +W) as one W-vector.
#include "attn_kernels.h"
#include "wave_ops.h"

#include <math.h>

#include <mutex>

namespace wick {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

template <int D>
struct Shape {
    static_assert(D == 16 || D == 32 || D == 64 || D == 128, "head_dim must be 16, 32, 64 or 128");
    static constexpr int KJ = D / 16;           // float4 K loads per lane per tile
    static constexpr int DB = D / 16;           // 16-row blocks of head dims in O^T
    static constexpr int W = DB < 4 ? DB : 4;   // floats per V load
    static constexpr int NSEG = DB / W;         // V loads per key row (2 for D=128)
    static constexpr int TG = 128 / D;          // tiles per softmax group (register budget)
};

__device__ __forceinline__ f4 mfma16x16x4(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Lazy reference max of the lean core (log2 units): weights 2^(s - m) stay
// below 2^8, so the running sums keep full f32 range and relative precision.
constexpr float kLazyMax = 8.0f;
// Starting reference max of the lazy core: finite, so 2^(s - m) needs no
// guard (a masked score, -inf, still gives 0) and the first finite score of a
// column replaces it.  A column that never sees a key keeps it, with l = 0.
constexpr float kLazyFloor = -1e30f;

// Max of two scores as gfx950's v_maximum3_f32: one instruction per 2-3 inputs,
// where fmaxf first quiets each input that might be a signalling NaN (v_max x, x
// per input).  It differs from fmaxf only for NaN inputs (propagated) and the
// sign of a zero maximum, which exp2(s - m) does not see.
__device__ __forceinline__ float smax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// max / sum over the four lanes that hold the same column (l, l^16, l^32, l^48).
// v_permlane16_swap / v_permlane32_swap (gfx950) hand each lane the pair
// {v[l], v[l^16]} / {v[l], v[l^32]} in a VALU op (checked on the device), so the
// column reduction needs no LDS round trip; a max or sum of the pair equals the
// xor-shuffle step bit for bit.
__device__ __forceinline__ float xor16_pair_max(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return smax(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xor32_pair_max(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return smax(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xor16_pair_sum(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xor32_pair_sum(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float col_max(float v) { return xor32_pair_max(xor16_pair_max(v)); }
__device__ __forceinline__ float col_sum(float v) { return xor32_pair_sum(xor16_pair_sum(v)); }

template <int W>
__device__ __forceinline__ void load_w(const float *p, float *out) {
    if constexpr (W == 4) {
        f4 x = *reinterpret_cast<const f4 *>(p);
        out[0] = x[0]; out[1] = x[1]; out[2] = x[2]; out[3] = x[3];
    } else if constexpr (W == 2) {
        f2 x = *reinterpret_cast<const f2 *>(p);
        out[0] = x[0]; out[1] = x[1];
    } else {
        out[0] = *p;
    }
}

// Head-dim index that register (r, db) of O^T lane group g holds.
template <int D>
__device__ __forceinline__ int out_dim(int g, int r, int db) {
    using S = Shape<D>;
    return 64 * (db / 4) + S::W * (4 * g + r) + (db % 4);
}

template <int D>
struct TileBuf {
    f4 k[Shape<D>::TG][Shape<D>::KJ];
    float v[Shape<D>::TG][4][Shape<D>::DB];
};

// Load the TG tiles starting at tile index `first` (keys kbeg + 16*tile ...).
// Rows at or past kend are clamped to kend-1 (always inside the cache) and
// masked out of the softmax later.
template <int D>
__device__ __forceinline__ void load_tiles(const float *__restrict__ Kh, const float *__restrict__ Vh, int kbeg,
                                           int kend, int first, int lane, TileBuf<D> &b) {
    using S = Shape<D>;
    const int i = lane & 15, g = lane >> 4;
#pragma unroll
    for (int u = 0; u < S::TG; u++) {
        const int p0 = kbeg + 16 * (first + u);
        const int pk = min(p0 + i, kend - 1);
        const float *kr = Kh + (size_t)pk * D + 4 * g;
#pragma unroll
        for (int j = 0; j < S::KJ; j++) b.k[u][j] = *reinterpret_cast<const f4 *>(kr + 16 * j);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int pv = min(p0 + 4 * g + m, kend - 1);
            const float *vr = Vh + (size_t)pv * D + S::W * i;
#pragma unroll
            for (int seg = 0; seg < S::NSEG; seg++) load_w<S::W>(vr + 64 * seg, &b.v[u][m][seg * S::W]);
        }
    }
}

// Running online-softmax state of one wave: column max, lane-partial sum and
// the unnormalised O^T accumulators.
template <int D>
struct WaveState {
    float m, l;
    f4 o[Shape<D>::DB];
};

template <int D, int CHAINS = 2>
__device__ __forceinline__ void compute_tiles(const TileBuf<D> &b, int kbeg, int first, int klimit, float scale,
                                              const f4 (&q)[Shape<D>::KJ], int lane, WaveState<D> &st) {
    using S = Shape<D>;
    const int g = lane >> 4;
    float sc[S::TG][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int u = 0; u < S::TG; u++) {
        // CHAINS independent accumulator chains (fewer if KJ is smaller),
        // interleaved so that consecutive MFMAs do not wait on each other's
        // results; more chains cost registers.
        constexpr int NCH = S::KJ < CHAINS ? S::KJ : CHAINS;
        f4 sch[NCH];
#pragma unroll
        for (int c = 0; c < NCH; c++) sch[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < S::KJ; jj += NCH) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
#pragma unroll
                for (int c = 0; c < NCH; c++) sch[c] = mfma16x16x4(b.k[u][jj + c][e], q[jj + c][e], sch[c]);
            }
        }
        f4 s = sch[0];
#pragma unroll
        for (int c = 1; c < NCH; c++) s += sch[c];
        const int key0 = kbeg + 16 * (first + u) + 4 * g;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            // wick rounds the dot product, then multiplies by scale (src/model.rs:539)
            const float x = (key0 + r < klimit) ? s[r] * scale : -INFINITY;
            sc[u][r] = x;
            mloc = fmaxf(mloc, x);
        }
    }
    mloc = col_max(mloc);
    const float mnew = fmaxf(st.m, mloc);
    const float mref = (mnew == -INFINITY) ? 0.f : mnew;
    const float alpha = exp2_fast((st.m - mref) * kLog2e);
    st.m = mnew;
    // alpha is exactly 1.0 where the max did not move; once the max settles
    // that holds for the whole wave and the rescale (a no-op) is skipped.
    if (!__all(alpha == 1.0f)) {
        st.l *= alpha;
#pragma unroll
        for (int db = 0; db < S::DB; db++) st.o[db] *= alpha;
    }
    float lsum = 0.f;
#pragma unroll
    for (int u = 0; u < S::TG; u++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            sc[u][r] = exp2_fast((sc[u][r] - mref) * kLog2e);
            lsum += sc[u][r];
        }
    }
    st.l += lsum;
#pragma unroll
    for (int u = 0; u < S::TG; u++) {
#pragma unroll
        for (int m = 0; m < 4; m++) {
#pragma unroll
            for (int db = 0; db < S::DB; db++) st.o[db] = mfma16x16x4(b.v[u][m][db], sc[u][m], st.o[db]);
        }
    }
}

// Stream keys [kbeg, kend) of one kv head through the wave, in groups of TG
// 16-key tiles: group n covers tiles tile0 + n*tstep .. +TG-1.  Keys at or past
// klimit (this lane's column limit, <= kend for decode) are masked.  Loads of
// the next group are issued before the current group is computed (PINGPONG),
// or each group is loaded then computed with half the registers, which buys
// more resident waves instead (the better trade for head_dim 128 decode).
template <int D, bool PINGPONG = true, int CHAINS = 2>
__device__ __forceinline__ void attend_range(const float *__restrict__ Kh, const float *__restrict__ Vh, int kbeg,
                                             int kend, int tile0, int tstep, int klimit, float scale,
                                             const f4 (&q)[Shape<D>::KJ], int lane, WaveState<D> &st) {
    const int ntiles = (kend - kbeg + 15) >> 4;
    klimit = min(klimit, kend);
    if constexpr (!PINGPONG) {
        TileBuf<D> b;
        for (int first = tile0; first < ntiles; first += tstep) {
            load_tiles<D>(Kh, Vh, kbeg, kend, first, lane, b);
            compute_tiles<D, CHAINS>(b, kbeg, first, klimit, scale, q, lane, st);
        }
        return;
    }
    TileBuf<D> ba, bb;
    int first = tile0;
    if (first >= ntiles) return;
    load_tiles<D>(Kh, Vh, kbeg, kend, first, lane, ba);
    for (;;) {
        int next = first + tstep;
        if (next < ntiles) load_tiles<D>(Kh, Vh, kbeg, kend, next, lane, bb);
        compute_tiles<D, CHAINS>(ba, kbeg, first, klimit, scale, q, lane, st);
        first = next;
        if (first >= ntiles) break;
        next = first + tstep;
        if (next < ntiles) load_tiles<D>(Kh, Vh, kbeg, kend, next, lane, ba);
        compute_tiles<D, CHAINS>(bb, kbeg, first, klimit, scale, q, lane, st);
        first = next;
        if (first >= ntiles) break;
    }
}

// Load this lane's share of 16 query rows as the B operand of QK:
// lane (col, g) holds q[col][16j + 4g .. +3] for every j.  Padding columns
// (valid == false) read the always-valid row `fallback` and are zeroed by a
// select: no branch, so the compiler does not wait for these loads before
// issuing the K/V loads that follow.
template <int D>
__device__ __forceinline__ void load_q(const float *qrow, const float *fallback, bool valid, int lane,
                                       f4 (&q)[Shape<D>::KJ]) {
    const int g = lane >> 4;
    const float *row = valid ? qrow : fallback;
    const float keep = valid ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < Shape<D>::KJ; j++) q[j] = *reinterpret_cast<const f4 *>(row + 16 * j + 4 * g) * keep;
}

// load_q without the padding mask: returns the factor (1 or 0) the caller
// folds into its own scaling of q, so nothing waits for the loads here.
template <int D>
__device__ __forceinline__ float load_q_raw(const float *qrow, const float *fallback, bool valid, int lane,
                                            f4 (&q)[Shape<D>::KJ]) {
    const int g = lane >> 4;
    const float *row = valid ? qrow : fallback;
#pragma unroll
    for (int j = 0; j < Shape<D>::KJ; j++) q[j] = *reinterpret_cast<const f4 *>(row + 16 * j + 4 * g);
    return valid ? 1.f : 0.f;
}

template <int D>
__device__ __forceinline__ void init_state(WaveState<D> &st) {
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int db = 0; db < Shape<D>::DB; db++) st.o[db] = f4{0.f, 0.f, 0.f, 0.f};
}

// ------------------------------------------------------------------ fused input preparation

// The per-token preparation of src/model.rs:464-480 for one row of D floats,
// bit-identical to wick's CPU arithmetic (and to prep_kernel): bias add;
// rmsnorm_inplace (src/kernels.rs:351-357) -- a sequential f32 sum of squares
// from -0.0, ss / D, 1 / sqrt(ss + eps) with IEEE divide and square root, then
// (x * scale) * w; rope (src/model.rs:404-414) -- two rounded products and a
// rounded sum per output, (sin, cos) from the host-filled table row.
// 16 lanes own a row: lane l of the group holds the rotation quad j = 4l
// (< D/2), i.e. elements j..j+3 and j+D/2..j+D/2+3, so all loads go out at
// once; the sum of squares is carried through the lanes in element order by a
// chain of shuffles (first half, then second half).  rowbase is the group's
// first lane; every lane of the group must call this with the same row.
// prep_load16 requests a row's inputs as one lane of its 16 holds them and
// prep_finish16 does the arithmetic, so that a caller can request several
// rows' inputs before it waits for any.
struct PrepIn {
    f4 u, w, bu, bw, nu, nw, c, sn;
};

template <int D>
__device__ __forceinline__ PrepIn prep_load16(const float *src, const float *bias, const float *norm,
                                              const float *cosr, const float *sinr, int l16) {
    constexpr int H = D / 2, NQ = H / 4;
    const int j = l16 < NQ ? 4 * l16 : 0;
    PrepIn in;
    in.u = *reinterpret_cast<const f4 *>(src + j);
    in.w = *reinterpret_cast<const f4 *>(src + j + H);
    in.bu = in.bw = in.nu = in.nw = in.c = in.sn = f4{0.f, 0.f, 0.f, 0.f};
    if (bias) {
        in.bu = *reinterpret_cast<const f4 *>(bias + j);
        in.bw = *reinterpret_cast<const f4 *>(bias + j + H);
    }
    if (norm) {
        in.nu = *reinterpret_cast<const f4 *>(norm + j);
        in.nw = *reinterpret_cast<const f4 *>(norm + j + H);
    }
    if (cosr) {
        in.c = *reinterpret_cast<const f4 *>(cosr + j);
        in.sn = *reinterpret_cast<const f4 *>(sinr + j);
    }
    return in;
}

// The arithmetic of prep_row16 on loaded inputs; bias / norm / rot say which
// steps apply (the pointers prep_load16 was given were non-null).
template <int D>
__device__ __forceinline__ void prep_finish16(PrepIn in, float *dst, bool bias, bool norm, float eps, bool rot,
                                              int l16, int rowbase) {
#pragma clang fp contract(off)
    constexpr int H = D / 2, NQ = H / 4;
    const bool mine = l16 < NQ;
    const int j = mine ? 4 * l16 : 0;
    f4 u = in.u, w = in.w;
    if (bias) {
        u = u + in.bu;
        w = w + in.bw;
    }
    if (norm) {
        float run = -0.0f;
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            float m = run;
            m = m + u.x * u.x;
            m = m + u.y * u.y;
            m = m + u.z * u.z;
            m = m + u.w * u.w;
            run = __shfl(m, rowbase + i, 64);
        }
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            float m = run;
            m = m + w.x * w.x;
            m = m + w.y * w.y;
            m = m + w.z * w.z;
            m = m + w.w * w.w;
            run = __shfl(m, rowbase + i, 64);
        }
        run = run / (float)D;
        const float scale = 1.0f / sqrtf(run + eps);
        u = u * scale * in.nu;
        w = w * scale * in.nw;
    }
    if (rot) {
        const f4 a = u * in.c - w * in.sn;
        const f4 b = w * in.c + u * in.sn;
        u = a;
        w = b;
    }
    if (mine) {
        *reinterpret_cast<f4 *>(dst + j) = u;
        *reinterpret_cast<f4 *>(dst + j + H) = w;
    }
}

template <int D>
__device__ __forceinline__ void prep_row16(const float *src, float *dst, const float *bias, const float *norm,
                                           float eps, const float *cosr, const float *sinr, int l16, int rowbase) {
    const PrepIn in = prep_load16<D>(src, bias, norm, cosr, sinr, l16);
    prep_finish16<D>(in, dst, bias != nullptr, norm != nullptr, eps, cosr != nullptr, l16, rowbase);
}

// ------------------------------------------------------------------ lean building blocks
//
// On gfx950 an f32 MFMA does not overlap vector ALU work: every VALU
// instruction a SIMD issues, from any wave, delays its MFMA pipe by about 5
// cycles, and every global dwordx4 load whose data returns to VGPRs by about
// 19 (measured: 1 VALU per 16x16x4 MFMA costs 16% of the matrix rate, 4 cost
// 40%).  The lean kernels therefore keep per-tile VALU work minimal:
//   - K/V tiles come through buffer loads: a wave-uniform resource over the kv
//     head's valid rows, a per-lane offset fixed for the whole loop and the
//     tile's position in a scalar offset, so no address arithmetic runs per
//     tile and rows past the end read as zero (no clamping);
//   - q is pre-multiplied by scale * log2(e), so scores come out of the MFMA
//     in log2 units and exp2 takes them directly (one extra rounding of q
//     against the reference's dot-then-scale; outputs move by ~1e-7);
//   - the QK products run as one accumulator chain (the MFMA pipe does not
//     stall on dependent chains), so no partial sums;
//   - masking only runs on groups that reach a limit.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float *base, unsigned bytes) {
    // Wave-uniform by construction; readfirstlane keeps it in SGPRs (otherwise
    // the compiler wraps every load in a per-lane waterfall loop).
    const unsigned long long p = (unsigned long long)base;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)p);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(p >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(((unsigned long long)hi << 32) | lo), (short)0,
                                             (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

__device__ __forceinline__ f4 bload4(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff) {
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    const u4 x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    return f4{__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]), __uint_as_float(x[3])};
}

// A group of TG 16-key tiles for the lean kernels, in the lane layout of
// load_tiles: lane (i = col, g) holds K[p0 + i][16j + 4g .. +3] and
// V[p0 + 4g + m][4i + 64 seg .. +3] (head_dim 64 and 128).
template <int D, int TG = Shape<D>::TG>
struct LeanGroup {
    f4 k[TG][Shape<D>::KJ];
    f4 v[TG][4][Shape<D>::NSEG];
};

// Buffer loads of the group starting at key p0 of the resource's kv head.
// vk, vv: the lane's fixed byte offsets (see lean_lane_offsets); rows past the
// resource's end read as zero.
template <int D>
__device__ __forceinline__ void lean_load(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, unsigned vk,
                                          unsigned vv, int p0, LeanGroup<D> &t) {
    using S = Shape<D>;
#pragma unroll
    for (int u = 0; u < S::TG; u++) {
        // p0 is wave-uniform; saying so keeps the loads out of waterfall loops
        const unsigned so = __builtin_amdgcn_readfirstlane((unsigned)(p0 + 16 * u) * D * 4u);
#pragma unroll
        for (int j = 0; j < S::KJ; j++) t.k[u][j] = bload4(rk, vk + 64 * j, so);
#pragma unroll
        for (int mm = 0; mm < 4; mm++)
#pragma unroll
            for (int seg = 0; seg < S::NSEG; seg++) t.v[u][mm][seg] = bload4(rv, vv + mm * D * 4 + seg * 256, so);
    }
    // The whole group's K and V loads go out before its first product: one
    // L2 round trip per step.  Left to itself the scheduler issues the K loads
    // one or two at a time between the products and the V loads after the
    // last of them (head_dim 128 T=512: 20.3 against 18.5 us).
    __builtin_amdgcn_sched_barrier(0);
}

// The same group through plain global loads from the kv head's rows, rows
// clamped to kend - 1 when `clamp` (the last group of a range).  Streaming
// from HBM these run faster than buffer loads (config 2 decode split kernel:
// 8.5 against 9.2 us).
template <int D, int TG = Shape<D>::TG>
__device__ __forceinline__ void lean_load_global_k(const float *__restrict__ Kh, int p0, int kend, bool clamp,
                                                   int lane, LeanGroup<D, TG> &t) {
    using S = Shape<D>;
    const int col = lane & 15, g = lane >> 4;
    const int last = clamp ? kend - 1 : 0x7fffffff;
#pragma unroll
    for (int u = 0; u < TG; u++) {
        const float *kr = Kh + (size_t)min(p0 + 16 * u + col, last) * D + 4 * g;
#pragma unroll
        for (int j = 0; j < S::KJ; j++) t.k[u][j] = *reinterpret_cast<const f4 *>(kr + 16 * j);
    }
}

// STREAM: V rows through nontemporal loads (the streaming cache policy).  On
// long HBM streams -- several groups per wave, or head_dim 128 -- they raise
// the decode's rate (config 5 per layer 98.5 -> 90.1 us; the Qwen2.5 shape at
// 512K positions 100.8 -> 90.6 us); on config 2's one group per wave they cost
// 0.15 us per call, and K through them costs more than it gains everywhere.
template <int D, int TG = Shape<D>::TG, bool STREAM = false>
__device__ __forceinline__ void lean_load_global_v(const float *__restrict__ Vh, int p0, int kend, bool clamp,
                                                   int lane, LeanGroup<D, TG> &t) {
    using S = Shape<D>;
    const int col = lane & 15, g = lane >> 4;
    const int last = clamp ? kend - 1 : 0x7fffffff;
#pragma unroll
    for (int u = 0; u < TG; u++) {
#pragma unroll
        for (int mm = 0; mm < 4; mm++) {
            const float *vr = Vh + (size_t)min(p0 + 16 * u + 4 * g + mm, last) * D + 4 * col;
#pragma unroll
            for (int seg = 0; seg < S::NSEG; seg++) {
                const f4 *src = reinterpret_cast<const f4 *>(vr + 64 * seg);
                if constexpr (STREAM)
                    t.v[u][mm][seg] = __builtin_nontemporal_load(src);
                else
                    t.v[u][mm][seg] = *src;
            }
        }
    }
}

template <int D, int TG = Shape<D>::TG, bool STREAM = false>
__device__ __forceinline__ void lean_load_global(const float *__restrict__ Kh, const float *__restrict__ Vh, int p0,
                                                 int kend, bool clamp, int lane, LeanGroup<D, TG> &t) {
    lean_load_global_k<D, TG>(Kh, p0, kend, clamp, lane, t);
    lean_load_global_v<D, TG, STREAM>(Vh, p0, kend, clamp, lane, t);
}

template <int D>
__device__ __forceinline__ void lean_lane_offsets(int lane, unsigned &vk, unsigned &vv) {
    const int col = lane & 15, g = lane >> 4;
    vk = (unsigned)((col * D + 4 * g) * 4);
    vv = (unsigned)((4 * g * D + 4 * col) * 4);
}

// One online-softmax step over a loaded group.  q is pre-scaled by
// scale * log2(e), so scores and the reference max m are in log2 units; the
// state (m, l, o) holds l = sum 2^(s - m), o = sum 2^(s - m) v.  Without
// LAZY m is the running max, -inf until a column has seen a key.  LAZY: m
// starts at kLazyFloor and moves (and l, o are rescaled) only
// when a column's score exceeds it by more than kLazyMax, so the weights stay
// below 2^kLazyMax and the rescale -- ~33 VALU instructions at head_dim 128,
// which cost MFMA issue slots -- runs on few steps after the first (prefill:
// T=512 18.5 -> 18.1 us).  Otherwise m is the running max (decode, where the
// extra test costs more than it saves).  When `masked`, keys at or past this
// lane's klimit get -inf.
template <int D, bool LAZY, int TG = Shape<D>::TG>
__device__ __forceinline__ void lean_step(const LeanGroup<D, TG> &t, const f4 (&q)[Shape<D>::KJ], int p0, bool masked,
                                          int klimit, int g, float &m, float &l, f4 (&o)[Shape<D>::DB]) {
    using S = Shape<D>;
    float sc[TG][4];
    // Prefill (LAZY): the wave's MFMA bursts run at raised issue priority, so
    // that another wave's softmax fills the gaps rather than competing with
    // them (config 3 T=2048 173.2 -> 167.6 us).
    if constexpr (LAZY) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int u = 0; u < TG; u++) {
        f4 sacc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < S::KJ; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) sacc = mfma16x16x4(t.k[u][j][e], q[j][e], sacc);
#pragma unroll
        for (int rr = 0; rr < 4; rr++) sc[u][rr] = sacc[rr];
    }
    if constexpr (LAZY) __builtin_amdgcn_s_setprio(0);
    if (masked) {
#pragma unroll
        for (int u = 0; u < TG; u++)
#pragma unroll
            for (int rr = 0; rr < 4; rr++) sc[u][rr] = (p0 + 16 * u + 4 * g + rr < klimit) ? sc[u][rr] : -INFINITY;
    }
    float lm = -INFINITY;
#pragma unroll
    for (int u = 0; u < TG; u++) lm = smax(lm, smax(smax(sc[u][0], sc[u][1]), smax(sc[u][2], sc[u][3])));
    const float cm = col_max(lm);
    float mx;
    if constexpr (LAZY) {
        const bool grow = cm > m + kLazyMax;  // never for cm = -inf
        if (__any(grow)) {
            const float alpha = grow ? exp2_fast(m - cm) : 1.0f;  // 0 from the floor
            l *= alpha;
#pragma unroll
            for (int db = 0; db < S::DB; db++) o[db] *= alpha;
            m = grow ? cm : m;
        }
        mx = m;
    } else {
        const float mnew = smax(m, cm);
        const float alpha = exp2_fast(m - ((mnew == -INFINITY) ? 0.f : mnew));
        if (!__all(alpha == 1.0f)) {
            l *= alpha;
#pragma unroll
            for (int db = 0; db < S::DB; db++) o[db] *= alpha;
        }
        m = mnew;
        mx = (m == -INFINITY) ? 0.f : m;  // every score is -inf then
    }
    float ls = 0.f;
#pragma unroll
    for (int u = 0; u < TG; u++)
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            sc[u][rr] = exp2_fast(sc[u][rr] - mx);
            ls += sc[u][rr];
        }
    l += ls;
    if constexpr (LAZY) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int u = 0; u < TG; u++)
#pragma unroll
        for (int mm = 0; mm < 4; mm++)
#pragma unroll
            for (int db = 0; db < S::DB; db++) o[db] = mfma16x16x4(t.v[u][mm][db / 4][db % 4], sc[u][mm], o[db]);
    if constexpr (LAZY) __builtin_amdgcn_s_setprio(0);
}

// The two-block prefill step at head_dim 128 (lean2), software-pipelined in
// the instruction stream: block A's QK products; then block B's QK products
// with A's masking and column max placed one VALU instruction between each
// two products; A's rescale (rare), weights and PV products; B's masking and
// column max between A's PV products; B's rescale, weights and PV products.
// The arithmetic is lean_step's (LAZY); only the order of independent
// instructions changes (config 3 T=2048: 172.2-173.4 -> 165.3-165.6 us).
template <int D, int TG>
__device__ __forceinline__ void lean_qk(const LeanGroup<D, TG> &t, const f4 (&q)[Shape<D>::KJ], float (&sc)[TG][4]) {
    using S = Shape<D>;
#pragma unroll
    for (int u = 0; u < TG; u++) {
        f4 sacc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < S::KJ; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) sacc = mfma16x16x4(t.k[u][j][e], q[j][e], sacc);
#pragma unroll
        for (int rr = 0; rr < 4; rr++) sc[u][rr] = sacc[rr];
    }
}

// masking (a select, not a branch, so the step stays one scheduling region)
// and the column max of the scores
template <int TG>
__device__ __forceinline__ void lean_mask_max(float (&sc)[TG][4], int p0, int klimit, int g, float &cm) {
#pragma unroll
    for (int u = 0; u < TG; u++)
#pragma unroll
        for (int rr = 0; rr < 4; rr++) sc[u][rr] = (p0 + 16 * u + 4 * g + rr < klimit) ? sc[u][rr] : -INFINITY;
    float lm = -INFINITY;
#pragma unroll
    for (int u = 0; u < TG; u++) lm = smax(lm, smax(smax(sc[u][0], sc[u][1]), smax(sc[u][2], sc[u][3])));
    cm = col_max(lm);
}

// the lazy reference max (rescale when a column passes m by kLazyMax), then
// the weights 2^(s - m) and their sum
template <int D, int TG>
__device__ __forceinline__ void lean_weights(const float (&sc)[TG][4], float cm, float &m, float &l,
                                             f4 (&o)[Shape<D>::DB], float (&e)[TG][4]) {
    using S = Shape<D>;
    const bool grow = cm > m + kLazyMax;  // never for cm = -inf
    if (__any(grow)) {
        const float alpha = grow ? exp2_fast(m - cm) : 1.0f;  // 0 from the floor
        l *= alpha;
#pragma unroll
        for (int db = 0; db < S::DB; db++) o[db] *= alpha;
        m = grow ? cm : m;
    }
    float ls = 0.f;
#pragma unroll
    for (int u = 0; u < TG; u++)
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            e[u][rr] = exp2_fast(sc[u][rr] - m);
            ls += e[u][rr];
        }
    l += ls;
}

template <int D, int TG>
__device__ __forceinline__ void lean_pv(const LeanGroup<D, TG> &t, const float (&e)[TG][4], f4 (&o)[Shape<D>::DB]) {
    using S = Shape<D>;
#pragma unroll
    for (int u = 0; u < TG; u++)
#pragma unroll
        for (int mm = 0; mm < 4; mm++)
#pragma unroll
            for (int db = 0; db < S::DB; db++) o[db] = mfma16x16x4(t.v[u][mm][db / 4][db % 4], e[u][mm], o[db]);
}

// scheduling groups for the region before the next sched_barrier: N times one
// MFMA then one VALU (transcendental included) instruction
template <int N>
__device__ __forceinline__ void interleave_mfma_valu() {
#pragma unroll
    for (int i = 0; i < N; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x402, 1, 0);
    }
}

template <int D, int TG>
__device__ __forceinline__ void lean_step2(const LeanGroup<D, TG> &t, const f4 (&q)[2][Shape<D>::KJ], int p0,
                                           const int (&klimit)[2], int g, float (&m)[2], float (&l)[2],
                                           f4 (&o)[2][Shape<D>::DB]) {
    float sa[TG][4], sb[TG][4], ea[TG][4], eb[TG][4], cma, cmb;
    __builtin_amdgcn_s_setprio(1);
    lean_qk<D, TG>(t, q[0], sa);
    __builtin_amdgcn_sched_barrier(0);
    lean_qk<D, TG>(t, q[1], sb);
    lean_mask_max<TG>(sa, p0, klimit[0], g, cma);
    interleave_mfma_valu<16>();
    __builtin_amdgcn_sched_barrier(0);
    lean_weights<D, TG>(sa, cma, m[0], l[0], o[0], ea);
    __builtin_amdgcn_sched_barrier(0);
    lean_pv<D, TG>(t, ea, o[0]);
    lean_mask_max<TG>(sb, p0, klimit[1], g, cmb);
    interleave_mfma_valu<16>();
    __builtin_amdgcn_sched_barrier(0);
    lean_weights<D, TG>(sb, cmb, m[1], l[1], o[1], eb);
    lean_pv<D, TG>(t, eb, o[1]);
    __builtin_amdgcn_s_setprio(0);
}

// ------------------------------------------------------------------ VALU decode core
//
// For a decode unit of NC <= 4 query heads (GQA groups of at most 4) the
// 16-column MFMA tiles leave at least 12 of their 16 columns idle, while
// gfx950's (unpacked) f32 VALU FMAs run at half the f32 MFMA rate, so this
// core runs the products on the VALU (head_dim 64).  A wave steps over groups of 32
// keys:
//   QK: lane (key kl = l/2, half hh = l%2) holds float4s 2j + hh (j < 8) of
//       its key's K row and of each head's q row: 8 dot4s per head, then the
//       pair's halves are added (DPP xor 1).  Scores are scaled into log2
//       units after the dot (q is not pre-scaled here).
//   softmax: per head, the wave's max (DPP / permlane), exp2, the sum over
//       the 32 keys; the weights go through the wave's own LDS slice.
//   PV: lane (dims 4*(l%16).., key group kq = l/16) accumulates keys kq + 4k
//       (k < 8) -- each V load instruction reads 4 whole rows, 1 KiB -- and the
//       4 key groups are summed across rows (permlane16/32 swaps) at the end.
// The wave's (m, l, O) per head leave through sm_m / sm_l / sm_o in the layout
// the workgroup merge reads.
// Wave-local preparation for the VALU core (RP): every wave prepares the
// unit's q rows itself (prep_load16 / prep_finish16, 16 lanes a row) into its
// own LDS slice, requesting their inputs right after its first group of
// tiles, so no workgroup barrier stands between the preparation's loads and
// the tiles' (one memory round trip before the first products instead of
// two: SmolLM2's fused decode 7.11 -> 6.55 us).  The wave whose keys hold
// position len - 1 -- not yet in the cache, which this kernel writes -- also
// prepares the new k and v rows, writes them to the cache and patches them
// into the tile registers of the lanes that hold that key.
struct WavePrep {
    const float *q;                  // the unit's first raw q row ([NC][64])
    const float *kraw, *vraw;        // the kv head's raw k / v rows
    const float *bq, *bk, *bv;       // biases (bq: the unit's first row) or null
    const float *qn, *kn;            // QK-norm weights or null
    const float *cosr, *sinr;        // rotation row of position len - 1
    float *kc, *vc;                  // cache rows at position len - 1
    float eps;
    int newkey;                      // len - 1 in the chunk that holds it, else -1
};

template <int NC, int NW, bool RP = false>
__device__ __forceinline__ void valu_core(const float *__restrict__ Kh, const float *__restrict__ Vh,
                                          f4 (&qr)[NC][8], float qf, int kbeg, int kend, int w, int lane,
                                          float (&swts)[NW][32][4], float (&sm_m)[NW][16], float (&sm_l)[NW][16],
                                          float (&sm_o)[NW][16][64], const WavePrep &rp = WavePrep{},
                                          float (*sqw)[64] = nullptr) {
    constexpr int D = 64, GK = 32;
    const int hh = lane & 1, kl = lane >> 1;
    const int dq = lane & 15, kq = lane >> 4;
    float m[NC], l[NC];
    f4 o[NC];
#pragma unroll
    for (int h = 0; h < NC; h++) {
        m[h] = -INFINITY;
        l[h] = 0.f;
        o[h] = f4{0.f, 0.f, 0.f, 0.f};
    }
    // RP: does this wave's range hold the new key?
    const bool holder = RP && rp.newkey >= kbeg && rp.newkey < kend && ((rp.newkey - kbeg) / GK) % NW == w;
    [[maybe_unused]] bool first = true;
    for (int p0 = kbeg + GK * w; p0 < kend; p0 += NW * GK) {
        const int last = kend - 1;
        // the group's K and V rows, clamped to the chunk (masked below)
        const int krow = min(p0 + kl, last);
        const float *kr = Kh + (size_t)krow * D + 4 * hh;
        f4 kv[8], vv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) kv[j] = *reinterpret_cast<const f4 *>(kr + 8 * j);
        int vrow[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            vrow[k] = min(p0 + kq + 4 * k, last);
            vv[k] = *reinterpret_cast<const f4 *>(Vh + (size_t)vrow[k] * D + 4 * dq);
        }
        if constexpr (RP) {
            if (first) {
                // the tiles are requested; now the preparation (its loads go
                // out behind them, its arithmetic waits for both)
                __builtin_amdgcn_sched_barrier(0);
                // q row r by lanes 16r..16r+15; in the holder also k by
                // lanes 0..15 and v by lanes 16..31 -- every input requested
                // before any arithmetic waits
                const int r = lane >> 4, l16 = lane & 15;
                const bool isk = r == 0;
                PrepIn qin, kvin;
                if (r < NC)
                    qin = prep_load16<D>(rp.q + r * D, rp.bq ? rp.bq + r * D : nullptr, rp.qn, rp.cosr, rp.sinr, l16);
                if (holder && r < 2)
                    kvin = prep_load16<D>(isk ? rp.kraw : rp.vraw, isk ? rp.bk : rp.bv, isk ? rp.kn : nullptr,
                                          isk ? rp.cosr : nullptr, isk ? rp.sinr : nullptr, l16);
                if (r < NC)
                    prep_finish16<D>(qin, sqw[r], rp.bq != nullptr, rp.qn != nullptr, rp.eps, true, l16, lane & 48);
                if (holder && r < 2)
                    prep_finish16<D>(kvin, sqw[NC + r], (isk ? rp.bk : rp.bv) != nullptr, isk && rp.kn != nullptr,
                                     rp.eps, isk, l16, lane & 48);
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int h = 0; h < NC; h++)
#pragma unroll
                    for (int j = 0; j < 8; j++) qr[h][j] = *reinterpret_cast<const f4 *>(&sqw[h][8 * j + 4 * hh]);
                if (holder && lane < 32) {
                    // the new k and v rows to the cache, a float4 a lane
                    const int rr = NC + (lane >> 4), c4 = 4 * (lane & 15);
                    *reinterpret_cast<f4 *>((lane < 16 ? rp.kc : rp.vc) + c4) =
                        *reinterpret_cast<const f4 *>(&sqw[rr][c4]);
                }
                first = false;
            }
            // the new key's rows in this group (wave-uniform test): from LDS
            if (holder && rp.newkey >= p0 && rp.newkey < p0 + GK) {
                if (krow == rp.newkey) {
#pragma unroll
                    for (int j = 0; j < 8; j++) kv[j] = *reinterpret_cast<const f4 *>(&sqw[NC][8 * j + 4 * hh]);
                }
#pragma unroll
                for (int k = 0; k < 8; k++)
                    if (vrow[k] == rp.newkey) vv[k] = *reinterpret_cast<const f4 *>(&sqw[NC + 1][4 * dq]);
            }
        }
        const bool valid = p0 + kl < kend;
        float s[NC];
#pragma unroll
        for (int h = 0; h < NC; h++) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                acc = fmaf(kv[j].x, qr[h][j].x, acc);
                acc = fmaf(kv[j].y, qr[h][j].y, acc);
                acc = fmaf(kv[j].z, qr[h][j].z, acc);
                acc = fmaf(kv[j].w, qr[h][j].w, acc);
            }
            acc += dpp_f<kDppQuadXor1>(acc);  // both lanes of the key: the whole dot
            s[h] = valid ? acc * qf : -INFINITY;
        }
#pragma unroll
        for (int h = 0; h < NC; h++) {
            const float mnew = fmaxf(m[h], wave_max(s[h]));  // key p0 is valid: finite
            const float alpha = exp2_fast(m[h] - mnew);      // 0 from the initial -inf
            const float e = exp2_fast(s[h] - mnew);
            l[h] = l[h] * alpha + wave_sum(hh == 0 ? e : 0.f);
            o[h] *= alpha;
            m[h] = mnew;
            if (hh == 0) swts[w][kl][h] = e;
        }
        // the wave reads back its own LDS writes (in order within a wave)
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const f4 wk = *reinterpret_cast<const f4 *>(&swts[w][kq + 4 * k][0]);
#pragma unroll
            for (int h = 0; h < NC; h++) o[h] += wk[h] * vv[k];
        }
    }
#pragma unroll
    for (int h = 0; h < NC; h++) {
        o[h].x = rows_sum(o[h].x);
        o[h].y = rows_sum(o[h].y);
        o[h].z = rows_sum(o[h].z);
        o[h].w = rows_sum(o[h].w);
    }
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < NC; h++) *reinterpret_cast<f4 *>(&sm_o[w][h][4 * dq]) = o[h];
    }
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < NC; h++) {
            sm_m[w][h] = m[h];
            sm_l[w][h] = l[h];
        }
    }
}

// ------------------------------------------------------------------ decode

// The key groups one wave of an interleaved split decode takes, in order: n
// groups of gk keys, the first at position p; next(p, j) gives the position of
// group j + 1 from group j's.  All fields are wave-uniform.  The kv head's
// groups are dealt round-robin to the waves of its nchunks workgroups (slot =
// chunk * waves + wave): F full rounds of `slots` groups, then one partial
// round.  Unit u starts its full rounds at round u mod F, so the kv heads (each
// on its own XCD when there are 8 units) do not read the same offsets of their
// caches at the same time (without the rotation the Llama-3-8B shape at 32768
// positions ran 48.6-48.8 us against 46.7-46.8).
struct KeyWalk {
    int p, n, step, wrap, full, tailp;

    __device__ static KeyWalk interleaved(int len, int nchunks, int chunk, int waves, int w, int gk, int unit) {
        const int slots = nchunks * waves, ngroups = (len + gk - 1) / gk;
        const int F = ngroups / slots, base = (chunk * waves + w) * gk, span = F * slots * gk;
        const int rot = F > 0 ? unit % F : 0;
        KeyWalk k;
        k.n = __builtin_amdgcn_readfirstlane(F + (span + base < len ? 1 : 0));
        k.p = __builtin_amdgcn_readfirstlane(rot * slots * gk + base);
        k.step = slots * gk;
        k.wrap = span;
        k.full = F;
        k.tailp = __builtin_amdgcn_readfirstlane(span + base);
        return k;
    }

    __device__ int next(int pos, int j) const {
        if (j + 1 == full) return tailp;
        pos += step;
        return pos >= wrap ? pos - wrap : pos;
    }
};

// Partial states of the split-K decode, per (unit, column): O [units][16][256][D],
// m and l [units][16][256] (unit = kv head x 16-head slice, column = query head
// of the slice, 256 = most chunks per call).  The chunk states of a column are
// contiguous, so the merge reads one contiguous block per column.
size_t decode_workspace_floats(int units, int head_dim) {
    return (size_t)units * 16 * kDecodeMaxChunks * (head_dim + 2);
}

template <int D>
struct DecodeSpace {
    float *o, *m, *l;
    __device__ DecodeSpace(float *part, int units) {
        o = part;
        m = o + (size_t)units * 16 * kDecodeMaxChunks * D;
        l = m + (size_t)units * 16 * kDecodeMaxChunks;
    }
    // index of (unit, column, chunk) in m / l; times D for o
    __device__ static size_t at(int unit, int col, int chunk) {
        return ((size_t)unit * 16 + col) * kDecodeMaxChunks + chunk;
    }
};

// One token (t = 1) over len cached positions, split-K: workgroup
// (unit, chunk) runs 4 waves over positions chunk*C .. +C of one kv head (or,
// with ILV, over its share of the kv head's key groups) for up to 16 of its
// query heads (unit = kv head x 16-head slice), so every K/V
// byte is read once for the whole GQA group.  With one chunk the output is
// written directly; otherwise the chunk's (max, sum, O) state per query head
// goes to the workspace and decode_merge_kernel, the next launch on the
// stream, combines them (the kernel boundary orders the two).
// PP: double-buffer the tile loads of consecutive groups.  When every wave
// takes at most one group (short chunks) the second buffer only costs
// registers -- 184 against 87 VGPRs at head_dim 64 -- so the launcher picks
// the single-buffered instance then.
// NW: waves per workgroup -- 4 for the split schedule; 8 (head_dim <= 64) for
// a single chunk per unit, so that short contexts give each wave at most one
// or two tile groups instead of two to four.
// TG: 16-key tiles per softmax group of the lean core (head_dim 64 and 128);
// one tile per group halves the products a wave runs after its last load.
// OPROJ: one chunk per unit and the output projection fused in (DecodeArgs'
// wo / oparts): workgroup (unit, row block) requests its rows of wo first,
// computes the unit's attention (every row block of a unit repeats it; each
// writes the same prepared k/v bits), keeps the normalised output in LDS and
// writes the unit's partial product for its rows.
// NC > 0 (head_dim 64, exactly NC <= 4 query heads per unit): the products
// run on the VALU core (valu_core) instead of the MFMA tiles.
// RP (PREP, NC > 0): the preparation is wave-local (WavePrep) instead of one
// shared LDS copy behind a workgroup barrier.
// ILV (NC == 0, 4 waves, several chunks): the interleaved key order
// (DecodeArgs::interleave, KeyWalk).
template <int D, bool PREP, bool PP = (D < 128), int NW = 4, int TG = Shape<D>::TG, bool OPROJ = false, int NC = 0,
          bool RP = false, bool ILV = false>
__global__ __launch_bounds__(64 * NW) void decode_kernel(const DecodeArgs a) {
    using S = Shape<D>;
    static_assert(NC == 0 || (D == 64 && NC <= 4), "the VALU core is for head_dim 64 and at most 4 heads");
    static_assert(!ILV || (NC == 0 && D >= 64 && !OPROJ), "the interleaved order is the lean MFMA core's");
    static_assert(!RP || (PREP && NC > 0), "wave-local preparation is the VALU core's");
    __shared__ float sm_m[NW][16], sm_l[NW][16];
    __shared__ __attribute__((aligned(16))) float sm_o[NW][16][D];
    __shared__ float sq[PREP && !RP ? 16 : 1][D];  // prepared q rows (PREP without RP)
    __shared__ __attribute__((aligned(16))) float sqw[RP ? NW : 1][RP ? NC + 2 : 1][RP ? D : 1];  // RP: per wave
    __shared__ float satt[OPROJ ? 16 * D : 1];  // normalised output of the unit's heads (OPROJ)
    __shared__ __attribute__((aligned(16))) float swts[NC > 0 ? NW : 1][32][4];  // VALU core weights

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int units = a.kv_heads * a.hslices;
    const int unit = blockIdx.x % units, chunk = OPROJ ? 0 : blockIdx.x / units;
    const int kvh = unit / a.hslices, slice = unit % a.hslices;
    const int col0 = slice * 16, ncols = min(16, a.group - col0);
    const int head0 = kvh * a.group + col0;
    const float *Kh = a.k + (size_t)kvh * a.capacity * D;
    const float *Vh = a.v + (size_t)kvh * a.capacity * D;
    // the cache length: the argument, or (graph-replayed decode loop) a device counter
    const int len = a.len_dev ? *a.len_dev : a.len;
    // ILV (DecodeArgs::interleave): the wave's key groups are dealt
    // round-robin over the kv head's chunks (KeyWalk) instead of one
    // contiguous range per chunk.  owner: the chunk that holds position len-1.
    const int kbeg = ILV ? 0 : chunk * a.chunk;  // (unused by ILV)
    const int kend = ILV ? len : min(kbeg + a.chunk, len);
    const int owner = ILV ? (len - 1) / (NW * 16 * TG) % a.nchunks : a.nchunks - 1;

    // OPROJ: this wave's kOprojRows rows of wo over the unit's ncols*D
    // columns, requested before anything waits on memory: lane l holds column
    // 64*j + l of row orow0 + r at wreg[r][j].
    float wreg[OPROJ ? kOprojRows : 1][OPROJ ? kOprojChunks : 1];
    int orow0 = 0, onrows = 0, cw = 0;
    if constexpr (OPROJ) {
        const int rblk = blockIdx.x / units;
        const int bend = min(a.hidden, (rblk + 1) * NW * kOprojRows);
        orow0 = rblk * NW * kOprojRows + w * kOprojRows;
        onrows = max(0, min(kOprojRows, bend - orow0));
        cw = ncols * D / 64;
        const float *wr = a.wo + (size_t)head0 * D + lane;
#pragma unroll
        for (int r = 0; r < kOprojRows; r++)
#pragma unroll
            for (int j = 0; j < kOprojChunks; j++)
                wreg[r][j] = (r < onrows && j < cw) ? wr[(size_t)(orow0 + r) * a.wo_ld + 64 * j] : 0.f;
    }

    const int col = lane & 15, g = lane >> 4;
    f4 q[S::KJ];
    float qkeep;  // 0 for the padding columns past the unit's ncols heads
    if constexpr (PREP && !RP) {
        // Rows: the unit's ncols q heads (to LDS), then -- in the workgroups
        // of the chunk that holds position len-1, the only ones that read it
        // -- the new k and v rows of the kv head (to the cache).  Workgroups of other
        // head slices of the same kv head write the same bits there.  The
        // barrier orders those stores before this workgroup's tile loads.
        const int pos = len - 1;
        const bool last = chunk == owner;
        const int nrows = ncols + (last ? 2 : 0);
        const float *cr = a.rope_cos + (size_t)pos * (D / 2), *sr = a.rope_sin + (size_t)pos * (D / 2);
        float *Kw = a.k + ((size_t)kvh * a.capacity + pos) * D;
        float *Vw = a.v + ((size_t)kvh * a.capacity + pos) * D;
        for (int r = w * 4 + (lane >> 4); r < nrows; r += 4 * NW) {
            if (r < ncols)
                prep_row16<D>(a.q + (size_t)(head0 + r) * D, sq[r], a.bq ? a.bq + (size_t)(head0 + r) * D : nullptr, a.qn,
                              a.eps, cr, sr, lane & 15, lane & 48);
            else if (r == ncols)
                prep_row16<D>(a.kraw + (size_t)kvh * D, Kw, a.bk ? a.bk + (size_t)kvh * D : nullptr, a.kn, a.eps, cr, sr,
                              lane & 15, lane & 48);
            else
                prep_row16<D>(a.vraw + (size_t)kvh * D, Vw, a.bv ? a.bv + (size_t)kvh * D : nullptr, nullptr, a.eps,
                              nullptr, nullptr, lane & 15, lane & 48);
        }
        __syncthreads();
        if constexpr (NC == 0) qkeep = load_q_raw<D>(sq[col], sq[0], col < ncols, lane, q);
    } else if constexpr (NC == 0) {
        qkeep = load_q_raw<D>(a.q + (size_t)(head0 + col) * D, a.q + (size_t)head0 * D, col < ncols, lane, q);
    }

    if constexpr (NC > 0) {
        // the unit's NC q rows, the lane's float4s 2j + hh of each
        f4 qr[NC > 0 ? NC : 1][8];
        const int hh = lane & 1;
        if constexpr (RP) {
            const int pos = len - 1;
            WavePrep rp;
            rp.q = a.q + (size_t)head0 * D;
            rp.kraw = a.kraw + (size_t)kvh * D;
            rp.vraw = a.vraw + (size_t)kvh * D;
            rp.bq = a.bq ? a.bq + (size_t)head0 * D : nullptr;
            rp.bk = a.bk ? a.bk + (size_t)kvh * D : nullptr;
            rp.bv = a.bv ? a.bv + (size_t)kvh * D : nullptr;
            rp.qn = a.qn;
            rp.kn = a.kn;
            rp.cosr = a.rope_cos + (size_t)pos * (D / 2);
            rp.sinr = a.rope_sin + (size_t)pos * (D / 2);
            rp.kc = a.k + ((size_t)kvh * a.capacity + pos) * D;
            rp.vc = a.v + ((size_t)kvh * a.capacity + pos) * D;
            rp.eps = a.eps;
            // only the owner chunk holds position len - 1 (the last one here)
            rp.newkey = chunk == owner ? pos : -1;
            valu_core<NC, NW, true>(Kh, Vh, qr, a.scale * kLog2e, kbeg, kend, w, lane, swts, sm_m, sm_l, sm_o, rp,
                                    sqw[w]);
        } else {
#pragma unroll
            for (int h = 0; h < NC; h++)
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    if constexpr (PREP)
                        qr[h][j] = *reinterpret_cast<const f4 *>(&sq[h][8 * j + 4 * hh]);
                    else
                        qr[h][j] = *reinterpret_cast<const f4 *>(a.q + (size_t)(head0 + h) * D + 8 * j + 4 * hh);
                }
            valu_core<NC, NW>(Kh, Vh, qr, a.scale * kLog2e, kbeg, kend, w, lane, swts, sm_m, sm_l, sm_o);
        }
    } else {

    WaveState<D> st;
    if constexpr (D >= 64) {
        // Lean core: q in log2 units, tiles through global loads (keys past
        // kend clamped and masked in the chunk's last group).  The wave's
        // first group of tiles is requested before q is scaled, so the stream
        // of K/V loads does not wait for q's round trip (config 2 split
        // kernel: the first K loads otherwise went out only after q arrived).
        const auto scale_q = [&] {
            const float f = qkeep * (a.scale * kLog2e);
#pragma unroll
            for (int j = 0; j < S::KJ; j++) q[j] *= f;
        };
        st.m = -INFINITY;
        st.l = 0.f;
#pragma unroll
        for (int db = 0; db < S::DB; db++) st.o[db] = f4{0.f, 0.f, 0.f, 0.f};
        constexpr int GK = 16 * TG;                 // keys per group
        constexpr bool kStreamV = D == 128 || PP;  // V through the streaming policy (lean_load_global_v)
        if constexpr (ILV && PP) {
            // the contiguous loops below over the walk's positions
            const KeyWalk walk = KeyWalk::interleaved(len, a.nchunks, chunk, NW, w, GK, unit);
            const int n = walk.n;
            LeanGroup<D, TG> ta, tb;
            int p0 = walk.p;
            if (n > 0) lean_load_global<D, TG, kStreamV>(Kh, Vh, p0, kend, p0 + GK > kend, lane, ta);
            __builtin_amdgcn_sched_barrier(0);
            scale_q();
            for (int j = 0; j < n; j += 2) {
                const int p1 = walk.next(p0, j);
                if (j + 1 < n) lean_load_global<D, TG, kStreamV>(Kh, Vh, p1, kend, p1 + GK > kend, lane, tb);
                lean_step<D, false, TG>(ta, q, p0, p0 + GK > kend, kend, g, st.m, st.l, st.o);
                if (j + 1 >= n) break;
                const int p2 = walk.next(p1, j + 1);
                if (j + 2 < n) lean_load_global<D, TG, kStreamV>(Kh, Vh, p2, kend, p2 + GK > kend, lane, ta);
                lean_step<D, false, TG>(tb, q, p1, p1 + GK > kend, kend, g, st.m, st.l, st.o);
                p0 = p2;
            }
        } else if constexpr (ILV) {
            const KeyWalk walk = KeyWalk::interleaved(len, a.nchunks, chunk, NW, w, GK, unit);
            const int n = walk.n;
            int p0 = walk.p, j = 0;
            if (n > 0) {
                LeanGroup<D, TG> t;
                const bool tail = p0 + GK > kend;
                lean_load_global_k<D, TG>(Kh, p0, kend, tail, lane, t);
                __builtin_amdgcn_sched_barrier(0);
                scale_q();
                if (a.stagger) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                lean_load_global_v<D, TG, kStreamV>(Vh, p0, kend, tail, lane, t);
                lean_step<D, false, TG>(t, q, p0, tail, kend, g, st.m, st.l, st.o);
                p0 = walk.next(p0, j++);
            }
            for (; j < n; p0 = walk.next(p0, j++)) {
                LeanGroup<D, TG> t;
                const bool tail = p0 + GK > kend;
                lean_load_global<D, TG, kStreamV>(Kh, Vh, p0, kend, tail, lane, t);
                lean_step<D, false, TG>(t, q, p0, tail, kend, g, st.m, st.l, st.o);
            }
        } else if constexpr (PP) {
            const int wbeg = __builtin_amdgcn_readfirstlane(kbeg + GK * w), step = NW * GK;
            // the next group's loads go out before this group's products
            LeanGroup<D, TG> ta, tb;
            int p0 = wbeg;
            if (p0 < kend) lean_load_global<D, TG, kStreamV>(Kh, Vh, p0, kend, p0 + GK > kend, lane, ta);
            __builtin_amdgcn_sched_barrier(0);
            scale_q();
            while (p0 < kend) {
                const int p1 = p0 + step;
                if (p1 < kend) lean_load_global<D, TG, kStreamV>(Kh, Vh, p1, kend, p1 + GK > kend, lane, tb);
                lean_step<D, false, TG>(ta, q, p0, p0 + GK > kend, kend, g, st.m, st.l, st.o);
                if (p1 >= kend) break;
                const int p2 = p1 + step;
                if (p2 < kend) lean_load_global<D, TG, kStreamV>(Kh, Vh, p2, kend, p2 + GK > kend, lane, ta);
                lean_step<D, false, TG>(tb, q, p1, p1 + GK > kend, kend, g, st.m, st.l, st.o);
                p0 = p2;
            }
        } else {
            const int wbeg = __builtin_amdgcn_readfirstlane(kbeg + GK * w), step = NW * GK;
            int p0 = wbeg;
            if (p0 < kend) {
                LeanGroup<D, TG> t;
                const bool tail = p0 + GK > kend;
                lean_load_global_k<D, TG>(Kh, p0, kend, tail, lane, t);
                // keeps the K loads ahead of the wait for q
                __builtin_amdgcn_sched_barrier(0);
                scale_q();
                // stagger: the V requests go out in K-arrival order, so the
                // last bytes of the transfer are V rows whose waves have
                // their QK products done (config 2: call 11.20 -> 11.11 us;
                // cache-resident grids, which are latency-bound, lose 0.1 us)
                if (a.stagger) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                lean_load_global_v<D, TG, kStreamV>(Vh, p0, kend, tail, lane, t);
                lean_step<D, false, TG>(t, q, p0, tail, kend, g, st.m, st.l, st.o);
                p0 += step;
            }
            for (; p0 < kend; p0 += step) {
                LeanGroup<D, TG> t;
                const bool tail = p0 + GK > kend;
                lean_load_global<D, TG, kStreamV>(Kh, Vh, p0, kend, tail, lane, t);
                lean_step<D, false, TG>(t, q, p0, tail, kend, g, st.m, st.l, st.o);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < S::KJ; j++) q[j] *= qkeep;
        init_state<D>(st);
        attend_range<D, PP>(Kh, Vh, kbeg, kend, w * S::TG, NW * S::TG, len, a.scale, q, lane, st);
        st.m *= kLog2e;  // the merges take maxima in log2 units
    }
    st.l = col_sum(st.l);

    if (g == 0) {
        sm_m[w][col] = st.m;
        sm_l[w][col] = st.l;
    }
#pragma unroll
    for (int db = 0; db < S::DB; db++)
#pragma unroll
        for (int r = 0; r < 4; r++) sm_o[w][col][out_dim<D>(g, r, db)] = st.o[db][r];
    }  // MFMA core
    __syncthreads();

    // Merge the NW waves of this workgroup (maxima in log2 units).  Wave 0
    // always holds the chunk's first key, so the merged max is finite.
    const DecodeSpace<D> ws(a.part, units);
    if (a.nchunks == 1) {
        // one element per thread: the divide is the long pole of the tail
        for (int idx = threadIdx.x; idx < ncols * D; idx += blockDim.x) {
            const int c = idx / D, d = idx % D;
            float M = -INFINITY;
#pragma unroll
            for (int ww = 0; ww < NW; ww++) M = fmaxf(M, sm_m[ww][c]);
            float o = 0.f, L = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ww++) {
                const float e = exp2_fast(sm_m[ww][c] - M);
                o += sm_o[ww][c][d] * e;
                L += sm_l[ww][c] * e;
            }
            if constexpr (OPROJ)
                satt[idx] = o / L;
            else
                a.att[(size_t)(head0 + c) * D + d] = o / L;
        }
        if constexpr (OPROJ) {
            // partial output projection of this wave's rows: the lane's
            // columns in order, then a fixed butterfly
            __syncthreads();
            float sum[kOprojRows];
#pragma unroll
            for (int r = 0; r < kOprojRows; r++) {
                sum[r] = 0.f;
#pragma unroll
                for (int j = 0; j < kOprojChunks; j++)
                    if (j < cw) sum[r] = fmaf(wreg[r][j], satt[64 * j + lane], sum[r]);
            }
#pragma unroll
            for (int r = 0; r < kOprojRows; r++) {
                sum[r] = wave_sum(sum[r]);
                if (lane == 0 && r < onrows) a.oparts[(size_t)unit * a.hidden + orow0 + r] = sum[r];
            }
        }
    } else {
        // 4 consecutive dims of one column per thread, which works out that
        // column's weights itself
        for (int idx = threadIdx.x; idx < ncols * (D / 4); idx += blockDim.x) {
            const int c = idx / (D / 4), d = 4 * (idx % (D / 4));
            float M = -INFINITY;
#pragma unroll
            for (int ww = 0; ww < NW; ww++) M = fmaxf(M, sm_m[ww][c]);
            f4 o = {0.f, 0.f, 0.f, 0.f};
            float L = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ww++) {
                const float e = exp2_fast(sm_m[ww][c] - M);
                o += *reinterpret_cast<const f4 *>(&sm_o[ww][c][d]) * e;
                L += sm_l[ww][c] * e;
            }
            const size_t s = DecodeSpace<D>::at(unit, c, chunk);
            *reinterpret_cast<f4 *>(ws.o + s * D + d) = o;
            if (d == 0) {
                ws.m[s] = M;
                ws.l[s] = L;
            }
        }
    }
}

// Log-sum-exp combine of two (max, O, sum) states handed over as swapped
// pairs; symmetric in the pair, and a pair of empty states (-inf maxima)
// stays empty.
template <typename P>
__device__ __forceinline__ void merge_pair(P pm, P po, P pl, float &M, float &acc, float &L) {
    const float m0 = __uint_as_float(pm[0]), m1 = __uint_as_float(pm[1]);
    const float M2 = fmaxf(m0, m1);
    const float Mr = (M2 == -INFINITY) ? 0.f : M2;
    const float e0 = exp2_fast(m0 - Mr), e1 = exp2_fast(m1 - Mr);
    acc = __uint_as_float(po[0]) * e0 + __uint_as_float(po[1]) * e1;
    L = __uint_as_float(pl[0]) * e0 + __uint_as_float(pl[1]) * e1;
    M = M2;
}

// Merge pass (maxima in log2 units): workgroup (query head, 16-dim slice)
// combines the nchunks (<= 256) partial states of one query head for 16 of its
// head dims; the grid holds exactly heads x D/16 workgroups.  Thread (grp, dd)
// of 16 groups owns children grp, grp + 16, ...: it loads their O, m and l
// together (one memory round trip) and merges them by log-sum-exp against its
// own running max; the 4 groups of each wave then combine pairwise in
// registers and the 4 wave states in one LDS step.  Child order within a
// thread and the combine tree are fixed: deterministic for a given nchunks.
// NB: child slots per thread, the fewest powers of two that cover nchunks
// (16 x NB >= nchunks), so a call with few chunks loads no dead slots.
template <int D, int NB>
__global__ __launch_bounds__(256) void decode_merge_kernel(const DecodeArgs a) {
    constexpr int DW = 16;                        // head dims per workgroup
    constexpr int NS = D / DW;                    // slices per column
    constexpr int G = 256 / DW;                   // thread groups over children
    static_assert(G * NB <= kDecodeMaxChunks, "child slots past the workspace");
    __shared__ float sm[4][DW], so[4][DW], sl[4][DW];
    const int units = a.kv_heads * a.hslices;
    const int ds = blockIdx.x % NS, head = blockIdx.x / NS;
    const int kvh = head / a.group, hh = head % a.group;
    const int col = hh % 16, unit = kvh * a.hslices + hh / 16;
    const DecodeSpace<D> ws(a.part, units);
    const size_t base = DecodeSpace<D>::at(unit, col, 0);
    const float *o = ws.o + base * D + ds * DW, *m = ws.m + base, *l = ws.l + base;
    const int tid = threadIdx.x;
    const int grp = tid / DW, dd = tid % DW;
    const int n = a.nchunks;

    // Every child slot ch < G * NB <= kDecodeMaxChunks lies inside the
    // workspace, so the loads are unconditional (no exec-mask branch per load
    // delays their issue) and the children past nchunks -- stale or never
    // written -- are replaced by a select afterwards.
    float vo[NB], vm[NB], vl[NB];
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const int ch = grp + u * G;
        vo[u] = o[(size_t)ch * D + dd];
        vm[u] = m[ch];
        vl[u] = l[ch];
    }
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const bool live = grp + u * G < n;
        vo[u] = live ? vo[u] : 0.f;
        vm[u] = live ? vm[u] : -INFINITY;
        vl[u] = live ? vl[u] : 0.f;
    }
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < NB; u++) M = fmaxf(M, vm[u]);
    const float Mref = (M == -INFINITY) ? 0.f : M;  // a group with no children
    float acc = 0.f, L = 0.f;
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const float e = exp2_fast(vm[u] - Mref);
        acc += vo[u] * e;
        L += vl[u] * e;
    }
    // The 4 groups of a wave (lanes l, l^16, l^32, l^48 hold the same head
    // dim) combine in registers, pairwise through permlane swaps; both lanes
    // of a pair compute the same bits (the combine is symmetric).  Then the 4
    // wave states meet in LDS.
    merge_pair(__builtin_amdgcn_permlane16_swap(__float_as_uint(M), __float_as_uint(M), false, false),
               __builtin_amdgcn_permlane16_swap(__float_as_uint(acc), __float_as_uint(acc), false, false),
               __builtin_amdgcn_permlane16_swap(__float_as_uint(L), __float_as_uint(L), false, false), M, acc, L);
    merge_pair(__builtin_amdgcn_permlane32_swap(__float_as_uint(M), __float_as_uint(M), false, false),
               __builtin_amdgcn_permlane32_swap(__float_as_uint(acc), __float_as_uint(acc), false, false),
               __builtin_amdgcn_permlane32_swap(__float_as_uint(L), __float_as_uint(L), false, false), M, acc, L);
    const int w = tid >> 6;
    if ((tid & 63) < DW) {
        sm[w][dd] = M;
        so[w][dd] = acc;
        sl[w][dd] = L;
    }
    __syncthreads();
    if (tid < DW) {
        float Mt = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) Mt = fmaxf(Mt, sm[ww][tid]);
        float ot = 0.f, Lt = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
            const float e = exp2_fast(sm[ww][tid] - Mt);
            ot += so[ww][tid] * e;
            Lt += sl[ww][tid] * e;
        }
        a.att[(size_t)head * D + ds * DW + tid] = ot / Lt;
    }
}

// ------------------------------------------------------------------ prefill

// Rows of one kv head are the flattened (token i, head hh) pairs r = i*group + hh,
// so the GQA heads of a token share every K/V tile.
// Workgroup = one 16-row block b of one kv head; its causal key range
// 0 .. start + last token of the block is split into 4 contiguous tile ranges,
// one per wave, whose states are merged through LDS.  Blocks are dispatched
// heaviest first (largest b), so the many workgroups of a causal launch
// balance across CUs without pairing, and every SIMD holds several waves
// (single-buffered tiles at head_dim 128 leave room for three) to overlap one
// wave's softmax with another's MFMAs.  The wave holding key 0 -- valid for
// every row -- keeps each merged max finite.
template <int D>
__device__ __forceinline__ void prefill_split_body(const PrefillArgs &a) {
    using S = Shape<D>;
    __shared__ float sm_m[4][16], sm_l[4][16];
    __shared__ float sm_o[4][16][D];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int kvh = blockIdx.x % a.kv_heads;
    // Heaviest causal blocks first.  When the whole grid is resident at once
    // (zigzag), the second half runs lightest first instead, so that the
    // workgroups dispatched side by side, idx and idx + nblocks/2, pair a heavy
    // block with a light one and every CU gets about the same number of tiles.
    const int idx = (int)(blockIdx.x / a.kv_heads), half = (a.nblocks + 1) >> 1;
    const int b = (a.zigzag && idx >= half) ? idx - half : a.nblocks - 1 - idx;
    const float *Kh = a.k + (size_t)kvh * a.capacity * D;
    const float *Vh = a.v + (size_t)kvh * a.capacity * D;
    const int col = lane & 15, g = lane >> 4;
    const int heads = a.kv_heads * a.group;
    const int nrows = a.t * a.group;
    const int r = 16 * b + col;
    const bool valid = r < nrows;
    const int i = valid ? r / a.group : 0, hh = valid ? r % a.group : 0;
    const int lim = valid ? a.start + i + 1 : 1;
    const int imax = min(16 * b + 15, nrows - 1) / a.group;
    const int kend = a.start + imax + 1;
    const int nt = (kend + 15) >> 4;
    const int ks = 16 * ((w * nt) >> 2), ke = min(16 * (((w + 1) * nt) >> 2), kend);

    f4 q[S::KJ];
    load_q<D>(a.q + (size_t)i * heads * D + (size_t)(kvh * a.group + hh) * D, a.q, valid, lane, q);
    WaveState<D> st;
    init_state<D>(st);
    attend_range<D, (D < 128), 4>(Kh, Vh, ks, ke, 0, S::TG, lim, a.scale, q, lane, st);
    st.l = col_sum(st.l);
    if (g == 0) {
        sm_m[w][col] = st.m;
        sm_l[w][col] = st.l;
    }
#pragma unroll
    for (int db = 0; db < S::DB; db++)
#pragma unroll
        for (int rr = 0; rr < 4; rr++) sm_o[w][col][out_dim<D>(g, rr, db)] = st.o[db][rr];
    __syncthreads();

    for (int idx = threadIdx.x; idx < 16 * D; idx += blockDim.x) {
        const int c = idx / D, d = idx % D;
        const int rc = 16 * b + c;
        if (rc >= nrows) break;  // rows beyond the chunk are padding
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) M = fmaxf(M, sm_m[ww][c]);
        float o = 0.f, L = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
            const float e = exp2_fast((sm_m[ww][c] - M) * kLog2e);
            o += sm_o[ww][c][d] * e;
            L += sm_l[ww][c] * e;
        }
        const int ic = rc / a.group, hc = rc % a.group;
        a.att[(size_t)ic * heads * D + (size_t)(kvh * a.group + hc) * D + d] = o / L;
    }
}

template <int D>
__global__ __launch_bounds__(256) void prefill_split_kernel(const PrefillArgs a) {
    prefill_split_body<D>(a);
}

// head_dim 128 held to 3 waves per SIMD (at most 168 VGPRs)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void prefill_split_kernel_d128(
    const PrefillArgs a) {
    prefill_split_body<128>(a);
}

// ------------------------------------------------------------------ lean prefill
//
// The split kernel above spends ~113 VALU instructions per 16-key tile on 64
// MFMAs at head_dim 128.  The lean variant keeps its work split (one or two
// 16-row blocks per workgroup, keys split over the 4 waves, heaviest blocks
// first) and runs each tile through lean_load / lean_step (~30 VALU per tile).
//
// Largest cache capacity the lean kernel addresses with 32-bit buffer offsets
// (bytes of one kv head's rows must fit a signed 32-bit range).
template <int D>
constexpr long long lean_max_capacity() { return 0x7fffffffLL / (D * 4); }

// head_dim 64 and 128.  One softmax step covers TG 16-key tiles (two at
// head_dim 64, so that the step's fixed VALU work -- column max, rescale --
// is spread over as many MFMAs as at head_dim 128).  RB consecutive 16-row
// blocks per workgroup: with two, every loaded tile serves both blocks (half
// the tile loads per product), at 2 waves per SIMD.
template <int D, int RB>
__device__ __forceinline__ void prefill_lean_body(const PrefillArgs &a) {
    using S = Shape<D>;
    static_assert(D == 64 || D == 128, "lean prefill: head_dim 64 or 128");
    static_assert(RB == 1 || RB == 2, "lean prefill: one or two row blocks");
    constexpr int TG = S::TG, R = 16 * RB;  // rows per workgroup
    __shared__ float sm_m[4][R], sm_l[4][R], sm_e[4][R], sm_inv[R];
    __shared__ int sm_row[R];
    __shared__ __attribute__((aligned(16))) float sm_o[4][R][D];
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kvh = blockIdx.x % a.kv_heads;
    const int nsb = (a.nblocks + RB - 1) / RB;
    const int idx = (int)(blockIdx.x / a.kv_heads), half = (nsb + 1) >> 1;
    const int sb = (a.zigzag && idx >= half) ? idx - half : nsb - 1 - idx;
    const float *Kh = a.k + (size_t)kvh * a.capacity * D;
    const float *Vh = a.v + (size_t)kvh * a.capacity * D;
    const int col = lane & 15, g = lane >> 4;
    const int heads = a.kv_heads * a.group;
    const int nrows = a.t * a.group;
    const int kend = a.start + min(R * sb + R - 1, nrows - 1) / a.group + 1;
    const int nt = (kend + 15) >> 4;
    const int ks = 16 * ((w * nt) >> 2), ke = min(16 * (((w + 1) * nt) >> 2), kend);

    const float c = a.scale * kLog2e;
    f4 q[RB][S::KJ];
    int klimit[RB], unmasked_end[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int r = R * sb + 16 * rb + col;
        const bool valid = r < nrows;
        const int i = valid ? r / a.group : 0, hh = valid ? r % a.group : 0;
        const int lim = valid ? a.start + i + 1 : kend;  // padding rows see every key
        // smallest limit in the block (a block wholly past the rows: its first row's)
        const int lim_min = a.start + min(R * sb + 16 * rb, nrows - 1) / a.group + 1;
        klimit[rb] = min(lim, ke);
        unmasked_end[rb] = min(lim_min, ke);
        const float *row = valid ? a.q + (size_t)i * heads * D + (size_t)(kvh * a.group + hh) * D : a.q;
        const float keep = valid ? c : 0.f;
#pragma unroll
        for (int j = 0; j < S::KJ; j++) q[rb][j] = *reinterpret_cast<const f4 *>(row + 16 * j + 4 * g) * keep;
    }
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(Kh, (unsigned)kend * D * 4u);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(Vh, (unsigned)kend * D * 4u);
    unsigned vk, vv;
    lean_lane_offsets<D>(lane, vk, vv);

    float m[RB], l[RB];  // m in log2 units
    f4 o[RB][S::DB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        m[rb] = kLazyFloor;
        l[rb] = 0.f;
#pragma unroll
        for (int db = 0; db < S::DB; db++) o[rb][db] = f4{0.f, 0.f, 0.f, 0.f};
    }
    const int nsteps = (ke - ks + 16 * TG - 1) / (16 * TG);
    for (int n = 0; n < nsteps; n++) {
        const int p0 = ks + 16 * TG * n;
        LeanGroup<D> t;
        lean_load<D>(rk, rv, vk, vv, p0, t);
        // keys past a row's causal limit or past the wave's range
        if constexpr (RB == 2 && D == 128) {
            lean_step2<D, TG>(t, q, p0, klimit, g, m, l, o);
        } else {
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
                lean_step<D, true>(t, q[rb], p0, p0 + 16 * TG > unmasked_end[rb], klimit[rb], g, m[rb], l[rb], o[rb]);
        }
    }
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const float ls = col_sum(l[rb]);
        if (g == 0) {
            sm_m[w][16 * rb + col] = m[rb];
            sm_l[w][16 * rb + col] = ls;
        }
#pragma unroll
        for (int db = 0; db < S::DB; db++)
#pragma unroll
            for (int rr = 0; rr < 4; rr++) sm_o[w][16 * rb + col][out_dim<D>(g, rr, db)] = o[rb][db][rr];
    }
    __syncthreads();
    // Merge the 4 waves' states (log2 units); wave 0 holds key 0, so M is
    // finite.  The per-column weights, 1/sum and output row come first, once
    // per column, so the per-element pass is 4 LDS float4 reads and FMAs.
    if (threadIdx.x < R) {
        const int cc = threadIdx.x, rc = min(R * sb + cc, nrows - 1);
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) M = fmaxf(M, sm_m[ww][cc]);
        float L = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
            const float e = exp2_fast(sm_m[ww][cc] - M);
            sm_e[ww][cc] = e;
            L += sm_l[ww][cc] * e;
        }
        sm_inv[cc] = 1.0f / L;
        const int ic = rc / a.group, hc = rc % a.group;
        sm_row[cc] = ic * heads + kvh * a.group + hc;
    }
    __syncthreads();
    const int ncols = min(R, nrows - R * sb);
    for (int x = threadIdx.x; x < ncols * (D / 4); x += blockDim.x) {
        const int cc = x / (D / 4), d = 4 * (x % (D / 4));
        f4 acc = *reinterpret_cast<const f4 *>(&sm_o[0][cc][d]) * sm_e[0][cc];
#pragma unroll
        for (int ww = 1; ww < 4; ww++) acc += *reinterpret_cast<const f4 *>(&sm_o[ww][cc][d]) * sm_e[ww][cc];
        *reinterpret_cast<f4 *>(a.att + (size_t)sm_row[cc] * D + d) = acc * sm_inv[cc];
    }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void prefill_lean_kernel_d128(
    const PrefillArgs a) {
    prefill_lean_body<128, 1>(a);
}

// Two row blocks per workgroup (234 VGPRs, 2 waves per SIMD), for grids that
// still give every CU two workgroups: config 3 T=2048 188.6 -> 175.9 us.  With
// fewer (T=512: one per CU) one block per workgroup is faster, 17.9 against
// 24.4 us.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void prefill_lean2_kernel_d128(
    const PrefillArgs a) {
    prefill_lean_body<128, 2>(a);
}

// head_dim 64 held to 4 waves per SIMD (120 VGPRs, no spills; left to
// itself the compiler takes 139 registers and 3 waves: config 4 95-97 us
// against 89.5-91 us)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void prefill_lean_kernel_d64(
    const PrefillArgs a) {
    prefill_lean_body<64, 1>(a);
}

// Two row blocks per workgroup at head_dim 64 (168 VGPRs, 3 waves per SIMD):
// config 4 82.5 -> 76.8 us per layer.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void prefill_lean2_kernel_d64(
    const PrefillArgs a) {
    prefill_lean_body<64, 2>(a);
}

// ------------------------------------------------------------------ append

// src rows [t][kv_heads*D] -> cache [kv_heads][capacity][D] at start.. (the
// cache write of src/model.rs:481-483).  Pure float4 copies: bit-exact.
template <int D>
__global__ __launch_bounds__(256) void append_kernel(const AppendArgs a) {
    constexpr int V4 = D / 4;
    const size_t total = (size_t)a.t * a.kv_heads * V4;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int j = (int)(idx % V4);
        const size_t rest = idx / V4;
        const int kvh = (int)(rest % a.kv_heads);
        const int i = (int)(rest / a.kv_heads);
        const size_t dst = ((size_t)kvh * a.capacity + a.start + i) * D + 4 * j;
        const size_t src = ((size_t)i * a.kv_heads + kvh) * D + 4 * j;
        *reinterpret_cast<f4 *>(a.k + dst) = *reinterpret_cast<const f4 *>(a.ksrc + src);
        *reinterpret_cast<f4 *>(a.v + dst) = *reinterpret_cast<const f4 *>(a.vsrc + src);
    }
}

// ------------------------------------------------------------------ static decode workspace
//
// The split-K partial states of wick_hip_attention_device_noalloc live in this
// file-scope array instead of a hipMalloc'd buffer, so that entry point never
// allocates.  Every GPU the library runs on holds its own copy until the
// process ends; all calls on one GPU share it, so such calls must not overlap.
// Host code never uses the array's name as an address: kernels receive the
// per-device address hipGetSymbolAddress returns (static_scratch_init).
static __device__ __align__(256) float scratch[kStaticScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_rc[kMaxDevices];
bool g_scratch_done[kMaxDevices];
}  // namespace

hipError_t static_scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_done[device]) {
        // the caller has made `device` current
        void *p = nullptr;
        g_scratch_rc[device] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[device] = g_scratch_rc[device] == hipSuccess ? static_cast<float *>(p) : nullptr;
        g_scratch_done[device] = true;
    }
    return g_scratch_rc[device];
}

float *static_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch_done[device] ? g_scratch_ptr[device] : nullptr;
}

// ------------------------------------------------------------------ launchers

#define WICK_DISPATCH_D(hd, KERNEL, ...)                                              \
    switch (hd) {                                                                     \
    case 16: hipLaunchKernelGGL(KERNEL<16>, __VA_ARGS__); break;                      \
    case 32: hipLaunchKernelGGL(KERNEL<32>, __VA_ARGS__); break;                      \
    case 64: hipLaunchKernelGGL(KERNEL<64>, __VA_ARGS__); break;                      \
    case 128: hipLaunchKernelGGL(KERNEL<128>, __VA_ARGS__); break;                    \
    default: return hipErrorInvalidValue;                                             \
    }

int decode_blocks_per_cu(int head_dim) {
    int n = 0;
    hipError_t e = hipErrorInvalidValue;
    switch (head_dim) {
    case 16: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<16, false>, 256, 0); break;
    case 32: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<32, false>, 256, 0); break;
    case 64: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<64, false>, 256, 0); break;
    case 128: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<128, false>, 256, 0); break;
    default: break;
    }
    return (e == hipSuccess && n > 0) ? n : 1;
}

// decode_kernel<D, ...> launched with the VALU core when the unit holds at
// most 4 query heads at head_dim 64 (the template's NC = the group).
// The VALU core instance; with PREP the preparation is wave-local (RP) for
// up to 3 heads (4 heads' q rows and tiles would not fit the registers of 8
// waves per workgroup without spilling).
template <int D, bool PREP, int NW, bool OPROJ, int NC>
void launch_valu_core(const DecodeArgs &a, dim3 grid, dim3 block, hipStream_t s) {
    constexpr int TG = Shape<D>::TG;
    hipLaunchKernelGGL((decode_kernel<D, PREP, false, NW, TG, OPROJ, NC, PREP && NC < 4>), grid, block, 0, s, a);
}

template <int D, bool PREP, bool PP, int NW, bool OPROJ = false>
void launch_decode_core(const DecodeArgs &a, dim3 grid, hipStream_t s) {
    constexpr int TG = Shape<D>::TG;
    const dim3 block(64 * NW);
    const int nc = (D == 64 && a.group <= 4) ? a.group : 0;
    if constexpr (D == 64) {
        switch (nc) {
        case 1: launch_valu_core<D, PREP, NW, OPROJ, 1>(a, grid, block, s); return;
        case 2: launch_valu_core<D, PREP, NW, OPROJ, 2>(a, grid, block, s); return;
        case 3: launch_valu_core<D, PREP, NW, OPROJ, 3>(a, grid, block, s); return;
        case 4: launch_valu_core<D, PREP, NW, OPROJ, 4>(a, grid, block, s); return;
        default: break;
        }
    }
    if constexpr (D >= 64 && NW == 4 && !OPROJ) {
        if (a.interleave) {
            hipLaunchKernelGGL((decode_kernel<D, PREP, PP, NW, TG, OPROJ, 0, false, true>), grid, block, 0, s, a);
            return;
        }
    }
    hipLaunchKernelGGL((decode_kernel<D, PREP, PP, NW, TG, OPROJ, 0>), grid, block, 0, s, a);
}

template <int D>
void launch_decode_d(const DecodeArgs &a, int grid, hipStream_t s) {
    if constexpr (D <= 64) {
        if (a.nchunks == 1 && a.chunk > 4 * Shape<D>::TG * 16) {
            // one chunk per unit: 8 waves, each with at most one or two groups
            const bool one8 = a.chunk <= 8 * Shape<D>::TG * 16;
            if (a.prep && one8)
                launch_decode_core<D, true, false, 8>(a, dim3(grid), s);
            else if (a.prep)
                launch_decode_core<D, true, true, 8>(a, dim3(grid), s);
            else if (one8)
                launch_decode_core<D, false, false, 8>(a, dim3(grid), s);
            else
                launch_decode_core<D, false, true, 8>(a, dim3(grid), s);
            return;
        }
    }
    // each of the 4 waves takes groups of TG 16-key tiles, stepping by 4 groups
    const bool one_group = a.chunk <= 4 * Shape<D>::TG * 16;
    if constexpr (D < 128) {
        if (one_group) {
            if (a.prep)
                launch_decode_core<D, true, false, 4>(a, dim3(grid), s);
            else
                launch_decode_core<D, false, false, 4>(a, dim3(grid), s);
            return;
        }
    }
    if (a.prep)
        launch_decode_core<D, true, (D < 128), 4>(a, dim3(grid), s);
    else
        launch_decode_core<D, false, (D < 128), 4>(a, dim3(grid), s);
}

template <int D>
void launch_merge(int nb, dim3 grid, const DecodeArgs &a, hipStream_t s) {
    switch (nb) {
    case 1: hipLaunchKernelGGL((decode_merge_kernel<D, 1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((decode_merge_kernel<D, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((decode_merge_kernel<D, 4>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((decode_merge_kernel<D, 8>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((decode_merge_kernel<D, 16>), grid, dim3(256), 0, s, a); break;
    }
}

hipError_t launch_decode(int head_dim, const DecodeArgs &a, int grid, hipStream_t s) {
    switch (head_dim) {
    case 16: launch_decode_d<16>(a, grid, s); break;
    case 32: launch_decode_d<32>(a, grid, s); break;
    case 64: launch_decode_d<64>(a, grid, s); break;
    case 128: launch_decode_d<128>(a, grid, s); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nchunks == 1) return e;
    const dim3 mgrid((unsigned)(a.kv_heads * a.group * (head_dim / 16)));
    // 16 thread groups x NB child slots cover the chunks
    const int nb = a.nchunks <= 16 ? 1 : a.nchunks <= 32 ? 2 : a.nchunks <= 64 ? 4 : a.nchunks <= 128 ? 8 : 16;
    switch (head_dim) {
    case 16: launch_merge<16>(nb, mgrid, a, s); break;
    case 32: launch_merge<32>(nb, mgrid, a, s); break;
    case 64: launch_merge<64>(nb, mgrid, a, s); break;
    case 128: launch_merge<128>(nb, mgrid, a, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool decode_interleaves(int head_dim, int group, int nchunks, int chunk) {
    // the lean MFMA core's 4-wave split (not the VALU core of head_dim 64 with
    // at most 4 heads per unit), with chunks of at least kDecodeInterleaveRounds
    // rounds of the 4 waves' key groups: every chunk's wave 0 then has a group
    // (len > (nchunks - 1) * chunk), and each wave about that many full rounds
    if (nchunks < 2 || (head_dim != 64 && head_dim != 128) || (head_dim == 64 && group <= 4)) return false;
    const int gk = 16 * (head_dim == 128 ? Shape<128>::TG : Shape<64>::TG);  // keys per group
    return chunk >= kDecodeInterleaveRounds * 4 * gk;
}

bool decode_oproj_supported(int head_dim, int group, int nchunks, int chunk) {
    // one chunk per unit, of at most kOprojMaxChunk keys: each wave of a
    // workgroup takes at most one group of tiles (8 waves x 32 keys at head_dim
    // 64; head_dim 128 loops over 16-key groups)
    if (nchunks != 1 || chunk > kOprojMaxChunk || (head_dim != 64 && head_dim != 128)) return false;
    const int ncols = group < kTileRows ? group : kTileRows;
    return ncols * head_dim <= 64 * kOprojChunks;
}

hipError_t launch_decode_oproj(int head_dim, DecodeArgs a, hipStream_t s) {
    if (!a.prep || !decode_oproj_supported(head_dim, a.group, a.nchunks, a.chunk)) return hipErrorInvalidValue;
    // 8 waves split the keys, one wo row each: the widest grid measured best
    // (1, 2, 4 rows per wave: 216 / 108 / 54 workgroups for SmolLM2, e2e
    // 1845 / 1824 / 1795 tok/s; 4 waves per workgroup 1728)
    constexpr int NW = 8;
    const int blocks = (a.hidden + NW * kOprojRows - 1) / (NW * kOprojRows);
    const dim3 grid((unsigned)(a.kv_heads * a.hslices * blocks));
    if (head_dim == 64)
        launch_decode_core<64, true, false, NW, true>(a, grid, s);
    else
        launch_decode_core<128, true, false, NW, true>(a, grid, s);
    return hipGetLastError();
}

int prefill_blocks_per_cu(int head_dim, int rows32) {
    int n = 0;
    hipError_t e = hipErrorInvalidValue;
    switch (head_dim) {
    case 16: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_split_kernel<16>, 256, 0); break;
    case 32: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_split_kernel<32>, 256, 0); break;
    case 64:
        e = rows32 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_lean2_kernel_d64, 256, 0)
                   : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_lean_kernel_d64, 256, 0);
        break;
    case 128:
        e = rows32 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_lean2_kernel_d128, 256, 0)
                   : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_lean_kernel_d128, 256, 0);
        break;
    default: break;
    }
    return (e == hipSuccess && n > 0) ? n : 1;
}

bool prefill_has_rows32(int head_dim, int capacity) {
    if (head_dim == 128) return capacity <= lean_max_capacity<128>();
    if (head_dim == 64) return capacity <= lean_max_capacity<64>();
    return false;
}

// A lean kernel with two row blocks per workgroup.
static bool prefill_uses_rows32(int head_dim, const PrefillArgs &a) {
    return a.rows32 && prefill_has_rows32(head_dim, a.capacity);
}

int prefill_grid(int head_dim, const PrefillArgs &a) {
    if (prefill_uses_rows32(head_dim, a)) return a.kv_heads * ((a.nblocks + 1) / 2);
    return a.kv_heads * a.nblocks;
}

hipError_t launch_prefill(int head_dim, const PrefillArgs &a, hipStream_t s) {
    const int grid = prefill_grid(head_dim, a);
    if (prefill_uses_rows32(head_dim, a) && head_dim == 128) {
        hipLaunchKernelGGL(prefill_lean2_kernel_d128, dim3(grid), dim3(256), 0, s, a);
    } else if (prefill_uses_rows32(head_dim, a)) {
        hipLaunchKernelGGL(prefill_lean2_kernel_d64, dim3(grid), dim3(256), 0, s, a);
    } else if (head_dim == 128 && a.capacity <= lean_max_capacity<128>()) {
        hipLaunchKernelGGL(prefill_lean_kernel_d128, dim3(grid), dim3(256), 0, s, a);
    } else if (head_dim == 64 && a.capacity <= lean_max_capacity<64>()) {
        hipLaunchKernelGGL(prefill_lean_kernel_d64, dim3(grid), dim3(256), 0, s, a);
    } else if (head_dim == 128) {
        hipLaunchKernelGGL(prefill_split_kernel_d128, dim3(grid), dim3(256), 0, s, a);
    } else {
        WICK_DISPATCH_D(head_dim, prefill_split_kernel, dim3(grid), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_append(int head_dim, const AppendArgs &a, hipStream_t s) {
    const size_t total = (size_t)a.t * a.kv_heads * (head_dim / 4);
    size_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks == 0) return hipSuccess;
    WICK_DISPATCH_D(head_dim, append_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace wick
