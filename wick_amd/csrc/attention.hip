// attention.hip -- causal GQA attention over a device-resident KV cache, gfx950.
//
// Replaces Model::attention (/root/reference/src/model.rs:518-553): for every
// (token i, query head h) of a chunk of t tokens at positions start..start+t,
//   att[i,h,:] = sum_{p <= start+i} softmax_p(q[i,h] . K[p, h/group] * scale) V[p, h/group, :]
// with scale = 1/sqrt(head_dim) (src/model.rs:527) and kv head h/group
// (src/model.rs:526,532).
//
// Both kernels are built on one wave-level core (attend_range): a wave owns 16
// "columns" -- 16 query heads of one kv head (decode) or 16 flattened
// (token, head) rows of one kv head (prefill) -- and streams 16-key tiles of K
// and V through two f32 MFMAs:
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

#include <math.h>

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

// max / sum over the four lanes that hold the same column (l, l^16, l^32, l^48)
__device__ __forceinline__ float col_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float col_sum(float v) {
    v += __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
}

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

template <int D>
__device__ __forceinline__ void compute_tiles(const TileBuf<D> &b, int kbeg, int first, int klimit, float scale,
                                              const f4 (&q)[Shape<D>::KJ], int lane, WaveState<D> &st) {
    using S = Shape<D>;
    const int g = lane >> 4;
    float sc[S::TG][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int u = 0; u < S::TG; u++) {
        f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < S::KJ; j++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (j & 1) s1 = mfma16x16x4(b.k[u][j][e], q[j][e], s1);
                else       s0 = mfma16x16x4(b.k[u][j][e], q[j][e], s0);
            }
        }
        const f4 s = s0 + s1;
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
    st.l *= alpha;
#pragma unroll
    for (int db = 0; db < S::DB; db++) st.o[db] *= alpha;
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
template <int D, bool PINGPONG = true>
__device__ __forceinline__ void attend_range(const float *__restrict__ Kh, const float *__restrict__ Vh, int kbeg,
                                             int kend, int tile0, int tstep, int klimit, float scale,
                                             const f4 (&q)[Shape<D>::KJ], int lane, WaveState<D> &st) {
    const int ntiles = (kend - kbeg + 15) >> 4;
    klimit = min(klimit, kend);
    if constexpr (!PINGPONG) {
        TileBuf<D> b;
        for (int first = tile0; first < ntiles; first += tstep) {
            load_tiles<D>(Kh, Vh, kbeg, kend, first, lane, b);
            compute_tiles<D>(b, kbeg, first, klimit, scale, q, lane, st);
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
        compute_tiles<D>(ba, kbeg, first, klimit, scale, q, lane, st);
        first = next;
        if (first >= ntiles) break;
        next = first + tstep;
        if (next < ntiles) load_tiles<D>(Kh, Vh, kbeg, kend, next, lane, ba);
        compute_tiles<D>(bb, kbeg, first, klimit, scale, q, lane, st);
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

template <int D>
__device__ __forceinline__ void init_state(WaveState<D> &st) {
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int db = 0; db < Shape<D>::DB; db++) st.o[db] = f4{0.f, 0.f, 0.f, 0.f};
}

// ------------------------------------------------------------------ decode

// Workspace layout (floats), independent of the per-call chunk count; each
// (unit, column) owns a contiguous run of child states, so a merge reads one
// contiguous block:
//   O0 [units][16 cols][256 chunks][D], m0 [units][16][256], l0 [units][16][256],
//   O1 [units][16 cols][16 groups][D],  m1 [units][16][16],  l1 [units][16][16]
size_t decode_workspace_floats(int units, int head_dim) {
    return (size_t)units * ((size_t)kDecodeMaxChunks * 16 * (head_dim + 2) + (size_t)kDecodeFan * 16 * (head_dim + 2));
}

// A set of partial (O, m, l) states: state (child ch, column col) lives at
// o[(col*cs + ch)*D ..], m[col*cs + ch], l[col*cs + ch].
struct PView {
    float *o, *m, *l;
    int cs;
};

template <int D>
struct DecodeSpace {
    PView p0, p1;  // per-chunk states and per-group states, both for unit 0
    __device__ DecodeSpace(float *part, int units) {
        const size_t U = (size_t)units;
        p0.o = part;
        p0.m = p0.o + U * 16 * kDecodeMaxChunks * D;
        p0.l = p0.m + U * 16 * kDecodeMaxChunks;
        p0.cs = kDecodeMaxChunks;
        p1.o = p0.l + U * 16 * kDecodeMaxChunks;
        p1.m = p1.o + U * 16 * kDecodeFan * D;
        p1.l = p1.m + U * 16 * kDecodeFan;
        p1.cs = kDecodeFan;
    }
    // The states of `unit`, starting at child `first`.
    __device__ static PView at(const PView &p, int unit, int first) {
        const size_t base = (size_t)unit * 16 * p.cs + first;
        return PView{p.o + base * D, p.m + base, p.l + base, p.cs};
    }
};

// Device-scope (sc1) stores and loads: they bypass the caches that are not
// coherent across the chip's XCDs, so a state stored by one workgroup and
// loaded by another after a counter handshake needs no L2 writeback or
// invalidate (both of which a release/acquire fence would issue per wave).
__device__ __forceinline__ void st_dev(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until this wave's device-scope stores have completed (are visible to
// every CU), then take a ticket from *cnt once the whole workgroup has done so.
// This is the release sequence the AMDGPU memory model uses for atomic stores,
// without the L2 writeback that only non-atomic stores need.
__device__ __forceinline__ int publish_and_count(int *cnt, int &ticket_smem) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) ticket_smem = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    return ticket_smem;
}

// Merge n <= 16 child states of one unit (view c) in child order, either into
// one state stored with device-scope stores (view out) or -- when att != NULL --
// into the normalised output att[(head0 + col)*D + d].  All child loads are
// issued together.  Fixed order: the result does not depend on which
// workgroup runs the merge.
template <int D>
__device__ void merge_children(const PView &c, int n, int ncols, const PView &out, float *att, int head0,
                               float (&sw)[16][kDecodeFan], float (&sml)[2][16][kDecodeFan]) {
    const int tid = threadIdx.x;
    if (tid < 16 * kDecodeFan) {
        const int col = tid / kDecodeFan, ch = tid % kDecodeFan;
        const bool live = ch < n && col < ncols;
        sml[0][col][ch] = live ? ld_dev(c.m + col * c.cs + ch) : -INFINITY;
        sml[1][col][ch] = live ? ld_dev(c.l + col * c.cs + ch) : 0.f;
    }
    float v[kDecodeFan];
    const int idx0 = tid;  // first (col, d) of this thread; ncols*D <= 2048 = 8 * 256
    __syncthreads();
    if (tid < 16) {
        float M = -INFINITY;
#pragma unroll
        for (int ch = 0; ch < kDecodeFan; ch++) M = fmaxf(M, sml[0][tid][ch]);
        const float Mref = (M == -INFINITY) ? 0.f : M;
        float L = 0.f;
#pragma unroll
        for (int ch = 0; ch < kDecodeFan; ch++) {
            const float e = exp2_fast((sml[0][tid][ch] - Mref) * kLog2e);
            sw[tid][ch] = e;
            L += sml[1][tid][ch] * e;
        }
        if (!att && tid < ncols) {
            st_dev(out.m + tid * out.cs, M);
            st_dev(out.l + tid * out.cs, L);
        }
        sml[1][tid][0] = L;  // total, read below for normalisation
    }
    __syncthreads();
    for (int idx = idx0; idx < ncols * D; idx += blockDim.x) {
        const int col = idx / D, d = idx % D;
#pragma unroll
        for (int ch = 0; ch < kDecodeFan; ch++) v[ch] = ch < n ? ld_dev(c.o + ((size_t)col * c.cs + ch) * D + d) : 0.f;
        float o = 0.f;
#pragma unroll
        for (int ch = 0; ch < kDecodeFan; ch++) o += v[ch] * sw[col][ch];
        if (att) att[(size_t)(head0 + col) * D + d] = o / sml[1][col][0];
        else st_dev(out.o + (size_t)col * out.cs * D + d, o);
    }
}

// One token (t = 1) over len cached positions, split-K: workgroup
// (unit, chunk) runs 4 waves over positions chunk*C .. +C of one kv head for
// up to 16 of its query heads (unit = kv head x 16-head slice), so every K/V
// byte is read once for the whole GQA group.  Partial (max, sum, O) states are
// merged by log-sum-exp, either by decode_merge_kernel (merge_mode 1) or in a
// fixed-order tree of fan-in 16 inside this kernel (merge_mode 0), whose
// last-arriving workgroup at each level does the merge and resets the level's
// counter (so no memset is needed between launches).
template <int D>
__global__ __launch_bounds__(256) void decode_kernel(const DecodeArgs a) {
    using S = Shape<D>;
    __shared__ float sm_m[4][16], sm_l[4][16];
    __shared__ float sm_o[4][16][D];
    __shared__ float sm_w[16][kDecodeFan], sm_ml[2][16][kDecodeFan];
    __shared__ int s_ticket;

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int units = a.kv_heads * a.hslices;
    const int unit = blockIdx.x % units, chunk = blockIdx.x / units;
    const int kvh = unit / a.hslices, slice = unit % a.hslices;
    const int col0 = slice * 16, ncols = min(16, a.group - col0);
    const int head0 = kvh * a.group + col0;
    const float *Kh = a.k + (size_t)kvh * a.capacity * D;
    const float *Vh = a.v + (size_t)kvh * a.capacity * D;
    const int kbeg = chunk * a.chunk, kend = min(kbeg + a.chunk, a.len);

    const int col = lane & 15, g = lane >> 4;
    f4 q[S::KJ];
    load_q<D>(a.q + (size_t)(head0 + col) * D, a.q + (size_t)head0 * D, col < ncols, lane, q);

    WaveState<D> st;
    init_state<D>(st);
    attend_range<D, (D < 128)>(Kh, Vh, kbeg, kend, w * S::TG, 4 * S::TG, a.len, a.scale, q, lane, st);
    st.l = col_sum(st.l);

    if (g == 0) {
        sm_m[w][col] = st.m;
        sm_l[w][col] = st.l;
    }
#pragma unroll
    for (int db = 0; db < S::DB; db++)
#pragma unroll
        for (int r = 0; r < 4; r++) sm_o[w][col][out_dim<D>(g, r, db)] = st.o[db][r];
    __syncthreads();

    // Merge the 4 waves of this workgroup.  Wave 0 always holds the chunk's
    // first key, so the merged max is finite.
    const DecodeSpace<D> ws(a.part, units);
    const PView mine = DecodeSpace<D>::at(ws.p0, unit, chunk);
    const bool in_kernel = a.merge_mode == 0;
    for (int idx = threadIdx.x; idx < ncols * D; idx += blockDim.x) {
        const int c = idx / D, d = idx % D;
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
        if (a.nchunks == 1) {
            a.att[(size_t)(head0 + c) * D + d] = o / L;
        } else if (in_kernel) {
            st_dev(mine.o + (size_t)c * mine.cs * D + d, o);
            if (d == 0) {
                st_dev(mine.m + c * mine.cs, M);
                st_dev(mine.l + c * mine.cs, L);
            }
        } else {
            mine.o[(size_t)c * mine.cs * D + d] = o;
            if (d == 0) {
                mine.m[c * mine.cs] = M;
                mine.l[c * mine.cs] = L;
            }
        }
    }
    if (a.nchunks == 1 || !in_kernel) return;

    // Level 1: the last of the (up to) 16 chunks of a group merges the group.
    const int grp = chunk / kDecodeFan, gfirst = grp * kDecodeFan;
    const int nin = min(kDecodeFan, a.nchunks - gfirst);
    int *cnt1 = a.counters + (size_t)unit * (kDecodeFan + 1) + grp;
    int *cnt2 = a.counters + (size_t)unit * (kDecodeFan + 1) + kDecodeFan;
    if (publish_and_count(cnt1, s_ticket) != nin - 1) return;
    if (threadIdx.x == 0) __hip_atomic_store(cnt1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    const PView child = DecodeSpace<D>::at(ws.p0, unit, gfirst);
    if (a.ngroups == 1) {
        merge_children<D>(child, nin, ncols, PView{}, a.att, head0, sm_w, sm_ml);
        return;
    }
    merge_children<D>(child, nin, ncols, DecodeSpace<D>::at(ws.p1, unit, grp), nullptr, head0, sm_w, sm_ml);

    // Level 2: the last group merger of this unit writes the output.
    if (publish_and_count(cnt2, s_ticket) != a.ngroups - 1) return;
    if (threadIdx.x == 0) __hip_atomic_store(cnt2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    merge_children<D>(DecodeSpace<D>::at(ws.p1, unit, 0), a.ngroups, ncols, PView{}, a.att, head0, sm_w, sm_ml);
}

// Separate merge pass (merge_mode 1): workgroup (unit, col) merges the
// nchunks (<= 256) partial states of one query head in chunk order; they are
// contiguous in the workspace.  Thread (grp, d) of 256/D groups owns children
// grp, grp + 256/D, ...; all of its O loads and the (m, l) loads (one child per
// thread) are issued before any is used, so the pass costs one memory round
// trip.  Per-thread sums run in child order and the group sums are combined
// in group order: deterministic for a given nchunks.
template <int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(const DecodeArgs a) {
    constexpr int G = 256 / D;                  // thread groups over children
    constexpr int NU = kDecodeMaxChunks / G;    // children per thread at most
    __shared__ float sw[kDecodeMaxChunks];
    __shared__ float red[4];
    __shared__ float so[G][D];
    const int units = a.kv_heads * a.hslices;
    const int unit = blockIdx.x / 16, col = blockIdx.x % 16;
    const int kvh = unit / a.hslices, slice = unit % a.hslices;
    const int col0 = slice * 16, ncols = min(16, a.group - col0);
    if (col >= ncols) return;
    const int head = kvh * a.group + col0 + col;
    const DecodeSpace<D> ws(a.part, units);
    const PView c = DecodeSpace<D>::at(ws.p0, unit, 0);
    const float *co = c.o + (size_t)col * c.cs * D;
    const float *cm = c.m + col * c.cs;
    const float *cl = c.l + col * c.cs;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = a.nchunks;
    const int grp = tid / D, d = tid % D;

    float v[NU];
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const int ch = grp + u * G;
        v[u] = ch < n ? co[(size_t)ch * D + d] : 0.f;
    }
    const float mv = tid < n ? cm[tid] : -INFINITY;
    const float lv = tid < n ? cl[tid] : 0.f;
    float M = mv;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    if (lane == 0) red[w] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float e = exp2_fast((mv - M) * kLog2e);
    sw[tid] = e;
    float L = lv * e;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) L += __shfl_xor(L, off);
    __syncthreads();
    if (lane == 0) red[w] = L;
    __syncthreads();
    L = (red[0] + red[1]) + (red[2] + red[3]);

    float o = 0.f;
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const int ch = grp + u * G;
        if (ch < n) o += v[u] * sw[ch];
    }
    so[grp][d] = o;
    __syncthreads();
    if (tid < D) {
        float acc = 0.f;
#pragma unroll
        for (int gg = 0; gg < G; gg++) acc += so[gg][tid];
        a.att[(size_t)head * D + tid] = acc / L;
    }
}

// ------------------------------------------------------------------ prefill

// Rows of one kv head are the flattened (token i, head hh) pairs r = i*group + hh,
// so the GQA heads of a token share every K/V tile.  Each wave owns a block of
// 16 rows and runs over all keys that block can see (0 .. start + last token),
// masking per row; with pairing, a wave takes row blocks b and nblocks-1-b so
// that every wave of a causal launch does the same amount of work.
template <int D>
__device__ __forceinline__ void prefill_block(const PrefillArgs &a, const float *Kh, const float *Vh, int kvh, int b,
                                              int lane) {
    using S = Shape<D>;
    const int col = lane & 15, g = lane >> 4;
    const int heads = a.kv_heads * a.group;
    const int nrows = a.t * a.group;
    const int r = 16 * b + col;
    const bool valid = r < nrows;
    const int i = valid ? r / a.group : 0, hh = valid ? r % a.group : 0;
    const int lim = valid ? a.start + i + 1 : 1;
    const int imax = min(16 * b + 15, nrows - 1) / a.group;
    const int kend = a.start + imax + 1;
    const size_t qoff = (size_t)i * heads * D + (size_t)(kvh * a.group + hh) * D;

    f4 q[S::KJ];
    load_q<D>(a.q + qoff, a.q, valid, lane, q);
    WaveState<D> st;
    init_state<D>(st);
    attend_range<D>(Kh, Vh, 0, kend, 0, S::TG, lim, a.scale, q, lane, st);
    const float inv_l = 1.0f / col_sum(st.l);
    if (!valid) return;
    float *out = a.att + qoff;
#pragma unroll
    for (int db = 0; db < S::DB; db++)
#pragma unroll
        for (int rr = 0; rr < 4; rr++) out[out_dim<D>(g, rr, db)] = st.o[db][rr] * inv_l;
}

template <int D>
__global__ __launch_bounds__(256) void prefill_kernel(const PrefillArgs a) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int kvh = blockIdx.x % a.kv_heads;
    const int item = (blockIdx.x / a.kv_heads) * 4 + w;
    if (item >= a.items) return;
    const float *Kh = a.k + (size_t)kvh * a.capacity * D;
    const float *Vh = a.v + (size_t)kvh * a.capacity * D;
    if (a.paired) {
        const int b1 = a.nblocks - 1 - item;
        prefill_block<D>(a, Kh, Vh, kvh, b1, lane);
        if (b1 != item) prefill_block<D>(a, Kh, Vh, kvh, item, lane);
    } else {
        prefill_block<D>(a, Kh, Vh, kvh, item, lane);
    }
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
    case 16: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<16>, 256, 0); break;
    case 32: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<32>, 256, 0); break;
    case 64: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<64>, 256, 0); break;
    case 128: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<128>, 256, 0); break;
    default: break;
    }
    return (e == hipSuccess && n > 0) ? n : 1;
}

hipError_t launch_decode(int head_dim, const DecodeArgs &a, int grid, hipStream_t s) {
    WICK_DISPATCH_D(head_dim, decode_kernel, dim3(grid), dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nchunks == 1 || a.merge_mode != 1) return e;
    const int units = a.kv_heads * a.hslices;
    WICK_DISPATCH_D(head_dim, decode_merge_kernel, dim3(units * 16), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_prefill(int head_dim, const PrefillArgs &a, int grid, hipStream_t s) {
    WICK_DISPATCH_D(head_dim, prefill_kernel, dim3(grid), dim3(256), 0, s, a);
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
