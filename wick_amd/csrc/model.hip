// model.hip -- the non-attention kernels of a device-resident Model::forward
// (/root/reference/src/model.rs:420-516): matrix-vector products with fused
// RMSNorm prologues and residual / SwiGLU / q-k-v epilogues, the embedding
// gather and the greedy sampler.
//
// Decode (t = 1) is HBM-bound: every weight is read once per token.  One wave
// owns one output row, streams it with float4 loads (a wave reads 1 KiB of the
// row per instruction) and reduces its 64 partial sums with a fixed butterfly,
// so results are deterministic run to run.  For t > 1 each wave handles 4
// tokens per weight pass (grid.y walks the token groups); the weight rows are
// then re-read from L2 / MALL once per group.
#include <hip/hip_runtime.h>

#include <math.h>

#include "model_kernels.h"
#include "wave_ops.h"

namespace wick {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot4(const f4 w, const f4 x, float acc) {
    acc = fmaf(w.x, x.x, acc);
    acc = fmaf(w.y, x.y, acc);
    acc = fmaf(w.z, x.z, acc);
    return fmaf(w.w, x.w, acc);
}

// Keeps (v, i) when v is larger, or equal at a smaller index: the first index
// of the maximum over the non-NaN values (NaN never compares greater).
__device__ __forceinline__ void arg_better(float v, int i, float &bv, int &bi) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

}  // namespace

// One wave per R output rows (rows R*wave .. R*wave+R-1), NT tokens per wave
// (token group blockIdx.y).  Column c4 (a float4 index) of a row is handled by
// lane c4 % 64; a pass covers 64*UNR float4s of every row.  All loads a pass
// needs -- weight rows, input rows, norm weight, and the residual being added
// to -- are issued before the first arithmetic on them, so a kernel whose rows
// fit one pass waits for memory once.
template <int NT, int R, int UNR, int EPI, bool NORM>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvArgs a) {
    static_assert(EPI != kEpiSwiglu || R == 1, "SwiGLU pairs one gate row with one up row");
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= a.rows) return;  // whole waves only; no barriers below
    const int tok0 = blockIdx.y * NT;
    const int nt = min(NT, a.t - tok0);
    const int C4 = a.cols >> 2;
    const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const f4 *X[NT];
#pragma unroll
    for (int tk = 0; tk < NT; tk++) X[tk] = reinterpret_cast<const f4 *>(a.x + (size_t)(tok0 + min(tk, nt - 1)) * a.cols);
    const f4 *W[R];
#pragma unroll
    for (int r = 0; r < R; r++) W[r] = reinterpret_cast<const f4 *>(a.w + (size_t)min(row0 + r, a.rows - 1) * a.cols);
    const f4 *W2 = EPI == kEpiSwiglu ? reinterpret_cast<const f4 *>(a.w2 + (size_t)row0 * a.cols) : W[0];
    const f4 *G = reinterpret_cast<const f4 *>(a.norm);

    // the first pass's weights go out before anything waits on memory
    f4 wv[R][UNR], wv2[UNR];
#pragma unroll
    for (int u = 0; u < UNR; u++) {
        const int c = lane + 64 * u;
#pragma unroll
        for (int r = 0; r < R; r++) wv[r][u] = c < C4 ? __builtin_nontemporal_load(W[r] + c) : zero;
        if (EPI == kEpiSwiglu) wv2[u] = c < C4 ? __builtin_nontemporal_load(W2 + c) : zero;
    }
    // the values the residual epilogue adds to (lane tk: token tk, one per row)
    float resid[EPI == kEpiResid ? R : 1];
    if constexpr (EPI == kEpiResid) {
        const float *src = a.resid ? a.resid : a.out0;
#pragma unroll
        for (int r = 0; r < R; r++)
            resid[r] = (lane < nt && row0 + r < a.rows) ? src[(size_t)(tok0 + lane) * a.ld0 + row0 + r] : 0.0f;
    }

    // rmsnorm (src/kernels.rs:343-349) of each input row: xn = x * scale * g
    float scale[NT];
    if (NORM) {
#pragma unroll
        for (int tk = 0; tk < NT; tk++) {
            float ss = 0.0f;
            for (int c = lane; c < C4; c += 64) {
                const f4 v = X[tk][c];
                ss = dot4(v, v, ss);
            }
            ss = wave_sum(ss);
            scale[tk] = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
        }
    }

    float acc[R][NT], acc2[NT];
#pragma unroll
    for (int tk = 0; tk < NT; tk++) {
        acc2[tk] = 0.0f;
#pragma unroll
        for (int r = 0; r < R; r++) acc[r][tk] = 0.0f;
    }
    for (int base = 0; base < C4; base += 64 * UNR) {
        if (base > 0) {
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int c = base + lane + 64 * u;
#pragma unroll
                for (int r = 0; r < R; r++) wv[r][u] = c < C4 ? __builtin_nontemporal_load(W[r] + c) : zero;
                if (EPI == kEpiSwiglu) wv2[u] = c < C4 ? __builtin_nontemporal_load(W2 + c) : zero;
            }
        }
        f4 xv[NT][UNR], gv[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int c = base + lane + 64 * u;
            if (NORM) gv[u] = c < C4 ? G[c] : zero;
#pragma unroll
            for (int tk = 0; tk < NT; tk++) xv[tk][u] = c < C4 ? X[tk][c] : zero;
        }
#pragma unroll
        for (int u = 0; u < UNR; u++) {
#pragma unroll
            for (int tk = 0; tk < NT; tk++) {
                f4 x = xv[tk][u];
                if (NORM) x = x * scale[tk] * gv[u];
#pragma unroll
                for (int r = 0; r < R; r++) acc[r][tk] = dot4(wv[r][u], x, acc[r][tk]);
                if (EPI == kEpiSwiglu) acc2[tk] = dot4(wv2[u], x, acc2[tk]);
            }
        }
    }
#pragma unroll
    for (int tk = 0; tk < NT; tk++) {
#pragma unroll
        for (int r = 0; r < R; r++) acc[r][tk] = wave_sum(acc[r][tk]);
        if (EPI == kEpiSwiglu) acc2[tk] = wave_sum(acc2[tk]);
    }
    // lane tk writes token tk's values
#pragma unroll
    for (int tk = 0; tk < NT; tk++) {
        if (lane != tk || tk >= nt) continue;
        const size_t tok = (size_t)tok0 + tk;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = row0 + r;
            if (row >= a.rows) break;
            const float d = acc[r][tk];
            if (EPI == kEpiStore || EPI == kEpiArgmax) {
                a.out0[tok * a.ld0 + row] = d;
            } else if (EPI == kEpiResid) {
                a.out0[tok * a.ld0 + row] = resid[r] + d;
            } else if (EPI == kEpiQkv) {
                if (row < a.split0)
                    a.out0[tok * a.ld0 + row] = d;
                else if (row < a.split1)
                    a.out1[tok * a.ld1 + (row - a.split0)] = d;
                else
                    a.out2[tok * a.ld2 + (row - a.split1)] = d;
            } else {  // silu_mul: g / (1 + exp(-g)) * u
                a.out0[tok * a.ld0 + row] = d / (1.0f + expf(-d)) * acc2[tk];
            }
        }
    }
    if constexpr (EPI == kEpiArgmax) {
        // the wave's rows in increasing order; argmax_kernel reduces the pairs
        static_assert(NT == 1 && R == kArgmaxRows, "one token, one pair per kArgmaxRows rows");
        if (lane == 0) {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int r = 0; r < R; r++)
                if (row0 + r < a.rows) arg_better(acc[r][0], row0 + r, bv, bi);
            reinterpret_cast<float2 *>(a.out1)[row0 / R] = make_float2(bv, __int_as_float(bi));
        }
    }
}

// One token, rows of up to 64 * UNR float4s (one pass): the input row is
// staged through LDS once per workgroup instead of being read by every wave.
// Thread t owns float4s t, t + 256, ... of the row: it loads x (plus, with
// NP > 0, the a.nparts partial vectors added in order -- the fused decode's
// per-unit output projections, the residual add of src/model.rs:486-487 --
// and the block-0 threads write that sum to a.xout), the norm weight, and its
// share of the sum of squares; the 4 waves' sums meet in LDS in a fixed order.
// Each wave owns R output rows, whose weights it requests first, so the
// kernel waits for memory once; epilogues as gemv_kernel's.
template <int R, int UNR, int EPI, bool NORM, int NP>
__global__ __launch_bounds__(256) void gemv1_kernel(const GemvArgs a) {
    static_assert(EPI != kEpiSwiglu || R == 1, "SwiGLU pairs one gate row with one up row");
    constexpr int XK = (64 * UNR + 255) / 256;  // float4s of the row per thread
    __shared__ f4 sx[256 * XK];
    __shared__ f4 sg[NORM ? 256 * XK : 1];
    __shared__ float sss[4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, t = threadIdx.x;
    const int row0 = (blockIdx.x * 4 + w) * R;
    const bool live = row0 < a.rows;  // every wave reaches the barrier
    const int C4 = a.cols >> 2;
    const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};

    // Loads from clamped, in-bounds indices with no condition, and selects
    // afterwards: a load under a per-lane condition becomes an exec-mask
    // branch of its own, which serialises the issue of the loads.
    f4 wv[R][UNR], wv2[UNR];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const f4 *W = reinterpret_cast<const f4 *>(a.w + (size_t)min(row0 + r, a.rows - 1) * a.cols);
#pragma unroll
        for (int u = 0; u < UNR; u++) wv[r][u] = __builtin_nontemporal_load(W + min(lane + 64 * u, C4 - 1));
    }
    if constexpr (EPI == kEpiSwiglu) {
        const f4 *W2 = reinterpret_cast<const f4 *>(a.w2 + (size_t)min(row0, a.rows - 1) * a.cols);
#pragma unroll
        for (int u = 0; u < UNR; u++) wv2[u] = __builtin_nontemporal_load(W2 + min(lane + 64 * u, C4 - 1));
    }
    float resid[EPI == kEpiResid ? R : 1];
    if constexpr (EPI == kEpiResid) {
        const float *src = a.resid ? a.resid : a.out0;
#pragma unroll
        for (int r = 0; r < R; r++) resid[r] = src[min(row0 + r, a.rows - 1)];
    }
    f4 xv[XK], gv[XK], pv[NP > 0 ? NP : 1][XK];
#pragma unroll
    for (int k = 0; k < XK; k++) {
        const int c = min(t + 256 * k, C4 - 1);
        xv[k] = reinterpret_cast<const f4 *>(a.x)[c];
        if (NORM) gv[k] = reinterpret_cast<const f4 *>(a.norm)[c];
#pragma unroll
        for (int p = 0; p < NP; p++)
            pv[p][k] = reinterpret_cast<const f4 *>(a.parts + (size_t)min(p, a.nparts - 1) * a.cols)[c];
    }
#pragma unroll
    for (int u = 0; u < UNR; u++) {
        const bool in = lane + 64 * u < C4;
#pragma unroll
        for (int r = 0; r < R; r++) wv[r][u] = in ? wv[r][u] : zero;
        if (EPI == kEpiSwiglu) wv2[u] = in ? wv2[u] : zero;
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < XK; k++) {
        const bool in = t + 256 * k < C4;
        xv[k] = in ? xv[k] : zero;
        if (NORM) gv[k] = in ? gv[k] : zero;
#pragma unroll
        for (int p = 0; p < NP; p++)
            if (p < a.nparts) xv[k] += in ? pv[p][k] : zero;
        const int c = t + 256 * k;
        sx[c] = xv[k];
        if (NORM) {
            sg[c] = gv[k];
            ss = dot4(xv[k], xv[k], ss);
        }
        if (NP > 0 && blockIdx.x == 0 && c < C4) reinterpret_cast<f4 *>(a.xout)[c] = xv[k];
    }
    if (NORM) {
        ss = wave_sum(ss);
        if (lane == 0) sss[w] = ss;
    }
    __syncthreads();
    float scale = 1.0f;
    if (NORM) {
        // rmsnorm (src/kernels.rs:343-349): xn = x * scale * g
        ss = (sss[0] + sss[1]) + (sss[2] + sss[3]);
        scale = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
    }
    if (!live) return;
    float acc[R], acc2 = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int u = 0; u < UNR; u++) {
        const int c = lane + 64 * u;
        if (c >= C4) break;
        f4 x = sx[c];
        if (NORM) x = x * scale * sg[c];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = dot4(wv[r][u], x, acc[r]);
        if (EPI == kEpiSwiglu) acc2 = dot4(wv2[u], x, acc2);
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
    if (EPI == kEpiSwiglu) acc2 = wave_sum(acc2);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = row0 + r;
            if (row >= a.rows) break;
            const float d = acc[r];
            if (EPI == kEpiStore || EPI == kEpiArgmax) {
                a.out0[row] = d;
            } else if (EPI == kEpiResid) {
                a.out0[row] = resid[r] + d;
            } else if (EPI == kEpiQkv) {
                if (row < a.split0)
                    a.out0[row] = d;
                else if (row < a.split1)
                    a.out1[row - a.split0] = d;
                else
                    a.out2[row - a.split1] = d;
            } else {  // silu_mul: g / (1 + exp(-g)) * u
                a.out0[row] = d / (1.0f + expf(-d)) * acc2;
            }
        }
        if constexpr (EPI == kEpiArgmax) {
            // the wave's rows in increasing order; argmax_kernel reduces the pairs
            static_assert(R == kArgmaxRows, "one pair per kArgmaxRows rows");
            float bv = -INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int r = 0; r < R; r++)
                if (row0 + r < a.rows) arg_better(acc[r], row0 + r, bv, bi);
            reinterpret_cast<float2 *>(a.out1)[row0 / R] = make_float2(bv, __int_as_float(bi));
        }
    }
}

// Several tokens (prompt chunks): out rows of W . X^T on the f32 matrix cores.
// A workgroup computes 16 output rows x 16*TB tokens as TB accumulators of
// v_mfma_f32_16x16x4_f32 (A = 16 weight rows x 4 k, B = 4 k x 16 tokens); the
// contraction index is permuted so each lane loads whole float4s: MFMA e of
// k-step s uses k = 16s + 4*(lane/16) + e for both operands.  Lane l then holds
// rows row0 + 4*(l/16) + r of token tok0 + 16b + l%16.  The input rows are
// already normalised (rmsnorm_kernel); the epilogues are gemv_kernel's.
__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

template <int EPI, int TB>
__global__ __launch_bounds__(256) void gemm_kernel(const GemvArgs a) {
    // workgroup = one tile of 16 rows x 16*TB tokens; its 4 waves split k in
    // four contiguous ranges and their partial tiles are summed through LDS
    __shared__ f4 red[3][TB][2][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int row0 = 16 * blockIdx.x;
    const int tok0 = blockIdx.y * 16 * TB;
    const int i = lane & 15, g = lane >> 4;
    const float *wr = a.w + (size_t)min(row0 + i, a.rows - 1) * a.cols + 4 * g;
    const float *w2r = EPI == kEpiSwiglu ? a.w2 + (size_t)min(row0 + i, a.rows - 1) * a.cols + 4 * g : wr;
    const float *xr[TB];
#pragma unroll
    for (int b = 0; b < TB; b++) xr[b] = a.x + (size_t)min(tok0 + 16 * b + i, a.t - 1) * a.cols + 4 * g;
    f4 acc[TB], acc2[TB];
#pragma unroll
    for (int b = 0; b < TB; b++) acc[b] = acc2[b] = f4{0.f, 0.f, 0.f, 0.f};
    auto step = [&](const f4 &wv, const f4 &w2v, const f4 (&xv)[TB]) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
#pragma unroll
            for (int b = 0; b < TB; b++) {
                acc[b] = mfma4(wv[e], xv[b][e], acc[b]);
                if (EPI == kEpiSwiglu) acc2[b] = mfma4(w2v[e], xv[b][e], acc2[b]);
            }
        }
    };
    // this wave's k range, in 16-wide steps
    const int steps = a.cols / 16;
    const int s0 = (w * steps) >> 2, s1 = ((w + 1) * steps) >> 2;
    constexpr int KU = 4;  // steps per load batch: all of a batch's loads go out together
    for (int st = s0; st < s1; st += KU) {
        f4 wv[KU], w2v[KU], xv[KU][TB];
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int k = 16 * min(st + u, s1 - 1);
            wv[u] = *reinterpret_cast<const f4 *>(wr + k);
            w2v[u] = wv[u];
            if (EPI == kEpiSwiglu) w2v[u] = *reinterpret_cast<const f4 *>(w2r + k);
#pragma unroll
            for (int b = 0; b < TB; b++) xv[u][b] = *reinterpret_cast<const f4 *>(xr[b] + k);
        }
#pragma unroll
        for (int u = 0; u < KU; u++)
            if (st + u < s1) step(wv[u], w2v[u], xv[u]);
    }
    if (w > 0) {
#pragma unroll
        for (int b = 0; b < TB; b++) {
            red[w - 1][b][0][lane] = acc[b];
            if (EPI == kEpiSwiglu) red[w - 1][b][1][lane] = acc2[b];
        }
    }
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int b = 0; b < TB; b++) {
#pragma unroll
        for (int ww = 0; ww < 3; ww++) {
            acc[b] += red[ww][b][0][lane];
            if (EPI == kEpiSwiglu) acc2[b] += red[ww][b][1][lane];
        }
    }
#pragma unroll
    for (int b = 0; b < TB; b++) {
        const int tok = tok0 + 16 * b + i;
        if (tok >= a.t) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = row0 + 4 * g + r;
            if (row >= a.rows) continue;
            const float d = acc[b][r];
            const size_t t = (size_t)tok;
            if (EPI == kEpiStore) {
                a.out0[t * a.ld0 + row] = d;
            } else if (EPI == kEpiResid) {
                a.out0[t * a.ld0 + row] += d;
            } else if (EPI == kEpiQkv) {
                if (row < a.split0)
                    a.out0[t * a.ld0 + row] = d;
                else if (row < a.split1)
                    a.out1[t * a.ld1 + (row - a.split0)] = d;
                else
                    a.out2[t * a.ld2 + (row - a.split1)] = d;
            } else {
                a.out0[t * a.ld0 + row] = d / (1.0f + expf(-d)) * acc2[b][r];
            }
        }
    }
}

// rmsnorm (src/kernels.rs:343-349) of t rows of n floats: one workgroup per row,
// a fixed-order reduction, xn = x * scale * g.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ g,
                                                      float eps, float *__restrict__ out, int n) {
    __shared__ float red[4];
    const float *xr = x + (size_t)blockIdx.x * n;
    float ss = 0.0f;
    for (int c = threadIdx.x; c < n; c += 256) ss = fmaf(xr[c], xr[c], ss);
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    float *o = out + (size_t)blockIdx.x * n;
    for (int c = threadIdx.x; c < n; c += 256) o[c] = xr[c] * scale * g[c];
}

// step (graph-replayed decode loop): the token is tokens[*step + i].
__global__ __launch_bounds__(256) void embed_kernel(const float *__restrict__ embed, const uint32_t *__restrict__ tokens,
                                                    const int *__restrict__ step, float *__restrict__ x, int hidden) {
    const int i = blockIdx.x;
    const int at = (step ? *step : 0) + i;
    const f4 *src = reinterpret_cast<const f4 *>(embed + (size_t)tokens[at] * hidden);
    f4 *dst = reinterpret_cast<f4 *>(x + (size_t)i * hidden);
    for (int c = threadIdx.x; c < hidden / 4; c += blockDim.x) dst[c] = src[c];
}

// sampler::argmax (src/sampler.rs:129-137): best = 0; for i: if x[i] > x[best]
// { best = i }.  That is the first index of the maximum over the non-NaN
// values (NaN never compares greater), except that a NaN at index 0 is never
// replaced.  One workgroup; each thread issues 8 float4 loads per pass before
// comparing.  Ties resolve to the smaller index.  With parts (the LM head's
// kEpiArgmax pairs, one per kArgmaxRows rows) the workgroup reduces those
// instead: a quarter of the values, each 2 floats, and every pair's index the
// smallest among its rows' maxima, so the result is the same.

// step, len (graph-replayed decode loop): the id goes to out[*step + 1], then
// *step and *len advance to the next forward's token and cache length.
// embed (greedy decode loop): the workgroup also copies the chosen id's
// embedding row (hidden floats) to xe, the next forward's input row, in place
// of that forward's embed_kernel launch.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ x, int n, uint32_t *__restrict__ out,
                                                      int *__restrict__ step, int *__restrict__ len,
                                                      const float *__restrict__ parts, const float *__restrict__ embed,
                                                      float *__restrict__ xe, int hidden) {
    constexpr int U = 8;
    __shared__ float sv[16];
    __shared__ int si[16];
    __shared__ int sbest;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    // x[0] (wick keeps index 0 when it is NaN) is requested with the rest
    const float x0 = threadIdx.x == 0 ? x[0] : 0.f;
    if (parts) {
        // two pairs per float4
        const int np = argmax_parts(n), np2 = np >> 1;
        const f4 *p4 = reinterpret_cast<const f4 *>(parts);
        for (int base = threadIdx.x; base < np2; base += U * 1024) {
            f4 v[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int c = base + 1024 * u;
                if (c < np2) v[u] = p4[c];
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int c = base + 1024 * u;
                if (c < np2) {
                    arg_better(v[u].x, __float_as_int(v[u].y), bv, bi);
                    arg_better(v[u].z, __float_as_int(v[u].w), bv, bi);
                }
            }
        }
        if ((np & 1) && threadIdx.x == 0) arg_better(parts[2 * np - 2], __float_as_int(parts[2 * np - 1]), bv, bi);
    } else {
        const int n4 = n >> 2;
        const f4 *x4 = reinterpret_cast<const f4 *>(x);
        for (int base = threadIdx.x; base < n4; base += U * 1024) {
            f4 v[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int c = base + 1024 * u;
                v[u] = c < n4 ? x4[c] : f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int c = base + 1024 * u;
                if (c < n4) {
                    arg_better(v[u].x, 4 * c, bv, bi);
                    arg_better(v[u].y, 4 * c + 1, bv, bi);
                    arg_better(v[u].z, 4 * c + 2, bv, bi);
                    arg_better(v[u].w, 4 * c + 3, bv, bi);
                }
            }
        }
        for (int i = 4 * n4 + threadIdx.x; i < n; i += 1024) arg_better(x[i], i, bv, bi);
    }
    // the wave's best pair on lane moves (no lane holds a NaN as its best, so
    // "better of two" is commutative and every lane ends with the wave's best)
    arg_better(dpp_f<kDppQuadXor1>(bv), dpp_i<kDppQuadXor1>(bi), bv, bi);
    arg_better(dpp_f<kDppQuadXor2>(bv), dpp_i<kDppQuadXor2>(bi), bv, bi);
    arg_better(dpp_f<kDppRowHalfMirror>(bv), dpp_i<kDppRowHalfMirror>(bi), bv, bi);
    arg_better(dpp_f<kDppRowMirror>(bv), dpp_i<kDppRowMirror>(bi), bv, bi);
    {
        const auto pv = __builtin_amdgcn_permlane16_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
        const auto pi = __builtin_amdgcn_permlane16_swap((unsigned)bi, (unsigned)bi, false, false);
        arg_better(__uint_as_float(pv[0]), (int)pi[0], bv, bi);
        arg_better(__uint_as_float(pv[1]), (int)pi[1], bv, bi);
    }
    {
        const auto pv = __builtin_amdgcn_permlane32_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
        const auto pi = __builtin_amdgcn_permlane32_swap((unsigned)bi, (unsigned)bi, false, false);
        arg_better(__uint_as_float(pv[0]), (int)pi[0], bv, bi);
        arg_better(__uint_as_float(pv[1]), (int)pi[1], bv, bi);
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = bv;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 16; k++) arg_better(sv[k], si[k], bv, bi);
        // all values NaN (bi unset) or x[0] NaN: wick keeps index 0
        if (bi == 0x7fffffff || isnan(x0)) bi = 0;
        if (step) {
            const int k = *step;
            out[k + 1] = (uint32_t)bi;
            *step = k + 1;
            *len += 1;
        } else {
            *out = (uint32_t)bi;
        }
        sbest = bi;
    }
    if (embed) {
        __syncthreads();
        const f4 *src = reinterpret_cast<const f4 *>(embed + (size_t)sbest * hidden);
        f4 *dst = reinterpret_cast<f4 *>(xe);
        for (int c = threadIdx.x; c < hidden / 4; c += blockDim.x) dst[c] = src[c];
    }
}

// ------------------------------------------------------------------ launchers

namespace {

template <int NT, int R, int UNR, int EPI>
hipError_t gemv_launch(const GemvArgs &a, hipStream_t s) {
    const int waves = (a.rows + R - 1) / R;
    const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)((a.t + NT - 1) / NT)), block(256);
    if (a.norm)
        hipLaunchKernelGGL((gemv_kernel<NT, R, UNR, EPI, true>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((gemv_kernel<NT, R, UNR, EPI, false>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <int R, int UNR, int EPI>
hipError_t gemv1_launch_unr(const GemvArgs &a, hipStream_t s) {
    const int waves = (a.rows + R - 1) / R;
    const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
    if (a.parts)
        hipLaunchKernelGGL((gemv1_kernel<R, UNR, EPI, true, kMaxParts>), grid, block, 0, s, a);
    else if (a.norm)
        hipLaunchKernelGGL((gemv1_kernel<R, UNR, EPI, true, 0>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((gemv1_kernel<R, UNR, EPI, false, 0>), grid, block, 0, s, a);
    return hipGetLastError();
}

// The unroll that covers the row (64 lanes x UNR float4s) with the fewest
// spare slots: every slot is a load (clamped in bounds), so spare ones cost
// load instructions (576 floats: 3; 1536: 6).
template <int R, int EPI>
hipError_t gemv1_launch(const GemvArgs &a, hipStream_t s) {
    const int need = ((a.cols >> 2) + 63) / 64;
    if (need <= 2) return gemv1_launch_unr<R, 2, EPI>(a, s);
    if (need <= 3) return gemv1_launch_unr<R, 3, EPI>(a, s);
    if (need <= 4) return gemv1_launch_unr<R, 4, EPI>(a, s);
    if (need <= 6) return gemv1_launch_unr<R, 6, EPI>(a, s);
    if (need <= 8) return gemv1_launch_unr<R, 8, EPI>(a, s);
    return hipErrorInvalidValue;
}

// One token: one row per wave (the LM head, kEpiStore / kEpiArgmax, 4 rows per
// wave to keep more of its 100+ MB in flight per wave), the input row through
// LDS when it fits one pass (64 * 8 float4s), else gemv_kernel.  Several
// tokens: 4 per wave, 4 float4s per lane per pass.
template <int EPI>
hipError_t gemv_epi(const GemvArgs &a, hipStream_t s) {
    const bool one_pass = a.cols <= 4 * 64 * 8;
    if constexpr (EPI == kEpiArgmax) {
        if (a.t != 1 || !a.out1) return hipErrorInvalidValue;
        if (a.cols <= 4 * 64 * 4) return gemv1_launch<kArgmaxRows, EPI>(a, s);
        return gemv_launch<1, kArgmaxRows, 4, EPI>(a, s);
    } else {
        if (a.t > 1) return gemv_launch<4, 1, 4, EPI>(a, s);
        if constexpr (EPI == kEpiStore) {
            if (a.cols <= 4 * 64 * 4) return gemv1_launch<4, EPI>(a, s);
            return gemv_launch<1, 4, 4, EPI>(a, s);
        }
        if (one_pass) return gemv1_launch<1, EPI>(a, s);
        return gemv_launch<1, 1, 8, EPI>(a, s);
    }
}

}  // namespace

hipError_t launch_gemv(int epi, const GemvArgs &a, hipStream_t s) {
    if (a.rows <= 0 || a.t <= 0) return hipSuccess;
    if (a.parts) {
        // the gate/up product after the fused decode + output projection
        if (epi != kEpiSwiglu || a.t != 1 || !a.norm || !a.xout || a.nparts < 1 || a.nparts > kMaxParts ||
            a.cols > 4 * 64 * 8)
            return hipErrorInvalidValue;
        return gemv1_launch<1, kEpiSwiglu>(a, s);
    }
    switch (epi) {
    case kEpiStore: return gemv_epi<kEpiStore>(a, s);
    case kEpiResid: return gemv_epi<kEpiResid>(a, s);
    case kEpiQkv: return gemv_epi<kEpiQkv>(a, s);
    case kEpiSwiglu: return gemv_epi<kEpiSwiglu>(a, s);
    case kEpiArgmax: return gemv_epi<kEpiArgmax>(a, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(int epi, const GemvArgs &a, hipStream_t s) {
    if (a.rows <= 0 || a.t <= 0) return hipSuccess;
    if (a.cols % 16 != 0 || a.norm) return hipErrorInvalidValue;
    constexpr int TB = 2;  // 32 tokens per workgroup tile
    const dim3 grid((unsigned)((a.rows + 15) / 16), (unsigned)((a.t + 16 * TB - 1) / (16 * TB))), block(256);
    switch (epi) {
    case kEpiStore: hipLaunchKernelGGL((gemm_kernel<kEpiStore, TB>), grid, block, 0, s, a); break;
    case kEpiResid: hipLaunchKernelGGL((gemm_kernel<kEpiResid, TB>), grid, block, 0, s, a); break;
    case kEpiQkv: hipLaunchKernelGGL((gemm_kernel<kEpiQkv, TB>), grid, block, 0, s, a); break;
    case kEpiSwiglu: hipLaunchKernelGGL((gemm_kernel<kEpiSwiglu, TB>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, const float *g, float eps, float *out, int t, int n, hipStream_t s) {
    if (t <= 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)t), dim3(256), 0, s, x, g, eps, out, n);
    return hipGetLastError();
}

hipError_t launch_embed(const float *embed, const uint32_t *tokens, float *x, int t, int hidden, hipStream_t s,
                        const int *step) {
    if (t <= 0) return hipSuccess;
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)t), dim3(256), 0, s, embed, tokens, step, x, hidden);
    return hipGetLastError();
}

__global__ void set_step_kernel(int *counters, int step, int len) {
    counters[0] = step;
    counters[1] = len;
}

hipError_t launch_set_step(int *counters, int step, int len, hipStream_t s) {
    hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(1), 0, s, counters, step, len);
    return hipGetLastError();
}

hipError_t launch_argmax(const float *x, int n, uint32_t *out, hipStream_t s, int *step, int *len, const float *parts,
                         const float *embed, float *xe, int hidden) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, x, n, out, step, len, parts, embed, xe, hidden);
    return hipGetLastError();
}

}  // namespace wick
