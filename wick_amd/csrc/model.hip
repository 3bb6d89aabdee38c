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

namespace wick {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float dot4(const f4 w, const f4 x, float acc) {
    acc = fmaf(w.x, x.x, acc);
    acc = fmaf(w.y, x.y, acc);
    acc = fmaf(w.z, x.z, acc);
    return fmaf(w.w, x.w, acc);
}

}  // namespace

// One wave per output row `row`, NT tokens per wave (token group blockIdx.y).
// Column c4 (a float4 index) of a row is handled by lane c4 % 64.
template <int NT, int EPI, bool NORM>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvArgs a) {
    constexpr int UNR = 4;  // float4 loads per lane in flight per operand
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;  // whole waves only; no barriers below
    const int tok0 = blockIdx.y * NT;
    const int nt = min(NT, a.t - tok0);
    const int C4 = a.cols >> 2;
    const f4 *X[NT];
#pragma unroll
    for (int tk = 0; tk < NT; tk++) X[tk] = reinterpret_cast<const f4 *>(a.x + (size_t)(tok0 + min(tk, nt - 1)) * a.cols);

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

    const f4 *W = reinterpret_cast<const f4 *>(a.w + (size_t)row * a.cols);
    const f4 *W2 = EPI == kEpiSwiglu ? reinterpret_cast<const f4 *>(a.w2 + (size_t)row * a.cols) : W;
    const f4 *G = reinterpret_cast<const f4 *>(a.norm);
    float acc[NT], acc2[NT];
#pragma unroll
    for (int tk = 0; tk < NT; tk++) acc[tk] = acc2[tk] = 0.0f;

    for (int base = lane; base < C4; base += 64 * UNR) {
        f4 wv[UNR], wv2[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int c = base + 64 * u;
            const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
            wv[u] = c < C4 ? __builtin_nontemporal_load(W + c) : zero;
            if (EPI == kEpiSwiglu) wv2[u] = c < C4 ? __builtin_nontemporal_load(W2 + c) : zero;
        }
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int c = base + 64 * u;
            if (c < C4) {
                f4 g = {1.0f, 1.0f, 1.0f, 1.0f};
                if (NORM) g = G[c];
#pragma unroll
                for (int tk = 0; tk < NT; tk++) {
                    f4 xv = X[tk][c];
                    if (NORM) xv = xv * scale[tk] * g;
                    acc[tk] = dot4(wv[u], xv, acc[tk]);
                    if (EPI == kEpiSwiglu) acc2[tk] = dot4(wv2[u], xv, acc2[tk]);
                }
            }
        }
    }
#pragma unroll
    for (int tk = 0; tk < NT; tk++) {
        acc[tk] = wave_sum(acc[tk]);
        if (EPI == kEpiSwiglu) acc2[tk] = wave_sum(acc2[tk]);
    }
    // lane tk writes token tk's value
#pragma unroll
    for (int tk = 0; tk < NT; tk++) {
        if (lane != tk || tk >= nt) continue;
        const size_t tok = (size_t)tok0 + tk;
        const float d = acc[tk];
        if (EPI == kEpiStore) {
            a.out0[tok * a.ld0 + row] = d;
        } else if (EPI == kEpiResid) {
            a.out0[tok * a.ld0 + row] += d;
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

__global__ __launch_bounds__(256) void embed_kernel(const float *__restrict__ embed, const uint32_t *__restrict__ tokens,
                                                    float *__restrict__ x, int hidden) {
    const int i = blockIdx.x;
    const f4 *src = reinterpret_cast<const f4 *>(embed + (size_t)tokens[i] * hidden);
    f4 *dst = reinterpret_cast<f4 *>(x + (size_t)i * hidden);
    for (int c = threadIdx.x; c < hidden / 4; c += blockDim.x) dst[c] = src[c];
}

// sampler::argmax (src/sampler.rs:129-137): best = 0; for i: if x[i] > x[best]
// { best = i }.  That is the first index of the maximum over the non-NaN
// values (NaN never compares greater), except that a NaN at index 0 is never
// replaced.  One workgroup; ties resolve to the smaller index.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ x, int n, uint32_t *__restrict__ out) {
    __shared__ float sv[16];
    __shared__ int si[16];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = x[i];
        if (v > bv || (v == bv && i < bi)) {
            bv = v;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = bv;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < (int)(blockDim.x >> 6); k++)
            if (sv[k] > bv || (sv[k] == bv && si[k] < bi)) {
                bv = sv[k];
                bi = si[k];
            }
        // all values NaN (bi unset) or x[0] NaN: wick keeps index 0
        if (bi == 0x7fffffff || isnan(x[0])) bi = 0;
        *out = (uint32_t)bi;
    }
}

// ------------------------------------------------------------------ launchers

namespace {

template <int NT, int EPI>
hipError_t gemv_nt(const GemvArgs &a, hipStream_t s) {
    const dim3 grid((unsigned)((a.rows + 3) / 4), (unsigned)((a.t + NT - 1) / NT)), block(256);
    if (a.norm)
        hipLaunchKernelGGL((gemv_kernel<NT, EPI, true>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((gemv_kernel<NT, EPI, false>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <int EPI>
hipError_t gemv_epi(const GemvArgs &a, hipStream_t s) {
    return a.t == 1 ? gemv_nt<1, EPI>(a, s) : gemv_nt<4, EPI>(a, s);
}

}  // namespace

hipError_t launch_gemv(int epi, const GemvArgs &a, hipStream_t s) {
    if (a.rows <= 0 || a.t <= 0) return hipSuccess;
    switch (epi) {
    case kEpiStore: return gemv_epi<kEpiStore>(a, s);
    case kEpiResid: return gemv_epi<kEpiResid>(a, s);
    case kEpiQkv: return gemv_epi<kEpiQkv>(a, s);
    case kEpiSwiglu: return gemv_epi<kEpiSwiglu>(a, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_embed(const float *embed, const uint32_t *tokens, float *x, int t, int hidden, hipStream_t s) {
    if (t <= 0) return hipSuccess;
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)t), dim3(256), 0, s, embed, tokens, x, hidden);
    return hipGetLastError();
}

hipError_t launch_argmax(const float *x, int n, uint32_t *out, hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, x, n, out);
    return hipGetLastError();
}

}  // namespace wick
