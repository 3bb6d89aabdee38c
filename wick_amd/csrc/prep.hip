// prep.hip -- the per-token input preparation of wick's Model::forward on the
// device: bias add, per-head RMSNorm of q and k (QK-norm), rotate-half RoPE of
// q and k, and the append of k and v to the device KV cache
// (/root/reference/src/model.rs:464-484).
//
// The output is bit-identical to wick's CPU arithmetic, so the cache the
// attention kernels read holds exactly the bits the CPU path would hold:
//   - one thread owns one (token, head) row of D floats and runs the CPU's
//     operations in the CPU's order: the sum of squares of rmsnorm_inplace
//     (/root/reference/src/kernels.rs:351-357) is a sequential f32 sum that
//     starts at -0.0 (Rust's f32 Sum);
//   - floating-point contraction is off, so a*c - b*s stays two roundings of
//     products and one of the difference, as in rope
//     (/root/reference/src/model.rs:404-414);
//   - the (sin, cos) pairs come from a table the host fills with the C
//     library's sinf / cosf of the f32 angle pos * inv_freq[i] -- the calls
//     f32::sin_cos makes on the CPU -- instead of device transcendentals;
//   - 1/sqrt uses IEEE division and square root (hipcc's default
//     correctly-rounded f32 divide and sqrt).
#include <hip/hip_runtime.h>

#include "attn_kernels.h"

namespace wick {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

template <int D>
__device__ __forceinline__ void load_row(const float *__restrict__ p, float (&x)[D]) {
#pragma unroll
    for (int j = 0; j < D; j += 4) {
        const f4 v = *reinterpret_cast<const f4 *>(p + j);
        x[j] = v.x;
        x[j + 1] = v.y;
        x[j + 2] = v.z;
        x[j + 3] = v.w;
    }
}

template <int D>
__device__ __forceinline__ void store_row(float *__restrict__ p, const float (&x)[D]) {
#pragma unroll
    for (int j = 0; j < D; j += 4) *reinterpret_cast<f4 *>(p + j) = f4{x[j], x[j + 1], x[j + 2], x[j + 3]};
}

}  // namespace

// One thread per row r of t * (heads + 2 * kv_heads): token i = r / R, slot
// s = r % R; slots [0, heads) are q heads (rewritten in place), the next
// kv_heads are k heads and the last kv_heads are v heads (written to the
// cache at position start + i).
template <int D>
__global__ __launch_bounds__(256) void prep_kernel(const PrepArgs a) {
#pragma clang fp contract(off)
    const int R = a.heads + 2 * a.kv_heads;
    const long long total = (long long)a.t * R;
    for (long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x; r < total;
         r += (long long)gridDim.x * blockDim.x) {
        const int i = (int)(r / R);
        const int s = (int)(r % R);
        const int pos = a.start + i;
        const float *src;
        float *dst;
        const float *bias = nullptr, *norm = nullptr;
        bool rope = true;
        if (s < a.heads) {
            src = dst = a.q + ((size_t)i * a.heads + s) * D;
            if (a.bq) bias = a.bq + (size_t)s * D;
            norm = a.qn;
        } else if (s < a.heads + a.kv_heads) {
            const int h = s - a.heads;
            src = a.ksrc + ((size_t)i * a.kv_heads + h) * D;
            dst = a.k + ((size_t)h * a.capacity + pos) * D;
            if (a.bk) bias = a.bk + (size_t)h * D;
            norm = a.kn;
        } else {
            const int h = s - a.heads - a.kv_heads;
            src = a.vsrc + ((size_t)i * a.kv_heads + h) * D;
            dst = a.v + ((size_t)h * a.capacity + pos) * D;
            if (a.bv) bias = a.bv + (size_t)h * D;
            rope = false;
        }
        float x[D];
        load_row<D>(src, x);
        if (bias) {  // src/model.rs:470-474
            float b[D];
            load_row<D>(bias, b);
#pragma unroll
            for (int j = 0; j < D; j++) x[j] = x[j] + b[j];
        }
        if (norm) {  // rmsnorm_inplace, src/kernels.rs:351-357
            float ss = -0.0f;
#pragma unroll
            for (int j = 0; j < D; j++) ss = ss + x[j] * x[j];
            ss = ss / (float)D;
            const float scale = 1.0f / sqrtf(ss + a.eps);
            float w[D];
            load_row<D>(norm, w);
#pragma unroll
            for (int j = 0; j < D; j++) x[j] = x[j] * scale * w[j];
        }
        if (rope) {  // rope, src/model.rs:404-414
            constexpr int H = D / 2;
            float c[H], sn[H];
            load_row<H>(a.rope_cos + (size_t)pos * H, c);
            load_row<H>(a.rope_sin + (size_t)pos * H, sn);
#pragma unroll
            for (int j = 0; j < H; j++) {
                const float u = x[j], w = x[j + H];
                x[j] = u * c[j] - w * sn[j];
                x[j + H] = w * c[j] + u * sn[j];
            }
        }
        store_row<D>(dst, x);
    }
}

hipError_t launch_prep(int head_dim, const PrepArgs &a, hipStream_t s) {
    const long long total = (long long)a.t * (a.heads + 2 * a.kv_heads);
    long long blocks = (total + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks == 0) return hipSuccess;
    const dim3 grid((unsigned)blocks), block(256);
    switch (head_dim) {
    case 16: hipLaunchKernelGGL(prep_kernel<16>, grid, block, 0, s, a); break;
    case 32: hipLaunchKernelGGL(prep_kernel<32>, grid, block, 0, s, a); break;
    case 64: hipLaunchKernelGGL(prep_kernel<64>, grid, block, 0, s, a); break;
    case 128: hipLaunchKernelGGL(prep_kernel<128>, grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace wick
