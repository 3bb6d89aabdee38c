// roofline_probe.hip -- measurement kernels for bench.py, not part of the
// attention path (built into libwick_probe.so, which nothing else loads).
//
// They give the practical ceilings a decode call is judged against on the
// same box and in the same run:
//   - read ceiling: one launch that only reads a buffer of the decode layer's
//     size (no compute, no stores), either each workgroup streaming one
//     contiguous slice -- the decode kernel's access pattern, a chunk of keys
//     per workgroup -- or all workgroups striding through the buffer together,
//     through plain or nontemporal (streaming cache policy) loads;
//   - launch floor: launch to launch of an empty kernel on a given grid.
#include <hip/hip_runtime.h>
#include <stddef.h>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kInFlight = 4;  // float4 loads per thread per iteration

// The sum is stored only if it equals a value no sum of the probe's inputs
// (ones) takes, so the loads cannot be dropped and nothing is written.
__device__ __forceinline__ void keep(f4 acc, float *sink) {
    const float s = (acc.x + acc.y) + (acc.z + acc.w);
    if (s == -1.0f) sink[blockIdx.x] = s;
}

template <bool NT>
__device__ __forceinline__ f4 ld(const f4 *p) {
    if constexpr (NT)
        return __builtin_nontemporal_load(p);
    else
        return *p;
}

template <bool NT>
__global__ __launch_bounds__(kThreads) void read_slices(const f4 *__restrict__ p, size_t n4, size_t per_wg,
                                                        float *sink) {
    const size_t beg = (size_t)blockIdx.x * per_wg;
    const size_t end = beg + per_wg < n4 ? beg + per_wg : n4;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    size_t i = beg + threadIdx.x;
    for (; i + (kInFlight - 1) * kThreads < end; i += kInFlight * kThreads) {
        f4 x[kInFlight];
#pragma unroll
        for (int u = 0; u < kInFlight; u++) x[u] = ld<NT>(p + i + u * kThreads);
#pragma unroll
        for (int u = 0; u < kInFlight; u++) acc += x[u];
    }
    for (; i < end; i += kThreads) acc += ld<NT>(p + i);
    keep(acc, sink);
}

template <bool NT>
__global__ __launch_bounds__(kThreads) void read_strided(const f4 *__restrict__ p, size_t n4, float *sink) {
    const size_t stride = (size_t)gridDim.x * kThreads;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i + (kInFlight - 1) * stride < n4; i += kInFlight * stride) {
        f4 x[kInFlight];
#pragma unroll
        for (int u = 0; u < kInFlight; u++) x[u] = ld<NT>(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < kInFlight; u++) acc += x[u];
    }
    for (; i < n4; i += stride) acc += ld<NT>(p + i);
    keep(acc, sink);
}

__global__ __launch_bounds__(kThreads) void empty_kernel() {}

}  // namespace

extern "C" {

// Read `bytes` (a multiple of 16) at buf on `grid` workgroups; `mode` bit 0
// picks the strided access pattern, bit 1 nontemporal loads.  sink: device
// array of at least `grid` floats (never written for a buffer of ones).
// Asynchronous on `stream`.  0 or a HIP error.
int wick_probe_read(const void *buf, size_t bytes, int grid, int mode, float *sink, void *stream) {
    if (!buf || !sink || grid < 1 || bytes % 16 != 0 || mode < 0 || mode > 3) return (int)hipErrorInvalidValue;
    const size_t n4 = bytes / 16;
    const hipStream_t s = (hipStream_t)stream;
    const f4 *p = (const f4 *)buf;
    const size_t per_wg = (n4 + grid - 1) / grid;
    switch (mode) {
    case 0: hipLaunchKernelGGL(read_slices<false>, dim3(grid), dim3(kThreads), 0, s, p, n4, per_wg, sink); break;
    case 1: hipLaunchKernelGGL(read_strided<false>, dim3(grid), dim3(kThreads), 0, s, p, n4, sink); break;
    case 2: hipLaunchKernelGGL(read_slices<true>, dim3(grid), dim3(kThreads), 0, s, p, n4, per_wg, sink); break;
    default: hipLaunchKernelGGL(read_strided<true>, dim3(grid), dim3(kThreads), 0, s, p, n4, sink); break;
    }
    return (int)hipGetLastError();
}

// An empty kernel on `grid` workgroups of 256 threads.
int wick_probe_empty(int grid, void *stream) {
    if (grid < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream);
    return (int)hipGetLastError();
}

}  // extern "C"
