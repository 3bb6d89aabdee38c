// synth.hip -- synthetic inputs for bench.py (not part of the attention path;
// built into libwick_probe.so beside the roofline probes, which nothing in the
// product loads).
//
// Values are N(0, 1) times a scale, drawn from wick's generator: xoshiro256**
// seeded through splitmix64 (Rng::new and Rng::next_u64,
// /root/reference/src/sampler.rs:33-55), made normal by Box-Muller in double:
// for each pair of draws a, b
//     u1 = ((a >> 11) + 1) / 2^53   in (0, 1]
//     u2 = (b >> 11) / 2^53         in [0, 1)
//     x0 = sqrt(-2 ln u1) cos(2 pi u2),  x1 = sqrt(-2 ln u1) sin(2 pi u2),
// each multiplied by the scale and rounded once to f32, x0 first.
// One benchmark configuration uses one seed.  Rows are generated in parallel,
// each from its own substream of Rng::new(seed): row j of tensor t starts from
// that state advanced by t long jumps (2^192 draws each) and j jumps (2^128
// draws each) -- the jump polynomials xoshiro256**'s authors publish for
// cutting one stream into non-overlapping parallel ones.  A row's values are
// its substream's pairs in order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

namespace {

constexpr uint64_t kJump[4] = {0x180ec6d33cfd0abaULL, 0xd5a61266f0c9392cULL, 0xa9582618e03fc9aaULL,
                               0x39abdc4529b1661cULL};
constexpr uint64_t kLongJump[4] = {0x76e15d3efefdcbbfULL, 0xc5004e441c522fb3ULL, 0x77710069854ee241ULL,
                                   0x39109bb02acbe635ULL};

__host__ __device__ inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

__host__ __device__ inline uint64_t next_u64(uint64_t s[4]) {
    const uint64_t out = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return out;
}

void seed_state(uint64_t seed, uint64_t s[4]) {
    uint64_t z = seed;
    for (int i = 0; i < 4; i++) {
        z += 0x9E3779B97F4A7C15ULL;
        uint64_t x = z;
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
        s[i] = x ^ (x >> 31);
    }
}

// s advanced by the draws the polynomial stands for (2^128 or 2^192)
void jump(uint64_t s[4], const uint64_t (&poly)[4]) {
    uint64_t a[4] = {0, 0, 0, 0};
    for (int w = 0; w < 4; w++)
        for (int b = 0; b < 64; b++) {
            if (poly[w] & (1ULL << b))
                for (int i = 0; i < 4; i++) a[i] ^= s[i];
            next_u64(s);
        }
    for (int i = 0; i < 4; i++) s[i] = a[i];
}

__global__ __launch_bounds__(256) void normal_rows_kernel(const uint64_t *__restrict__ states, long long rows,
                                                          int row_len, float scale, float *__restrict__ out) {
    const long long r = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    uint64_t s[4] = {states[4 * r], states[4 * r + 1], states[4 * r + 2], states[4 * r + 3]};
    float *o = out + r * (long long)row_len;
    constexpr double kInv53 = 1.0 / 9007199254740992.0;  // 2^-53
    constexpr double kTwoPi = 6.283185307179586;
    for (int i = 0; i < row_len; i += 2) {
        const uint64_t a = next_u64(s), b = next_u64(s);
        const double u1 = (double)((a >> 11) + 1) * kInv53, u2 = (double)(b >> 11) * kInv53;
        const double rad = sqrt(-2.0 * log(u1)), th = kTwoPi * u2;
        o[i] = (float)(rad * cos(th) * (double)scale);
        o[i + 1] = (float)(rad * sin(th) * (double)scale);
    }
}

}  // namespace

extern "C" {

// out[rows][row_len] (device, row_len even) = tensor `tensor` of the
// configuration seeded with `seed`, times `scale`.  Synchronous on `stream`
// (the per-row generator states are computed on the host, staged through a
// device buffer freed before return).  0 or a HIP error code.
int wick_synth_normal(float *out, int tensor, long long rows, int row_len, unsigned long long seed, float scale,
                      void *stream) {
    if (!out || tensor < 0 || rows < 1 || row_len < 2 || row_len % 2) return (int)hipErrorInvalidValue;
    const hipStream_t st = (hipStream_t)stream;
    uint64_t s[4];
    seed_state(seed, s);
    for (int t = 0; t < tensor; t++) jump(s, kLongJump);
    std::vector<uint64_t> states((size_t)rows * 4);
    for (long long r = 0; r < rows; r++) {
        for (int i = 0; i < 4; i++) states[(size_t)r * 4 + i] = s[i];
        jump(s, kJump);
    }
    uint64_t *dev = nullptr;
    hipError_t e = hipMalloc(&dev, states.size() * sizeof(uint64_t));
    if (e != hipSuccess) return (int)e;
    e = hipMemcpyAsync(dev, states.data(), states.size() * sizeof(uint64_t), hipMemcpyHostToDevice, st);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(normal_rows_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, dev, rows,
                           row_len, scale, out);
        e = hipGetLastError();
    }
    const hipError_t es = hipStreamSynchronize(st);
    if (e == hipSuccess) e = es;
    const hipError_t ef = hipFree(dev);
    if (e == hipSuccess) e = ef;
    return (int)e;
}

}  // extern "C"
