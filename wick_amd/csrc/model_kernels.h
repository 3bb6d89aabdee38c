// Internal interface between the device-resident forward (model_api.cpp) and
// its HIP kernels (model.hip).  Not installed; the public boundary is
// include/wick_hip_model.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wick {

// What a gemv_kernel does with the dot products of one output row.
enum GemvEpilogue {
    kEpiStore = 0,   // out0[tok][row] = dot
    kEpiResid = 1,   // out0[tok][row] += dot            (the residual adds of src/model.rs:487, :503)
    kEpiQkv = 2,     // rows split over out0 / out1 / out2 (q, k, v of src/model.rs:452-462)
    kEpiSwiglu = 3,  // out0[tok][row] = silu(dot_w) * dot_w2   (silu_mul, src/kernels.rs:373-378)
    kEpiArgmax = 4,  // kEpiStore for one token, and the first greedy step: out1 gets one
                     // (value, index) pair per kArgmaxRows rows, see launch_argmax
};

// Most partial vectors the gate/up product adds to its input row.
constexpr int kMaxParts = 4;

// Logit rows per argmax partial (the LM head's rows per wave).
constexpr int kArgmaxRows = 4;
__host__ __device__ inline int argmax_parts(int rows) { return (rows + kArgmaxRows - 1) / kArgmaxRows; }

struct GemvArgs {
    const float *x;       // input rows [t][cols]
    const float *norm;    // RMSNorm weight [cols] applied to each input row first, or null
    const float *w;       // [rows][cols] row-major (wick's layout)
    const float *w2;      // kEpiSwiglu: the up matrix [rows][cols]
    float *out0, *out1, *out2;
    int ld0, ld1, ld2;    // per-token strides (floats) of the outputs
    int split0, split1;   // kEpiQkv: rows [0,split0) -> out0, [split0,split1) -> out1, the rest -> out2
    int rows, cols, t;
    float eps;
    // kEpiSwiglu, one token, cols <= 2048: the input row is x + parts[0] + ...
    // + parts[nparts-1] (nparts <= kMaxParts partial vectors of cols floats,
    // added in that order: the fused decode's per-unit output projections);
    // the wave of row 0 also writes that sum to xout.  Null parts: x as is.
    const float *parts;
    int nparts;
    float *xout;
    // kEpiResid: the value added to, resid[tok][row] (stride ld0); null: out0 itself
    const float *resid;
};

// out rows of a matrix-vector (or small matrix-matrix) product with the
// epilogue `epi`; t tokens, cols % 4 == 0.
hipError_t launch_gemv(int epi, const GemvArgs &a, hipStream_t s);

// The same products for prompt chunks on the matrix cores: a.x holds normalised
// rows (a.norm must be null), cols % 16 == 0.
hipError_t launch_gemm(int epi, const GemvArgs &a, hipStream_t s);

// out[i][:] = rmsnorm(x[i][:], g, eps) for i < t rows of n floats.
hipError_t launch_rmsnorm(const float *x, const float *g, float eps, float *out, int t, int n, hipStream_t s);

// x[i][:] = embed[tokens[i]][:] for i < t (token ids already validated).
// step: when non-null, the token of row i is tokens[*step + i] (device counter).
hipError_t launch_embed(const float *embed, const uint32_t *tokens, float *x, int t, int hidden, hipStream_t s,
                        const int *step = nullptr);

// *out = sampler::argmax(x[0..n)) (first index of the maximum).
// step, len: when non-null, the id goes to out[*step + 1] and both counters
// advance by one (the graph-replayed decode loop).
// parts: when non-null, the argmax_parts(n) pairs the kEpiArgmax product wrote
// for x (pair p: the best of rows kArgmaxRows*p.., as value and the index's
// bits), which are reduced instead of the n logits.
// embed, xe: when non-null, embed's row for the chosen id (hidden floats,
// hidden % 4 == 0) is also copied to xe (the next forward's input row).
hipError_t launch_argmax(const float *x, int n, uint32_t *out, hipStream_t s, int *step = nullptr, int *len = nullptr,
                         const float *parts = nullptr, const float *embed = nullptr, float *xe = nullptr,
                         int hidden = 0);
// counters[0] = step, counters[1] = len: the state a replayed decode step reads (a kernel,
// not a host copy, so the values travel with the launch).
hipError_t launch_set_step(int *counters, int step, int len, hipStream_t s);

}  // namespace wick
