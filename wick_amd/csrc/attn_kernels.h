// Internal interface between the C ABI (api.cpp) and the HIP kernels
// (attention.hip).  Not installed; the public boundary is include/wick_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "wick_hip.h"

namespace wick {

// Most split-K chunks one decode call uses per (kv head, 16-head slice).
constexpr int kDecodeMaxChunks = 256;
// Longest context the automatic decode schedule serves with one chunk per unit
// (config 2 at 512 positions: 10.1 us as one 8-wave chunk per kv head against
// 7.0 us split over 16 workgroups plus the merge).
constexpr int kDecodeSingleChunkMax = 192;
constexpr int kTileRows = 16;  // query rows (or heads) per MFMA column block

struct DecodeArgs {
    const float *q;   // [heads*D] (one token); raw projections when prep != 0
    float *k;         // layer base, [kv_heads][capacity][D]
    float *v;
    float *att;       // [heads*D]
    float *part;      // partial states, see decode_workspace_floats
    int capacity, len, kv_heads, group, hslices, chunk, nchunks;
    // a grid of at least two workgroups per CU, streaming from HBM: each wave
    // requests its first group's V rows only once its K rows have arrived
    int stagger;
    // Key order of a split: 0 = chunk c takes positions c*chunk .. +chunk;
    // 1 (only where decode_interleaves holds) = wave w of chunk c takes the
    // key groups (i*nchunks + c)*waves + w of the whole context, i = 0, 1, ...
    // (the full rounds i rotated per unit).
    int interleave;
    float scale;
    // Fused input preparation (prep != 0): q is raw; kraw / vraw [kv_heads*D]
    // are the new token's raw k and v, prepared and appended at position len-1
    // by the workgroups of the chunk that holds it.  Biases / norms may be null.
    int prep;
    const float *kraw, *vraw;
    const float *bq, *bk, *bv, *qn, *kn;
    const float *rope_cos, *rope_sin;  // [capacity][D/2] tables
    float eps;
    // When non-null the kernels read the cache length here instead of len (a
    // HIP graph replays one decode step for successive lengths); chunk and
    // nchunks must then suit every length it takes: plan_decode's plan for it.
    const int *len_dev;
    // Fused output projection (launch_decode_oproj; one chunk per unit): the
    // grid is units x row blocks of 8 * kOprojRows rows; workgroup (unit, b)
    // multiplies the unit's attention output by its rows of wo ([hidden]
    // [wo_ld], wick's o_proj layout) restricted to the unit's columns, and
    // writes that partial product to oparts[unit][row].  att is not written.
    const float *wo;
    float *oparts;
    int hidden, wo_ld;
};

// Fused output projection: rows per wave, and the most 64-column chunks of a
// unit's output (ncols * head_dim <= 64 * kOprojChunks).
constexpr int kOprojRows = 1;
constexpr int kOprojChunks = 4;
// Longest chunk the fused form takes (8 waves x one 32-key group each).
constexpr int kOprojMaxChunk = 8 * 2 * 16;

// Fewest rounds of key groups per wave (chunk / (4 waves x keys per group))
// for the interleaved split order.
constexpr int kDecodeInterleaveRounds = 4;

struct PrefillArgs {
    const float *q;   // [t][heads*D]
    const float *k;   // layer base, [kv_heads][capacity][D]
    const float *v;
    float *att;       // [t][heads*D]
    int capacity, t, start, kv_heads, group, nblocks;
    int zigzag;       // the grid is resident at once; pair heavy and light blocks
    int rows32;       // lean kernels: two 16-row blocks per workgroup
    float scale;
};

struct AppendArgs {
    const float *ksrc, *vsrc;  // [t][kv_heads*D]
    float *k, *v;              // layer base, [kv_heads][capacity][D]
    int capacity, start, t, kv_heads;
};

struct PrepArgs {
    float *q;                        // [t][heads*D], rewritten in place
    const float *ksrc, *vsrc;        // [t][kv_heads*D]
    float *k, *v;                    // layer base, [kv_heads][capacity][D]
    const float *bq, *bk, *bv;       // [heads*D], [kv_heads*D], [kv_heads*D] or null (no bias)
    const float *qn, *kn;            // [D] or null (no QK-norm)
    const float *rope_cos, *rope_sin;  // [capacity][D/2]
    int capacity, start, t, heads, kv_heads;
    float eps;
};

// Floats of decode workspace needed for `units` (kv head, head slice) pairs.
size_t decode_workspace_floats(int units, int head_dim);

// The static decode workspace of wick_hip_attention_device_noalloc: a
// file-scope __device__ array of this many floats (32 MiB) on every device.
constexpr size_t kStaticScratchFloats = size_t(8) << 20;
// Resolve the array's address on `device`, which must be current; once per
// device (later calls return the first result).
hipError_t static_scratch_init(int device);
// The address static_scratch_init found on `device`, or null.
float *static_scratch(int device);

// Decode workgroups one CU holds at once (from the kernel's register and LDS use).
int decode_blocks_per_cu(int head_dim);
// The same for the split prefill kernel.
int prefill_blocks_per_cu(int head_dim, int rows32);
// Whether the prefill kernel for this shape can take two row blocks per workgroup.
bool prefill_has_rows32(int head_dim, int capacity);

// Launches decode_kernel and, when it splits the keys, decode_merge_kernel.
hipError_t launch_decode(int head_dim, const DecodeArgs &a, int grid, hipStream_t s);
// Whether decode_kernel's fused output projection serves this plan (head_dim
// 64 or 128, one chunk of at most kOprojMaxChunk keys per unit, the unit's
// columns fit kOprojChunks).
bool decode_oproj_supported(int head_dim, int group, int nchunks, int chunk);
// Whether a split plan takes the interleaved key order (DecodeArgs::interleave).
bool decode_interleaves(int head_dim, int group, int nchunks, int chunk);
// The fused decode + partial output projection (a.prep set, a.nchunks == 1):
// units x ceil(hidden / (8 kOprojRows)) workgroups of 8 waves.
hipError_t launch_decode_oproj(int head_dim, DecodeArgs a, hipStream_t s);
int prefill_grid(int head_dim, const PrefillArgs &a);
hipError_t launch_prefill(int head_dim, const PrefillArgs &a, hipStream_t s);
hipError_t launch_append(int head_dim, const AppendArgs &a, hipStream_t s);
// prep.hip: bias, QK-norm, RoPE of q and k; k and v appended to the cache.
hipError_t launch_prep(int head_dim, const PrepArgs &a, hipStream_t s);

// Shape and stream of a cache handle (api.cpp), for the device-resident forward.
struct KvInfo {
    int layers, capacity, kv_heads, head_dim;
    hipStream_t stream;
};
bool kv_info(const wick_hip_kv *kv, KvInfo *out);

// src/model.rs:464-485 for one layer on device arrays, as wick_hip_attend_device
// except that q_dev is scratch (its contents afterwards are unspecified): for
// one token the preparation runs in the decode kernel's prologue.
// len_dev (t = 1 only): the decode kernels read the cache length there (a
// captured step replayed for successive positions); start still chooses the
// launch plan, which decode_plan_key identifies.
int attend_model(wick_hip_kv *kv, int layer, int heads, float *q_dev, const float *k_dev, const float *v_dev, int t,
                 int start, float *att_dev, const int *len_dev = nullptr);

// attend_model for one token with the output projection fused in: oparts
// [units][hidden] receives each (kv head, 16-head slice) unit's partial
// product wo[:, unit's columns] . att[unit's columns]; their sum in unit order
// is wo . att.  Returns WICK_HIP_OK, or 1 (nothing launched) when the fused
// form does not serve this shape -- the caller then uses attend_model and a
// separate product.  *units_out: the number of partial vectors.
int attend_model_oproj(wick_hip_kv *kv, int layer, int heads, float *q_dev, const float *k_dev, const float *v_dev,
                       int start, const float *wo, int hidden, float *oparts, int *units_out,
                       const int *len_dev = nullptr);

// The decode launch plan (chunk size and count) for `heads` query heads over
// len cached positions: equal keys launch the same kernels on the same grids.
long long decode_plan_key(const wick_hip_kv *kv, int heads, int len);

// Record the message wick_hip_last_error() returns on this thread; returns code.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace wick
