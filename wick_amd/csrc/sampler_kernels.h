// sampler_kernels.h -- the device sampler's kernel interface (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct wick_hip_sampler;

namespace wick {

constexpr int kSampleParts = 16;  // most workgroups of the split kernel
constexpr int kFastK = 64;        // top-k up to this is taken per slice, then merged
constexpr int kSliceMax = 12288;  // longest slice whose keys the split kernel holds in registers

// One draw of Sampler::sample (/root/reference/src/sampler.rs:73-127).
struct SampleArgs {
    float *logits;  // [vocab], 16-byte aligned; penalised in place
    int vocab;
    const uint32_t *history;  // [n_history]
    int n_history;
    uint32_t *flags;  // [(vocab + 31) / 32] bitset, all zero between draws
    uint64_t *rng;    // xoshiro256** state [4]
    uint32_t *out;    // the drawn id
    float temperature, top_p, min_p, penalty;
    uint32_t top_k;
    // Candidate sets larger than the in-LDS list are radix-sorted in global
    // memory: keys in key0/key1, ids in res_idx/idx1 ([vocab] each).
    uint32_t *key0, *key1, *idx1;
    uint32_t *res_idx;  // [vocab] the candidates in wick's order
    float *res_prob;    // [vocab] their probabilities after normalisation
    int *res_meta;      // {k, keep, internal check (0 = ok)}
    // The split kernel: `parts` slices of `slice` ids (a multiple of 32), each
    // leaving its argmax in part_val/part_id or its k best (key << 32 | id) in
    // part_cand[g * kFastK ..] with their count in part_count[g] (-1: too many
    // ties, the final kernel takes the whole vocabulary).
    int parts, slice;
    int split_top_k;  // slices fit kSliceMax
    float *part_val;
    uint32_t *part_id;
    unsigned long long *part_cand;
    int *part_count;
};

hipError_t launch_sample(const SampleArgs &a, hipStream_t s);

// For the model's generate loop (model_api.cpp).
int sampler_enqueue(wick_hip_sampler *s, float *logits, const uint32_t *history, int n_history, uint32_t *out);
hipStream_t sampler_stream(const wick_hip_sampler *s);
int sampler_vocab(const wick_hip_sampler *s);
bool sampler_reads_history(const wick_hip_sampler *s);

}  // namespace wick
