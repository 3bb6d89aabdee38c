// wave_ops.h -- whole-wave (64-lane) reductions for gfx950 on VALU lane moves.
//
// A reduction through __shfl_xor is one ds_bpermute (an LDS-pipe round trip)
// per step; here the steps within a row of 16 lanes are DPP moves folded into
// the add (quad_perm xor 1, xor 2, row_half_mirror, row_mirror) and the steps
// across rows are gfx950's v_permlane16_swap / v_permlane32_swap, which hand
// each lane the pair {v[l], v[l^16]} / {v[l], v[l^32]}.  Every step adds two
// values whose lanes then hold the same sum (addition is commutative), so all
// 64 lanes end with the same bits, in a fixed order: deterministic run to run.
#pragma once

#include <hip/hip_runtime.h>

namespace wick {

constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2, 3, 0, 1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- lane 7 - i within 8
constexpr int kDppRowMirror = 0x140;      // lane i <- lane 15 - i within 16

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}

// Sum over the 64 lanes; every lane gets the same bits.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<kDppQuadXor1>(v);
    v += dpp_f<kDppQuadXor2>(v);
    v += dpp_f<kDppRowHalfMirror>(v);
    v += dpp_f<kDppRowMirror>(v);
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Maximum over the 64 lanes (fmaxf at every step); every lane gets the same bits.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
    v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
    v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppRowMirror>(v));
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// Sum of the 4 lanes l, l^16, l^32, l^48 (the same column of every row of 16).
__device__ __forceinline__ float rows_sum(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

}  // namespace wick
