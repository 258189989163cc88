// Wave reductions on DPP row operations, for device code.
//
// The chain quad_perm(1,0,3,2), quad_perm(2,3,0,1), row_half_mirror and
// row_mirror leaves every lane of a 16-lane row with the row's reduction;
// row_bcast:15 (into rows 1 and 3) and row_bcast:31 (into rows 2 and 3)
// then leave the wave's reduction in lane 63.  Each step is one VALU
// instruction, where a __shfl_xor butterfly step is an LDS round trip
// (ds_bpermute).  Lanes a step does not write keep their own value, which is
// neutral for max and argmax; sums pass 0 for them.
#pragma once
#include <hip/hip_runtime.h>

namespace rsv {

template <int CTRL, int RM = 0xF>
__device__ __forceinline__ float dpp_or_zero(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, RM, 0xF, false));
}
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ float dpp_or_self(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, RM, 0xF, false));
}
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ int dpp_or_self(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, RM, 0xF, false);
}

// Sum over the wave; valid in lane 63.
__device__ __forceinline__ float wave_sum_last(float v) {
    v += dpp_or_zero<0xB1>(v);
    v += dpp_or_zero<0x4E>(v);
    v += dpp_or_zero<0x141>(v);
    v += dpp_or_zero<0x140>(v);
    v += dpp_or_zero<0x142, 0xA>(v);
    v += dpp_or_zero<0x143, 0xC>(v);
    return v;
}
// Max over the wave; valid in lane 63.
__device__ __forceinline__ float wave_max_last(float v) {
    v = fmaxf(v, dpp_or_self<0xB1>(v));
    v = fmaxf(v, dpp_or_self<0x4E>(v));
    v = fmaxf(v, dpp_or_self<0x141>(v));
    v = fmaxf(v, dpp_or_self<0x140>(v));
    v = fmaxf(v, dpp_or_self<0x142, 0xA>(v));
    v = fmaxf(v, dpp_or_self<0x143, 0xC>(v));
    return v;
}
// (value, index) with the larger value, the smaller index among equal
// values; valid in lane 63.
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ void argmax_step(float &bv, int &bi) {
    const float ov = dpp_or_self<CTRL, RM>(bv);
    const int oi = dpp_or_self<CTRL, RM>(bi);
    if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
    }
}
__device__ __forceinline__ void wave_argmax_last(float &bv, int &bi) {
    argmax_step<0xB1>(bv, bi);
    argmax_step<0x4E>(bv, bi);
    argmax_step<0x141>(bv, bi);
    argmax_step<0x140>(bv, bi);
    argmax_step<0x142, 0xA>(bv, bi);
    argmax_step<0x143, 0xC>(bv, bi);
}

}  // namespace rsv
