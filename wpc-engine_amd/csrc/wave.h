// Whole-wave (64-lane) sum and max on gfx950 through DPP lane exchanges:
// quad permutations, the half-row and row mirrors, then row broadcasts of
// lane 15 and lane 31 carry the row results up to lane 63, which holds the
// total; readlane 63 gives it to every lane. Each step is a VALU operation
// with a DPP source, so the reduction never goes through LDS (a
// cross-lane ds_bpermute per step costs an LDS round trip).
//
// The additions are a fixed tree, the same on every call: results are
// deterministic, with the tree's rounding (not an index-order sum).
#pragma once
#include <hip/hip_runtime.h>

namespace wpcg {

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float wave_dpp(float old, float v)
{
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int wave_dpp_i(int old, int v)
{
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xF, false);
}

constexpr int WDPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int WDPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int WDPP_HALF_MIRROR = 0x141; // lane i <-> 7-i within each 8
constexpr int WDPP_MIRROR = 0x140;      // lane i <-> 15-i within each 16
constexpr int WDPP_BCAST15 = 0x142;     // lane 15 of each row to the next row
constexpr int WDPP_BCAST31 = 0x143;     // lane 31 to rows 2 and 3

__device__ __forceinline__ float wave_sum(float v)
{
    v += wave_dpp<WDPP_XOR1>(0.0f, v);
    v += wave_dpp<WDPP_XOR2>(0.0f, v);
    v += wave_dpp<WDPP_HALF_MIRROR>(0.0f, v);
    v += wave_dpp<WDPP_MIRROR>(0.0f, v);           // every lane: its row's sum
    v += wave_dpp<WDPP_BCAST15, 0xA>(0.0f, v);     // rows 1, 3: + the row before
    v += wave_dpp<WDPP_BCAST31, 0xC>(0.0f, v);     // rows 2, 3: + rows 0..1
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, wave_dpp<WDPP_XOR1>(-INFINITY, v));
    v = fmaxf(v, wave_dpp<WDPP_XOR2>(-INFINITY, v));
    v = fmaxf(v, wave_dpp<WDPP_HALF_MIRROR>(-INFINITY, v));
    v = fmaxf(v, wave_dpp<WDPP_MIRROR>(-INFINITY, v));
    v = fmaxf(v, wave_dpp<WDPP_BCAST15, 0xA>(-INFINITY, v));
    v = fmaxf(v, wave_dpp<WDPP_BCAST31, 0xC>(-INFINITY, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ int wave_sum_i(int v)
{
    v += wave_dpp_i<WDPP_XOR1>(0, v);
    v += wave_dpp_i<WDPP_XOR2>(0, v);
    v += wave_dpp_i<WDPP_HALF_MIRROR>(0, v);
    v += wave_dpp_i<WDPP_MIRROR>(0, v);
    v += wave_dpp_i<WDPP_BCAST15, 0xA>(0, v);
    v += wave_dpp_i<WDPP_BCAST31, 0xC>(0, v);
    return __builtin_amdgcn_readlane(v, 63);
}

}  // namespace wpcg
