// The expert-grouped GEMM's X format: each 128-value block of an X row as
// x ~= s_b * Q / 2^21 with s_b = max|x_b| / 127 and
// Q = rint(x * 127 * 2^21 / max|x_b|) = d0*2^21 + d1*2^14 + d2*2^7 + d3
// (int8 digits: d0 = Q >> 21, d1..d3 7-bit fields), stored as a record of
// 512 bytes per (row, block) in the order the GEMM's LDS operand wants it,
// plus {s_b 2^-7, sum(x_b)} per (row, block). Shared by the GEMM's digit
// pass and the prefill kernels that write the format themselves.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace wpcg {

// Byte of value k (0..127) of a block, digit d, in its 512-byte record:
// piece (h = k >> 6, q = k & 3, d), byte ((k >> 3) & 7) + 8 ((k >> 2) & 1),
// the order in which lane group q's 16-byte code word holds the codes.
__device__ __forceinline__ int dg_pos(int k, int d)
{
    return (k >> 6) * 256 + (k & 3) * 64 + d * 16 + ((k >> 3) & 7) + 8 * ((k >> 2) & 1);
}

// One block held by the 32 lanes of a half wave (lane l: values
// 4 (l & 31) .. +3 in v): its max |x| and sum over the 32 lanes by DPP
// inside rows of 16 and the row swap, then its digits written to the
// 512-byte record at st (LDS). Returns {s_b 2^-7, sum} on every lane.
__device__ __forceinline__ float2 digit_block(const float (&v)[4], uint8_t* st)
{
    const int k0 = 4 * (threadIdx.x & 31);
    uint32_t mb = __float_as_uint(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    float sm = (v[0] + v[1]) + (v[2] + v[3]);
    mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0xB1, 0xF, 0xF, false));
    sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0xB1, 0xF, 0xF, false));
    mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x4E, 0xF, 0xF, false));
    sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0x4E, 0xF, 0xF, false));
    mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x141, 0xF, 0xF, false));
    sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0x141, 0xF, 0xF, false));
    mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x140, 0xF, 0xF, false));
    sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0x140, 0xF, 0xF, false));
    const auto mr = __builtin_amdgcn_permlane16_swap(mb, mb, false, false);
    const float Mx = __uint_as_float(max((uint32_t)mr[0], (uint32_t)mr[1]));
    const auto sr = __builtin_amdgcn_permlane16_swap(__float_as_uint(sm), __float_as_uint(sm), false, false);
    const float Sx = __uint_as_float(sr[0]) + __uint_as_float(sr[1]);
    const float inv = Mx > 0.0f ? (127.0f * 2097152.0f) * __builtin_amdgcn_rcpf(Mx) : 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int Q = (int)rintf(v[q] * inv);
        const int k = k0 + q;
        st[dg_pos(k, 0)] = (uint8_t)(Q >> 21);
        st[dg_pos(k, 1)] = (uint8_t)((Q >> 14) & 127);
        st[dg_pos(k, 2)] = (uint8_t)((Q >> 7) & 127);
        st[dg_pos(k, 3)] = (uint8_t)(Q & 127);
    }
    return make_float2(Mx * (1.0f / 127.0f) * 0x1p-7f, Sx);  // s_b 2^-7
}

}  // namespace wpcg
