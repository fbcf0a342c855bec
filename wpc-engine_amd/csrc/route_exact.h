// The MoE router's tail in the reference's arithmetic, for one wave:
// softmax_inplace (wpc-runtime/src/norm.rs:28-43) of the router scores and
// route (qwen3_moe_model.rs:376-402). Used by the routing launch and by the
// EXACT expert GEMV launch that routes itself.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

// the reference's exp as device code (every includer of ref_expf.h in a
// HIP source defines it so)
#ifndef REF_EXPF_FN
#define REF_EXPF_FN __device__ __forceinline__
#endif
#include "ref_expf.h"
#include "wave.h"

namespace wpcg {

constexpr int RT_PER = 8;  // scores per lane: n <= 64 * RT_PER

// ((e[0] + e[1]) + e[2]) + ... + e[n-1], each sum rounded: the index-order
// sum of norm.rs:36-38. The LDS reads go out 16 bytes and 32 values at a
// time so the chain of additions does not wait on each read.
__device__ __forceinline__ float ordered_sum(const float* e, int n)
{
    float s = 0.0f;
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = reinterpret_cast<const float4*>(e + i)[u];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            s = __fadd_rn(s, v[u].x);
            s = __fadd_rn(s, v[u].y);
            s = __fadd_rn(s, v[u].z);
            s = __fadd_rn(s, v[u].w);
        }
    }
    for (; i < n; i++) s = __fadd_rn(s, e[i]);
    return s;
}

// The lane holding the largest (bv, bi) over the wave, ordered by value
// and then by the lower index (v > u, or v == u and i < j), in every lane:
// the reduction steps of wave_max with the comparison carried along. The
// order is total on the candidates (no NaN; -0 and +0 tie and their
// indices decide), so the winner does not depend on the reduction's shape.
__device__ __forceinline__ void wave_argmax(float& bv, int& bi)
{
    auto take = [&](float ov, int oi) {
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    };
    take(wave_dpp<WDPP_XOR1>(-INFINITY, bv), wave_dpp_i<WDPP_XOR1>(0x7fffffff, bi));
    take(wave_dpp<WDPP_XOR2>(-INFINITY, bv), wave_dpp_i<WDPP_XOR2>(0x7fffffff, bi));
    take(wave_dpp<WDPP_HALF_MIRROR>(-INFINITY, bv), wave_dpp_i<WDPP_HALF_MIRROR>(0x7fffffff, bi));
    take(wave_dpp<WDPP_MIRROR>(-INFINITY, bv), wave_dpp_i<WDPP_MIRROR>(0x7fffffff, bi));
    take(wave_dpp<WDPP_BCAST15, 0xA>(-INFINITY, bv), wave_dpp_i<WDPP_BCAST15, 0xA>(0x7fffffff, bi));
    take(wave_dpp<WDPP_BCAST31, 0xC>(-INFINITY, bv), wave_dpp_i<WDPP_BCAST31, 0xC>(0x7fffffff, bi));
    bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 63));
    bi = __builtin_amdgcn_readlane(bi, 63);
}

// softmax of scores[0..n) then top_k strict-`>` scans (the largest
// remaining probability, the lowest index on ties, never NaN or -inf), the
// chosen weights divided by their sum in chosen order when norm_topk and
// the sum is positive; unfilled slots get id -1, weight 0. Called by every
// lane of one wave (no other wave takes part); e is LDS scratch of n floats
// (16-byte aligned) and tab of 32 doubles, ids / w the outputs (LDS or
// global memory), written by lane 0. The exps go through e so that each
// lane adds them in index order; exp's table is read from its copy in tab
// (a lookup in the constant array was a memory round trip after the
// scores arrived); each scan is a DPP reduction (through LDS lane
// exchanges the eight scans cost ~2.4 us).
__device__ __forceinline__ void softmax_route_wave(const float* __restrict__ scores, int n, int top_k,
                                                   int norm_topk, int32_t* ids, float* w, float* e, double* tab)
{
    const int lane = threadIdx.x & 63;
    {
        constexpr double T[32] = REF_EXPF_TABLE;
        if (lane < 32) tab[lane] = T[lane];
    }
    float v[RT_PER];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < RT_PER; j++) {
        const int i = lane + 64 * j;
        v[j] = i < n ? scores[i] : -INFINITY;
        m = fmaxf(m, v[j]);
    }
    m = wave_max(m);
    // the table's LDS writes come before the lookups (one wave)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < RT_PER; j++) {
        const int i = lane + 64 * j;
        if (i < n) {
            v[j] = ref_expf_tab(__fsub_rn(v[j], m), tab);
            e[i] = v[j];
        }
    }
    // one wave: its LDS writes are performed before its later reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float s = ordered_sum(e, n);  // every lane, the same additions
#pragma unroll
    for (int j = 0; j < RT_PER; j++) {
        const int i = lane + 64 * j;
        if (i < n) {
            if (s > 0.0f) v[j] = __fdiv_rn(v[j], s);
            if (!(v[j] > -INFINITY)) v[j] = -INFINITY;  // NaN is never chosen
        }
    }
    int got = 0;
    for (int k = 0; k < top_k; k++) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < RT_PER; j++)
            if (v[j] > bv) { bv = v[j]; bi = lane + 64 * j; }
        wave_argmax(bv, bi);
        if (!(bv > -INFINITY)) break;
#pragma unroll
        for (int j = 0; j < RT_PER; j++)
            if (lane + 64 * j == bi) v[j] = -INFINITY;
        if (lane == 0) { ids[k] = bi; w[k] = bv; }
        got = k + 1;
    }
    if (lane == 0) {  // lane 0 rereads its own writes
        float sw = 0.0f;
        if (norm_topk)
            for (int k = 0; k < got; k++) sw = __fadd_rn(sw, w[k]);
        if (norm_topk && sw > 0.0f)
            for (int k = 0; k < got; k++) w[k] = __fdiv_rn(w[k], sw);
        for (int k = got; k < top_k; k++) { ids[k] = -1; w[k] = 0.0f; }
    }
}

}  // namespace wpcg
