// The MoE pieces of the batched prefill that have no one-token counterpart:
// the router over a batch of rows, the grouping of the (token, slot) pairs
// by expert (so one weight fetch serves every token routed to an expert),
// and the ordered combine of the experts' outputs into the residual rows.
// One-token semantics they restate (paths of the reference repository):
//   router logits       DenseLinear::matvec (wpc-runtime/src/weights.rs:59-78)
//   expert loop, combine  qwen3_moe_model.rs:509-530
#include <hip/hip_runtime.h>

#include "wpcg_internal.hpp"

namespace wpcg {
namespace {

// R[t][e] = sum_k X[t][k] * W[e][k] for a tile of 16 experts x 16 rows per
// workgroup: thread (e, t) runs its dot in index order with fused
// multiply-adds over K chunks of 128 staged in LDS (rows padded by one
// float, so the 16 rows of a chunk fall in 16 banks).
constexpr int RT_K = 128;
__global__ __launch_bounds__(256) void k_pf_router(const float* __restrict__ X, const float* __restrict__ W,
                                                   int T, int E, int K, float* __restrict__ R)
{
    __shared__ float xs[16][RT_K + 1];
    __shared__ float ws[16][RT_K + 1];
    const int e0 = blockIdx.x * 16, t0 = blockIdx.y * 16;
    const int te = threadIdx.x >> 4, tt = threadIdx.x & 15;
    float acc = 0.0f;
    for (int k0 = 0; k0 < K; k0 += RT_K) {
        for (int i = threadIdx.x; i < 16 * RT_K; i += 256) {
            const int r = i / RT_K, k = i % RT_K;
            const bool in = k0 + k < K;
            xs[r][k] = in && t0 + r < T ? X[(size_t)(t0 + r) * K + k0 + k] : 0.0f;
            ws[r][k] = in && e0 + r < E ? W[(size_t)(e0 + r) * K + k0 + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < RT_K; k++) acc = fmaf(xs[tt][k], ws[te][k], acc);
        __syncthreads();
    }
    if (t0 + tt < T && e0 + te < E) R[(size_t)(t0 + tt) * E + e0 + te] = acc;
}

// The P = T * top_k pairs q = t * top_k + k, sorted by expert, ties in pair
// order: pair_tok[i] is the token of the i-th sorted pair, pair_pos[q] the
// sorted position of pair q; work items {expert, first sorted pair, count
// <= GEMM_GROUP_COLS} cover every expert's run. One workgroup; slots with
// id < 0 (fewer finite probabilities than top_k) belong to no expert.
constexpr int GR_WG = 1024;
__global__ __launch_bounds__(GR_WG) void k_pf_group(const int32_t* __restrict__ ids, int P, int E,
                                                    int top_k, int* __restrict__ pair_tok,
                                                    int* __restrict__ pair_pos, int* __restrict__ items,
                                                    int* __restrict__ nitems)
{
    __shared__ int sid[PF_MAX_PAIRS];
    __shared__ int cnt[ROUTE_MAXN], off[ROUTE_MAXN], ioff[ROUTE_MAXN];
    for (int e = threadIdx.x; e < E; e += GR_WG) cnt[e] = 0;
    for (int q = threadIdx.x; q < P; q += GR_WG) sid[q] = ids[q];
    __syncthreads();
    for (int q = threadIdx.x; q < P; q += GR_WG) {
        const int e = sid[q];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
        else pair_pos[q] = -1;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int o = 0, io = 0;
        for (int e = 0; e < E; e++) {
            off[e] = o;
            ioff[e] = io;
            o += cnt[e];
            io += (cnt[e] + GEMM_GROUP_COLS - 1) / GEMM_GROUP_COLS;
        }
        *nitems = io;
    }
    __syncthreads();
    // stable placement: wave w takes experts w, w + 16, ...; a ballot per
    // 64 pairs gives each match its rank among the earlier matches
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int e = wave; e < E; e += GR_WG / 64) {
        int run = off[e];
        for (int q0 = 0; q0 < P; q0 += 64) {
            const int q = q0 + lane;
            const bool hit = q < P && sid[q] == e;
            const uint64_t mask = __ballot(hit);
            if (hit) {
                const int at = run + __popcll(mask & ((1ull << lane) - 1));
                pair_tok[at] = q / top_k;
                pair_pos[q] = at;
            }
            run += __popcll(mask);
        }
    }
    for (int e = threadIdx.x; e < E; e += GR_WG)
        for (int c = 0, i = ioff[e]; c < cnt[e]; c += GEMM_GROUP_COLS, i++) {
            items[3 * i] = e;
            items[3 * i + 1] = off[e] + c;
            items[3 * i + 2] = min(GEMM_GROUP_COLS, cnt[e] - c);
        }
}

// X[t] += sum over slots k in order of w[t][k] * D[pair_pos[t * top_k + k]]
// (the expert outputs in sorted-pair rows); slots with no expert add 0.
__global__ __launch_bounds__(256) void k_pf_combine(float* __restrict__ X, const float* __restrict__ D,
                                                    const float* __restrict__ w, const int* __restrict__ pair_pos,
                                                    int top_k, int H)
{
    const int t = blockIdx.y;
    const int h = blockIdx.x * 256 + threadIdx.x;
    if (h >= H) return;
    float acc = 0.0f;
    for (int k = 0; k < top_k; k++) {
        const int p = pair_pos[t * top_k + k];
        if (p >= 0) acc = fmaf(w[t * top_k + k], D[(size_t)p * H + h], acc);
    }
    X[(size_t)t * H + h] += acc;
}

}  // namespace

hipError_t launch_pf_router(const float* X, const float* W, int T, int E, int K, float* R, hipStream_t s)
{
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_pf_router, dim3((E + 15) / 16, (T + 15) / 16), dim3(256), 0, s, X, W, T, E, K, R);
    return hipGetLastError();
}

hipError_t launch_pf_group(const int32_t* ids, int P, int E, int top_k, int* pair_tok, int* pair_pos, int* items,
                           int* nitems, hipStream_t s)
{
    if (P < 1 || P > PF_MAX_PAIRS || E < 1 || E > ROUTE_MAXN) return hipErrorInvalidValue;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_pf_group, dim3(1), dim3(GR_WG), 0, s, ids, P, E, top_k, pair_tok, pair_pos, items, nitems);
    return hipGetLastError();
}

hipError_t launch_pf_combine(float* X, const float* D, const float* w, const int* pair_pos, int T, int top_k, int H,
                             hipStream_t s)
{
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_pf_combine, dim3((H + 255) / 256, T), dim3(256), 0, s, X, D, w, pair_pos, top_k, H);
    return hipGetLastError();
}

}  // namespace wpcg
