// The MoE pieces of the batched prefill that have no one-token counterpart:
// the router over a batch of rows, the grouping of the (token, slot) pairs
// by expert (so one weight fetch serves every token routed to an expert),
// and the ordered combine of the experts' outputs into the residual rows.
// One-token semantics they restate (paths of the reference repository):
//   router logits       DenseLinear::matvec (wpc-runtime/src/weights.rs:59-78)
//   expert loop, combine  qwen3_moe_model.rs:509-530
#include <hip/hip_runtime.h>

#include "wave.h"
#include "wpcg_internal.hpp"
#include "xdigits.h"
#include "xpack.h"

namespace wpcg {
namespace {

// A buffer resource over [base, base + bytes): loads past the end return
// zeros without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// R[t][e] = sum_k X[t][k] * W[e][k] on the fp32 matrix cores: workgroup
// (16 experts, 16 rows), each of its 8 waves one eighth of K with every
// 16-byte load of its slice in flight at once (RU per operand and lane: a
// whole eighth of a 2048-wide row), then the eighths added in order through
// LDS. Lane (q, r) of a wave reads 16 bytes of X row t0 + r and of W row
// e0 + r at k0 + 4q; with component i of both, v_mfma_f32_16x16x4_f32 adds
// X[r][k0 + 4kk + i] * W[c][k0 + 4kk + i] over kk, so four instructions
// cover k0 .. k0 + 15 (two accumulators, alternate 16-value groups). Rows
// past T or E read row 0 and are never written. K % 128 == 0. The loads
// are range-checked buffer loads: a load past the wave's eighth reads
// zeros, with no branch between the loads (a guarded load per 16 values
// made the compiler wait for each before the next: 10.5 us for 256 rows of
// 2048 over 128 experts). (Four waves with four loads in flight each waited
// on eight load round trips in a row: 9.4 us.)
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef unsigned rt_u32x4 __attribute__((ext_vector_type(4)));
constexpr int RT_WG = 512, RT_U = 16;
__global__ __launch_bounds__(RT_WG) void k_pf_router(const float* __restrict__ X, const float* __restrict__ W,
                                                     int T, int E, int K, float* __restrict__ R)
{
    __shared__ f32x4v red[8][64];
    const int e0 = blockIdx.x * 16, t0 = blockIdx.y * 16;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    const int kq = K / 8, kb = wave * kq;
    // the tile's rows (uniform resources); rows past T or E read row 0
    const auto xrs = buf_rsrc(X + (size_t)t0 * K, min(16, T - t0) * K * 4);
    const auto wrs = buf_rsrc(W + (size_t)e0 * K, min(16, E - e0) * K * 4);
    const int xo = (t0 + r < T ? r : 0) * K + kb + 4 * q, wo = (e0 + r < E ? r : 0) * K + kb + 4 * q;
    f32x4v d0 = {0.f, 0.f, 0.f, 0.f}, d1 = d0;
    for (int k = 0; k < kq; k += 16 * RT_U) {
        float4 a[RT_U], b[RT_U];
#pragma unroll
        for (int u = 0; u < RT_U; u++) {
            const bool in = k + 16 * u < kq;
            const rt_u32x4 av = __builtin_amdgcn_raw_buffer_load_b128(xrs, in ? (xo + k + 16 * u) * 4 : 0x7FFFFFF0, 0, 0);
            const rt_u32x4 bv = __builtin_amdgcn_raw_buffer_load_b128(wrs, in ? (wo + k + 16 * u) * 4 : 0x7FFFFFF0, 0, 0);
            __builtin_memcpy(&a[u], &av, 16);
            __builtin_memcpy(&b[u], &bv, 16);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load out before the first product
#pragma unroll
        for (int u = 0; u < RT_U; u += 2) {
            d0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].x, b[u].x, d0, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u + 1].x, b[u + 1].x, d1, 0, 0, 0);
            d0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].y, b[u].y, d0, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u + 1].y, b[u + 1].y, d1, 0, 0, 0);
            d0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].z, b[u].z, d0, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u + 1].z, b[u + 1].z, d1, 0, 0, 0);
            d0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].w, b[u].w, d0, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u + 1].w, b[u + 1].w, d1, 0, 0, 0);
        }
    }
    red[wave][lane] = d0 + d1;
    __syncthreads();
    if (wave == 0) {
        // lane (g, j) holds rows (tokens) 4g..4g+3 of column (expert) j
        const f32x4v s4 = ((red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane])) +
                          ((red[4][lane] + red[5][lane]) + (red[6][lane] + red[7][lane]));
        const int g = lane >> 4, j = lane & 15;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + 4 * g + i, e = e0 + j;
            if (t < T && e < E) R[(size_t)t * E + e] = s4[i];
        }
    }
}

// RMSNorm of rows of X (FAST arithmetic: fused multiply-add squares,
// 1 / sqrt(mean + eps), then (x * scale) * w) written straight as the
// GEMM's packed X, with no fp32 copy and no packing launch: workgroup
// (16-row tile q, block b). Every workgroup of a tile computes its 16 row
// norms itself (each row is read from L2 once per block: 256 workgroups for
// 256 rows of 2048 beat 64 workgroups of four blocks each, 15 us), then
// stages its block of the normed rows in LDS and packs it.
constexpr int RP_BG = 1;
__global__ __launch_bounds__(256) void k_rms_pack(const float* __restrict__ X, const float* __restrict__ w, int n,
                                                  int H, float eps, int XT, uint32_t* __restrict__ xf,
                                                  float* __restrict__ xsum)
{
    __shared__ float rstd[16];
    __shared__ __align__(16) float tile[16][132];
    __shared__ float red[2][4][16];
    const int q = blockIdx.x, r = threadIdx.x >> 4, p = threadIdx.x & 15;
    const int row = 16 * q + r;
    // row r's squares by its 16 threads (lanes 16r..16r+15 of one wave)
    float ss = 0.0f;
    if (row < n)
#pragma unroll 8
        for (int k = 4 * p; k < H; k += 64) {
            const float4 v = *reinterpret_cast<const float4*>(X + (size_t)row * H + k);
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
    ss += __shfl_xor(ss, 8);
    ss += __shfl_xor(ss, 4);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 1);
    if (p == 0) rstd[r] = __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(__fdiv_rn(ss, (float)H), eps)));
    __syncthreads();
    const int b1 = min(H / 128, (int)(blockIdx.y + 1) * RP_BG);
    const int rr = threadIdx.x >> 4, cc = (threadIdx.x & 15) * 8, mrow = 16 * q + rr;
    for (int b = blockIdx.y * RP_BG; b < b1; b++) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int k = b * 128 + cc + 4 * h;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (mrow < n) v = *reinterpret_cast<const float4*>(X + (size_t)mrow * H + k);
            const float4 g = *reinterpret_cast<const float4*>(w + k);
            const float sc = rstd[rr];
            *reinterpret_cast<float4*>(&tile[rr][cc + 4 * h]) =
                make_float4(__fmul_rn(__fmul_rn(v.x, sc), g.x), __fmul_rn(__fmul_rn(v.y, sc), g.y),
                            __fmul_rn(__fmul_rn(v.z, sc), g.z), __fmul_rn(__fmul_rn(v.w, sc), g.w));
        }
        __syncthreads();
        pack_tile_split(&tile[0][0], 132, min(16, n - 16 * q), b, q, XT, xf, xsum, red);
    }
}

// o_proj's K-slices added in slice order with its bias and the residual into
// X (the new residual, as k_gemm_reduce writes it), and that row's RMSNorm
// (FAST, as k_rms_norm rows computes it: each thread's squares by fused
// multiply-adds, the wave sums, the four waves in a fixed order) into XN:
// one workgroup of 256 threads per row, H <= 256 * RN_MAXV. With dg, the
// normed row also as the expert GEMM's X digits (xdigits.h; the values
// k_pf_digits would read from XN), staged in LDS.
constexpr int RN_MAXV = PF_NORM_MAXH / 256;
__global__ __launch_bounds__(256) void k_pf_reduce_norm(const float* __restrict__ part, int kg, int Mp,
                                                        int rows_pad, int H, const float* __restrict__ bias,
                                                        float* __restrict__ X, const float* __restrict__ w,
                                                        float eps, float* __restrict__ XN, uint8_t* __restrict__ dg,
                                                        float2* __restrict__ dxs)
{
    __shared__ float red[4];
    __shared__ float xn_s[PF_NORM_MAXH];
    __shared__ __align__(16) uint8_t rec[PF_NORM_MAXH / 128 + 1][512];  // the last: blocks past the row
    const int m = blockIdx.x;
    const size_t slice = (size_t)Mp * rows_pad;
    float v[RN_MAXV];
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < RN_MAXV; i++) {
        const int k = threadIdx.x + 256 * i;
        if (k < H) {
            const float* p = part + (size_t)m * rows_pad + k;
            float s = p[0];
            for (int q = 1; q < kg; q++) s = s + p[q * slice];
            if (bias) s += bias[k];
            s += X[(size_t)m * H + k];
            v[i] = s;
            sq = fmaf(s, s, sq);
        }
    }
    sq = wave_sum(sq);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
    __syncthreads();
    const float total = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(__fdiv_rn(total, (float)H), eps)));
#pragma unroll
    for (int i = 0; i < RN_MAXV; i++) {
        const int k = threadIdx.x + 256 * i;
        if (k < H) {
            const float xn = __fmul_rn(__fmul_rn(v[i], scale), w[k]);
            X[(size_t)m * H + k] = v[i];
            XN[(size_t)m * H + k] = xn;
            xn_s[k] = xn;
        }
    }
    if (!dg) return;  // uniform
    __syncthreads();
    // half wave hw takes blocks hw, hw + 8, ... (whole passes: a block past
    // the row is digitised from zeros into the spare record)
    const int nb = H / 128, hw = threadIdx.x >> 5, k0 = 4 * (threadIdx.x & 31);
    for (int b0 = 0; b0 < nb; b0 += 8) {
        const int b = b0 + hw;
        const bool ok = b < nb;
        float v4[4];
#pragma unroll
        for (int q = 0; q < 4; q++) v4[q] = ok ? xn_s[b * 128 + k0 + q] : 0.0f;
        const float2 sx = digit_block(v4, rec[ok ? b : PF_NORM_MAXH / 128]);
        if (ok && (threadIdx.x & 31) == 0) dxs[(size_t)m * nb + b] = sx;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nb * 32; i += 256)
        *reinterpret_cast<rt_u32x4*>(dg + (size_t)m * nb * 512 + i * 16) =
            *reinterpret_cast<const rt_u32x4*>(&rec[i >> 5][(i & 31) * 16]);
}

// The P = T * top_k pairs q = t * top_k + k, sorted by expert, ties in pair
// order: pair_tok[i] is the token of the i-th sorted pair, pair_pos[q] the
// sorted position of pair q; work items {expert, first sorted pair, count
// <= GEMM_GROUP_COLS} cover every expert's run. One workgroup; slots with
// id < 0 (fewer finite probabilities than top_k) belong to no expert.
// A token's top_k experts are distinct (route() picks each index at most
// once), so the pairs of one expert come from distinct tokens, in token
// order: the rank of pair (t, k) in its expert's run is the number of
// tokens before t that chose the expert. Each expert keeps a bitmask of
// the tokens that chose it; a pair's rank is the popcount of the bits below
// its token, computed by every pair at once. (A stable placement by one
// ballot per expert and 64 pairs, in order, took 25 us for 2048 pairs.)
constexpr int GR_WG = 1024;
constexpr int GR_TW = PF_GROUP_MAXT / 32;          // bitmask words per expert
constexpr int GR_PT = PF_MAX_PAIRS / GR_WG;        // pairs per thread at most
__global__ __launch_bounds__(GR_WG) void k_pf_group(const int32_t* __restrict__ ids, int P, int E,
                                                    int top_k, int* __restrict__ pair_tok,
                                                    int* __restrict__ pair_pos, int* __restrict__ items,
                                                    int* __restrict__ nitems)
{
    __shared__ uint32_t tmask[ROUTE_MAXN][GR_TW];
    __shared__ int off[ROUTE_MAXN], ioff[ROUTE_MAXN];
    for (int i = threadIdx.x; i < E * GR_TW; i += GR_WG) tmask[i / GR_TW][i % GR_TW] = 0u;
    int myid[GR_PT];
#pragma unroll
    for (int u = 0; u < GR_PT; u++) {
        const int q = threadIdx.x + u * GR_WG;
        myid[u] = q < P ? ids[q] : -1;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < GR_PT; u++) {
        const int q = threadIdx.x + u * GR_WG;
        if (q >= P) break;
        const int e = myid[u], t = q / top_k;
        if (e >= 0 && e < E) atomicOr(&tmask[e][t >> 5], 1u << (t & 31));
        else pair_pos[q] = -1;
    }
    __syncthreads();
    // exclusive prefix sums of the counts and of the item counts (E <= 256:
    // a Hillis-Steele scan over LDS)
    const int e_me = threadIdx.x;
    int c_me = 0;
    if (e_me < E)
#pragma unroll
        for (int w = 0; w < GR_TW; w++) c_me += __popc(tmask[e_me][w]);
    const int i_me = (c_me + GEMM_GROUP_COLS - 1) / GEMM_GROUP_COLS;
    if (e_me < ROUTE_MAXN) {
        off[e_me] = c_me;
        ioff[e_me] = i_me;
    }
    __syncthreads();
    for (int d = 1; d < ROUTE_MAXN; d <<= 1) {
        int a = 0, b = 0;
        if (e_me < ROUTE_MAXN && e_me >= d) {
            a = off[e_me - d];
            b = ioff[e_me - d];
        }
        __syncthreads();
        if (e_me < ROUTE_MAXN && e_me >= d) {
            off[e_me] += a;
            ioff[e_me] += b;
        }
        __syncthreads();
    }
    if (e_me < ROUTE_MAXN) {  // inclusive -> exclusive
        off[e_me] -= c_me;
        ioff[e_me] -= i_me;
    }
    if (e_me == ROUTE_MAXN - 1) *nitems = ioff[e_me] + i_me;
    __syncthreads();
    // every pair's place: its expert's offset plus the tokens before its own
#pragma unroll
    for (int u = 0; u < GR_PT; u++) {
        const int q = threadIdx.x + u * GR_WG;
        if (q >= P) break;
        const int e = myid[u];
        if (e < 0 || e >= E) continue;
        const int t = q / top_k, tw = t >> 5;
        int rank = __popc(tmask[e][tw] & ((1u << (t & 31)) - 1u));
        for (int w = 0; w < tw; w++) rank += __popc(tmask[e][w]);
        const int at = off[e] + rank;
        pair_tok[at] = t;
        pair_pos[q] = at;
    }
    if (e_me < E)
        for (int c = 0, i = ioff[e_me]; c < c_me; c += GEMM_GROUP_COLS, i++) {
            items[3 * i] = e_me;
            items[3 * i + 1] = off[e_me] + c;
            items[3 * i + 2] = min(GEMM_GROUP_COLS, c_me - c);
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
    if (K % 128 || T < 1 || E < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_router, dim3((E + 15) / 16, (T + 15) / 16), dim3(RT_WG), 0, s, X, W, T, E, K, R);
    return hipGetLastError();
}

hipError_t launch_rms_pack_rows(const float* X, const float* w, int n, int H, float eps, void* xf, float* xsum,
                                hipStream_t s)
{
    if (n < 1 || H < 128 || H % 128) return hipErrorInvalidValue;
    (void)hipGetLastError();
    const dim3 grid((unsigned)((n + 15) / 16), (unsigned)((H / 128 + RP_BG - 1) / RP_BG));
    hipLaunchKernelGGL(k_rms_pack, grid, dim3(256), 0, s, X, w, n, H, eps, gemm_rows_tiles(n),
                       static_cast<uint32_t*>(xf), xsum);
    return hipGetLastError();
}

hipError_t launch_pf_reduce_norm(const float* part, int kg, int M, int H, int rows_pad, const float* bias, float* X,
                                 const float* w, float eps, float* XN, void* dg, float* dxs, hipStream_t s)
{
    if (M < 1 || kg < 1 || H < 1 || H > 256 * RN_MAXV || rows_pad < H || (dg && (H % 128 || !dxs)))
        return hipErrorInvalidValue;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_pf_reduce_norm, dim3((unsigned)M), dim3(256), 0, s, part, kg, gemm_rows_tiles(M) / 4 * 32,
                       rows_pad, H, bias, X, w, eps, XN, static_cast<uint8_t*>(dg), reinterpret_cast<float2*>(dxs));
    return hipGetLastError();
}

hipError_t launch_pf_group(const int32_t* ids, int P, int E, int top_k, int* pair_tok, int* pair_pos, int* items,
                           int* nitems, hipStream_t s)
{
    // the tokens' bitmasks hold PF_GROUP_MAXT tokens
    if (P < 1 || P > PF_MAX_PAIRS || E < 1 || E > ROUTE_MAXN || top_k < 1 || P / top_k > PF_GROUP_MAXT ||
        P % top_k)
        return hipErrorInvalidValue;
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
