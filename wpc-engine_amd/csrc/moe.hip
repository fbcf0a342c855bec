// Qwen3-MoE sparse-MLP pieces on gfx950: the fp32 router (DenseLinear),
// softmax, top-k routing, SiLU*up and the weighted combine of the chosen
// experts' outputs. The expert GEMVs themselves are the dequant-GEMV kernels
// (gemv.hip) with device-side expert selection, so a routed layer needs no
// host round trip.
//
// Every piece here reproduces the reference's arithmetic exactly, operation
// for operation (Rust does not contract or reassociate): products and sums
// round separately, sums run in index order, exp is the host libm's expf
// (ref_expf.h). The FAST router is the one exception (a parallel sum).
#include <hip/hip_runtime.h>

#define REF_EXPF_FN __device__ __forceinline__
#include "ref_expf.h"
#include "route_exact.h"
#include "wpcg_internal.hpp"
#include "wave.h"

namespace wpcg {
namespace {

// ---- DenseLinear::matvec (wpc-runtime/src/weights.rs:59-78) -------------
// y[r] = sum_i W[r][i] * x[i], W row-major [out_f][in_f].
// EXACT: one lane per row, index order, product and sum rounded separately;
// each lane walks its own row (16-byte loads, reused from cache lines).
__global__ __launch_bounds__(64) void k_dense_exact(const float* __restrict__ w,
                                                    const float* __restrict__ x,
                                                    const float* __restrict__ bias,
                                                    float* __restrict__ y, int out_f, int in_f)
{
    const int r = blockIdx.x * 64 + threadIdx.x;
    const float* row = w + (size_t)min(r, out_f - 1) * in_f;
    float acc = 0.0f;
    int i = 0;
    if ((in_f & 3) == 0) {
#pragma unroll 4
        for (; i < in_f; i += 4) {
            const float4 v = *reinterpret_cast<const float4*>(row + i);
            acc = __fadd_rn(acc, __fmul_rn(v.x, x[i]));
            acc = __fadd_rn(acc, __fmul_rn(v.y, x[i + 1]));
            acc = __fadd_rn(acc, __fmul_rn(v.z, x[i + 2]));
            acc = __fadd_rn(acc, __fmul_rn(v.w, x[i + 3]));
        }
    }
    for (; i < in_f; i++) acc = __fadd_rn(acc, __fmul_rn(row[i], x[i]));
    if (r < out_f) y[r] = bias ? __fadd_rn(acc, bias[r]) : acc;
}

// The same sums for in_f % 4 == 0, DE_ROWS rows per workgroup. The whole
// workgroup stages K chunks of the rows' products w*x (each rounded, as the
// reference rounds it before adding) into LDS, double buffered, while lanes
// 0..DE_ROWS-1 of wave 0 add their rows' products in index order: one
// addition per value. A row's stride is 4 floats past a multiple of 32, so
// up to sixteen rows' 16-byte reads hit distinct banks. Each lane adds runs of 128
// products: the run's 32 reads go out, then its additions (runs of 32
// read a run ahead cost ~2x per addition: the compiler waited for every
// read in flight at the loop edge); a chunk's products past in_f are zeros
// (adding them changes nothing: the sum starts at +0.0 and never becomes
// -0.0).
constexpr int DE_K = 512, DE_RUN = 32;  // DE_RUN float4s per run
template <int DE_ROWS>
__global__ __launch_bounds__(256) void k_dense_exact_lds(const float* __restrict__ w,
                                                        const float* __restrict__ x,
                                                        const float* __restrict__ bias,
                                                        float* __restrict__ y, int out_f, int in_f)
{
    __shared__ __align__(16) float ws[2][DE_ROWS][DE_K + 4];
    const int r0 = blockIdx.x * DE_ROWS, t = threadIdx.x;
    const int nch = (in_f + DE_K - 1) / DE_K;
    constexpr int PER = DE_ROWS * DE_K / 4 / 256;  // 16-byte loads of W per thread and chunk
    float4 st[PER], xq[PER];
    auto load = [&](int c) {
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int idx = t + 256 * u, rr = idx / (DE_K / 4), k = c * DE_K + 4 * (idx % (DE_K / 4));
            const int row = min(r0 + rr, out_f - 1);
            const bool in = k < in_f;
            st[u] = in ? *reinterpret_cast<const float4*>(w + (size_t)row * in_f + k) : make_float4(0.f, 0.f, 0.f, 0.f);
            xq[u] = in ? *reinterpret_cast<const float4*>(x + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store = [&](int b) {
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int idx = t + 256 * u;
            const float4 p = make_float4(__fmul_rn(st[u].x, xq[u].x), __fmul_rn(st[u].y, xq[u].y),
                                         __fmul_rn(st[u].z, xq[u].z), __fmul_rn(st[u].w, xq[u].w));
            *reinterpret_cast<float4*>(&ws[b][idx / (DE_K / 4)][4 * (idx % (DE_K / 4))]) = p;
        }
    };
    load(0);
    store(0);
    __syncthreads();
    float acc = 0.0f;
    for (int c = 0; c < nch; c++) {
        const int b = c & 1;
        if (c + 1 < nch) load(c + 1);
        if (t < DE_ROWS) {
            // whole runs of 128 products: 32 reads out, then 128 additions
            const int len = min(DE_K, in_f - c * DE_K);
            const int nr = (len + 4 * DE_RUN - 1) / (4 * DE_RUN);
            const float4* pr = reinterpret_cast<const float4*>(&ws[b][t][0]);
            for (int g = 0; g < nr; g++) {
                float4 V[DE_RUN];
#pragma unroll
                for (int u = 0; u < DE_RUN; u++) V[u] = pr[g * DE_RUN + u];
#pragma unroll
                for (int u = 0; u < DE_RUN; u++) {
                    acc = __fadd_rn(acc, V[u].x);
                    acc = __fadd_rn(acc, V[u].y);
                    acc = __fadd_rn(acc, V[u].z);
                    acc = __fadd_rn(acc, V[u].w);
                }
            }
        }
        if (c + 1 < nch) store(b ^ 1);
        __syncthreads();
    }
    if (t < DE_ROWS && r0 + t < out_f) y[r0 + t] = bias ? __fadd_rn(acc, bias[r0 + t]) : acc;
}

// FAST: one workgroup of 4 waves per row, wave q taking the q-th quarter of
// it, 16-byte loads with every load of a pass issued before any is used,
// fixed-order tree sums (deterministic, not the reference's order). With nw
// set, x is RMSNorm'd on the fly (norm.rs:4-13): y = W (x * nw) /
// sqrt(mean(x^2) + eps), the sum of squares taken from the x the workgroup
// reads anyway. With x_add set, the input is x + x_add (a deferred K-slice
// of the GEMV that made x). (A wave per row and 4 rows per workgroup made
// each CU read 4 copies of x, nw and x_add besides its rows: 3.45 us for the
// 128 x 2048 router with x_add.)
__global__ __launch_bounds__(256) void k_dense_fast(const float* __restrict__ w,
                                                    const float* __restrict__ x,
                                                    const float* __restrict__ bias,
                                                    float* __restrict__ y, int out_f, int in_f,
                                                    const float* __restrict__ nw, float eps,
                                                    const float* __restrict__ x_add)
{
    __shared__ float red[2][4];
    // the wave index as a uniform value: read per lane it made the row
    // slices' buffer resources lane-varying, and every load a loop over lanes
    const int r = blockIdx.x, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const float* row = w + (size_t)r * in_f;
    float acc = 0.0f, sq = 0.0f;
    if ((in_f & 3) == 0) {
        // the wave's float4s [f0, f1) of the row; buffer loads over exactly
        // those bytes of the row, x, nw and x_add (past them zeros, no access)
        constexpr int DF_U = 2;  // float4s per lane per pass
        const int q4 = in_f / 4, per = (q4 + 3) / 4;
        const int f0 = min(q4, wave * per), nb = (min(q4, f0 + per) - f0) * 16;
        auto rs = [&](const float* p, int bytes) {
            return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, bytes, 0x00020000);
        };
        const auto wr = rs(row + 4 * f0, nb), xr = rs(x + 4 * f0, nb);
        const auto nr = rs(nw ? nw + 4 * f0 : x, nw ? nb : 0), ar = rs(x_add ? x_add + 4 * f0 : x, x_add ? nb : 0);
        for (int base = 0; base < per; base += 64 * DF_U) {
            float4 v[DF_U], u[DF_U], n4[DF_U], a4[DF_U];
#pragma unroll
            for (int q = 0; q < DF_U; q++) {
                const int off = (base + 64 * q + lane) * 16;
                v[q] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
                u[q] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
                if (nw) n4[q] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(nr, off, 0, 0));
                if (x_add) a4[q] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ar, off, 0, 0));
            }
#pragma unroll
            for (int q = 0; q < DF_U; q++) {
                float4 uq = u[q];
                if (x_add) {
                    uq.x += a4[q].x; uq.y += a4[q].y; uq.z += a4[q].z; uq.w += a4[q].w;
                }
                if (nw) {
                    sq = fmaf(uq.x, uq.x, sq); sq = fmaf(uq.y, uq.y, sq);
                    sq = fmaf(uq.z, uq.z, sq); sq = fmaf(uq.w, uq.w, sq);
                    uq.x *= n4[q].x; uq.y *= n4[q].y; uq.z *= n4[q].z; uq.w *= n4[q].w;
                }
                acc = fmaf(v[q].x, uq.x, acc);
                acc = fmaf(v[q].y, uq.y, acc);
                acc = fmaf(v[q].z, uq.z, acc);
                acc = fmaf(v[q].w, uq.w, acc);
            }
        }
    } else {
        for (int i = threadIdx.x; i < in_f; i += 256) {
            float u = x[i];
            if (x_add) u += x_add[i];
            if (nw) {
                sq = fmaf(u, u, sq);
                u *= nw[i];
            }
            acc = fmaf(row[i], u, acc);
        }
    }
    acc = wave_sum(acc);
    if (nw) sq = wave_sum(sq);
    if (lane == 0) {
        red[0][wave] = acc;
        red[1][wave] = sq;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float a = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
        if (nw) {
            const float s2 = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
            a *= __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(__fdiv_rn(s2, (float)in_f), eps)));
        }
        y[r] = bias ? a + bias[r] : a;
    }
}

// ---- softmax_inplace (wpc-runtime/src/norm.rs:28-43) ---------------------
// max (f32::max drops NaN like fmaxf; order-free), e_i = exp(x_i - max),
// sum in index order, then x_i = e_i / sum when sum > 0. One workgroup.
constexpr int SM_WG = 256;
__global__ __launch_bounds__(SM_WG) void k_softmax(float* __restrict__ x, int n)
{
    __shared__ float red[SM_WG / 64];
    __shared__ float s_sum;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += SM_WG) m = fmaxf(m, x[i]);
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int i = threadIdx.x; i < n; i += SM_WG) x[i] = ref_expf(__fsub_rn(x[i], m));
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (int i = 0; i < n; i++) s = __fadd_rn(s, x[i]);
        s_sum = s;
    }
    __syncthreads();
    const float s = s_sum;
    if (s > 0.0f)
        for (int i = threadIdx.x; i < n; i += SM_WG) x[i] = __fdiv_rn(x[i], s);
}

// ---- Qwen3MoeModel::route (qwen3_moe_model.rs:376-402) -------------------
// top_k strict-`>` scans: each takes the largest remaining value, the lowest
// index on ties, and never a NaN or -inf (`score > best` with best starting
// at -inf). With norm_topk the chosen weights are divided by their sum
// (taken in chosen order) when it is positive. Unfilled slots get id -1,
// weight 0. One wave; n <= 64*RT_PER.
__global__ __launch_bounds__(64) void k_route(const float* __restrict__ p, int n, int top_k,
                                              int norm_topk, int32_t* __restrict__ ids,
                                              float* __restrict__ w)
{
    const int lane = threadIdx.x;
    float v[RT_PER];
#pragma unroll
    for (int j = 0; j < RT_PER; j++) {
        const int i = lane + 64 * j;
        v[j] = i < n ? p[i] : -INFINITY;
        if (!(v[j] > -INFINITY)) v[j] = -INFINITY;  // NaN is never chosen
    }
    int got = 0;
    for (int k = 0; k < top_k; k++) {
        // best (value, index) of this lane, then of the wave
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < RT_PER; j++)
            if (v[j] > bv) { bv = v[j]; bi = lane + 64 * j; }
        wave_argmax(bv, bi);  // the scan of softmax_route_wave
        if (!(bv > -INFINITY)) break;  // nothing left to choose
#pragma unroll
        for (int j = 0; j < RT_PER; j++)
            if (lane + 64 * j == bi) v[j] = -INFINITY;
        if (lane == 0) { ids[k] = bi; w[k] = bv; }
        got = k + 1;
    }
    if (lane == 0) {
        for (int k = got; k < top_k; k++) { ids[k] = -1; w[k] = 0.0f; }
        if (norm_topk) {  // lane 0 rereads its own writes
            float s = 0.0f;
            for (int k = 0; k < got; k++) s = __fadd_rn(s, w[k]);
            if (s > 0.0f)
                for (int k = 0; k < got; k++) w[k] = __fdiv_rn(w[k], s);
        }
    }
}

// ---- softmax_inplace + route in one wave (the MoE router's tail) ----------
// Same arithmetic as k_softmax then k_route (softmax_route_wave).
__global__ __launch_bounds__(64) void k_softmax_route(const float* __restrict__ scores, int n,
                                                      int top_k, int norm_topk,
                                                      int32_t* __restrict__ ids,
                                                      float* __restrict__ w)
{
    __shared__ __align__(16) float e[64 * RT_PER];
    __shared__ double tab[32];
    // row blockIdx.x of a batch (one row: 0)
    softmax_route_wave(scores + (size_t)blockIdx.x * n, n, top_k, norm_topk, ids + (size_t)blockIdx.x * top_k,
                       w + (size_t)blockIdx.x * top_k, e, tab);
}

// ---- SiLU(g) * u (qwen3_moe_model.rs:518-522, model.rs:527-531) ----------
__global__ __launch_bounds__(256) void k_silu_mul(const float* __restrict__ g,
                                                  const float* __restrict__ u,
                                                  float* __restrict__ out, size_t n)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    const float silu = __fdiv_rn(gv, __fadd_rn(1.0f, ref_expf(-gv)));
    out[i] = __fmul_rn(silu, u[i]);
}

// ---- mlp_out = sum over chosen k of w_k * y_k (qwen3_moe_model.rs:526-528)
// in chosen order from 0; slots with id < 0 were never run.
// With `add`, out = add + that sum (residual[i] += mlp_out[i], :531-533).
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ ys,
                                                 const int32_t* __restrict__ ids,
                                                 const float* __restrict__ w, int top_k,
                                                 float* out, int h, const float* add)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= h) return;
    float acc = 0.0f;
    for (int k = 0; k < top_k; k++)
        if (ids[k] >= 0) acc = __fadd_rn(acc, __fmul_rn(w[k], ys[(size_t)k * h + i]));
    out[i] = add ? __fadd_rn(add[i], acc) : acc;
}

}  // namespace

// Rows per workgroup of the EXACT router: two rows, 64 workgroups for 128
// experts, spread the row loads over more CUs than sixteen rows did (each
// row's index-order chain is the same length either way): EXACT
// Qwen3-30B-A3B-shaped decode 212.1 -> 214.2 tok/s (4 rows: 213.6).
constexpr int DE_ROWS_L = 2;
hipError_t launch_dense(const float* w, int out_f, int in_f, int mode, const float* x,
                        const float* bias, float* y, hipStream_t s, const float* nw, float eps,
                        const float* x_add)
{
    (void)hipGetLastError();
    if (mode == WPCG_MODE_EXACT) {
        if (nw || x_add) return hipErrorInvalidValue;  // EXACT normalises in its own launch
        if (in_f % 4 == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0)
            hipLaunchKernelGGL(k_dense_exact_lds<DE_ROWS_L>, dim3((out_f + DE_ROWS_L - 1) / DE_ROWS_L), dim3(256), 0,
                               s, w, x, bias, y, out_f, in_f);
        else
            hipLaunchKernelGGL(k_dense_exact, dim3((out_f + 63) / 64), dim3(64), 0, s, w, x, bias, y,
                               out_f, in_f);
    } else {
        hipLaunchKernelGGL(k_dense_fast, dim3(out_f), dim3(256), 0, s, w, x, bias, y,
                           out_f, in_f, nw, eps, x_add);
    }
    return hipGetLastError();
}

hipError_t launch_softmax(float* x, int n, hipStream_t s)
{
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_softmax, dim3(1), dim3(SM_WG), 0, s, x, n);
    return hipGetLastError();
}

int route_max_n() { return 64 * RT_PER; }

hipError_t launch_route(const float* p, int n, int top_k, int norm_topk, int32_t* ids, float* w,
                        hipStream_t s)
{
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_route, dim3(1), dim3(64), 0, s, p, n, top_k, norm_topk, ids, w);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float* g, const float* u, float* out, size_t n, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, out, n);
    return hipGetLastError();
}

hipError_t launch_combine(const float* ys, const int32_t* ids, const float* w, int top_k,
                          float* out, int h, const float* add, hipStream_t s)
{
    if (h == 0) return hipSuccess;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_combine, dim3((h + 255) / 256), dim3(256), 0, s, ys, ids, w, top_k, out, h, add);
    return hipGetLastError();
}

hipError_t launch_softmax_route(const float* scores, int n, int top_k, int norm_topk, int32_t* ids,
                                float* w, hipStream_t s)
{
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_softmax_route, dim3(1), dim3(64), 0, s, scores, n, top_k, norm_topk, ids, w);
    return hipGetLastError();
}

}  // namespace wpcg
