// Kernels of the device-resident decode step: one token through the dense
// Qwen3 / Qwen3-MoE decoder (Model::forward_token, model.rs:419-547;
// Qwen3MoeModel::forward_token, qwen3_moe_model.rs:406-542) without leaving
// the GPU. The position and the input token live in device memory
// (DecodeState, tokens[]), so one step is a fixed sequence of launches that
// a HIP graph can replay token after token; the argmax at the end writes
// the next input token.
//
// EXACT mode reproduces the reference's fp32 arithmetic operation for
// operation (index-order sums, products and sums rounded separately, libm
// exp via ref_expf.h, correctly rounded division and square root). FAST
// mode keeps every elementwise step but takes long sums (the RMSNorm over
// the hidden size) as fixed-order trees.
#include <hip/hip_runtime.h>

#define REF_EXPF_FN __device__ __forceinline__
#include "ref_expf.h"
#include "wpcg_internal.hpp"
#include "wave.h"
#include "xpack.h"

namespace wpcg {
namespace {

// Correctly rounded square root (IEEE, as f32::sqrt): the plain builtin
// expands to the hardware estimate plus a rounding fixup; __fsqrt_rn, without
// OCML's rounded-operation mode, is the bare estimate (up to 1 ulp off).
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }

// A buffer resource over [base, base + bytes): loads past the end return
// zeros without touching memory.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// ---- rms_norm (wpc-runtime/src/norm.rs:4-13) -------------------------------
// mean_sq = (sum x_i^2) / n; scale = 1 / sqrt(mean_sq + eps);
// out_i = x_i * scale * w_i. One workgroup of NW threads.
constexpr int NW = 256;

// ((0 + v0^2) + v1^2) + ... in index order with separate roundings, by one
// thread. The next sixteen values are requested (clamped in bounds, no
// branch) before the current sixteen are added, so the load latency hides
// behind the chain of additions.
__device__ __forceinline__ float ordered_sumsq(const float* v, int n)
{
    float s = 0.0f;
    if (((uintptr_t)v & 15) != 0) {
        for (int i = 0; i < n; i++) s = __fadd_rn(s, __fmul_rn(v[i], v[i]));
        return s;
    }
    const float4* v4 = reinterpret_cast<const float4*>(v);
    const int n4 = n >> 2, nfull = n4 & ~3;  // float4s in whole groups of four
    if (nfull) {
        float4 cur[4];
#pragma unroll
        for (int u = 0; u < 4; u++) cur[u] = v4[u];
        for (int c = 0; c < nfull; c += 4) {
            float4 nxt[4];
#pragma unroll
            for (int u = 0; u < 4; u++) nxt[u] = v4[min(c + 4 + u, n4 - 1)];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                s = __fadd_rn(s, __fmul_rn(cur[u].x, cur[u].x));
                s = __fadd_rn(s, __fmul_rn(cur[u].y, cur[u].y));
                s = __fadd_rn(s, __fmul_rn(cur[u].z, cur[u].z));
                s = __fadd_rn(s, __fmul_rn(cur[u].w, cur[u].w));
            }
#pragma unroll
            for (int u = 0; u < 4; u++) cur[u] = nxt[u];
        }
    }
    for (int i = nfull * 4; i < n; i++) s = __fadd_rn(s, __fmul_rn(v[i], v[i]));
    return s;
}

// ((0 + q0) + q1) + ... in index order, by one thread, from 16-byte aligned
// LDS (q = the squares, rounded, already computed by the whole workgroup and
// padded with +0.0 to os_padded(n) values: adding +0.0 to the sum, which
// starts at +0.0 and never becomes -0.0, changes nothing). The chain is one
// addition per value, in chunks of 128: a chunk's 32 16-byte reads all go
// out, then its 128 additions run as the reads return. (Groups of 32 values
// read a group ahead measured 10-13 clocks per addition on one lane: the
// compiler copies the look-ahead registers at the loop edge and waits for
// every read there; whole chunks of 128 run at ~7, a chain from registers
// at ~4.6.)
constexpr int OS_CHUNK = 32;  // float4s per chunk
__device__ __forceinline__ int os_padded(int n) { return (n + 4 * OS_CHUNK - 1) / (4 * OS_CHUNK) * (4 * OS_CHUNK); }
__device__ __forceinline__ float ordered_sum_lds(const float* q, int n)
{
    const float4* q4 = reinterpret_cast<const float4*>(q);
    const int nc = os_padded(n) / (4 * OS_CHUNK);
    float s = 0.0f;
    for (int c = 0; c < nc; c++) {
        float4 v[OS_CHUNK];
#pragma unroll
        for (int u = 0; u < OS_CHUNK; u++) v[u] = q4[c * OS_CHUNK + u];
#pragma unroll
        for (int u = 0; u < OS_CHUNK; u++) {
            s = __fadd_rn(s, v[u].x);
            s = __fadd_rn(s, v[u].y);
            s = __fadd_rn(s, v[u].z);
            s = __fadd_rn(s, v[u].w);
        }
    }
    return s;
}

// EXACT: the workgroup stores every square (rounded) into LDS, zero padded,
// and one thread adds them in index order (n <= 256).
template <int MODE>
__device__ float sum_squares(const float* x, int n, float* red)
{
    __shared__ float s_total;
    __shared__ __align__(16) float s_sq[MODE == WPCG_MODE_EXACT ? 256 : 4];
    if (MODE == WPCG_MODE_EXACT) {
        for (int i = threadIdx.x; i < os_padded(n); i += blockDim.x)
            s_sq[i] = i < n ? __fmul_rn(x[i], x[i]) : 0.0f;
        __syncthreads();
        if (threadIdx.x == 0) s_total = ordered_sum_lds(s_sq, n);
    } else {
        float s = 0.0f;
        for (int i = threadIdx.x; i < n; i += blockDim.x) s = fmaf(x[i], x[i], s);
        s = wave_sum(s);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
        __syncthreads();
        if (threadIdx.x == 0) {
            float t = 0.0f;
            for (int w = 0; w < (int)(blockDim.x >> 6); w++) t += red[w];
            s_total = t;
        }
    }
    __syncthreads();
    return s_total;
}

// x is staged in LDS once (n <= RN_LDS; longer vectors are read from global
// memory twice). EXACT: the workgroup also stores every square (rounded) in
// LDS, and one thread adds them in index order; FAST: a tree from registers.
constexpr int RN_LDS = 8192;
template <int MODE>
__global__ __launch_bounds__(NW) void k_rms_norm(const float* __restrict__ x,
                                                 const float* __restrict__ w, int n, float eps,
                                                 float* __restrict__ out)
{
    x += (size_t)blockIdx.x * n;  // row blockIdx.x of a batch (one row: 0)
    out += (size_t)blockIdx.x * n;
    __shared__ __align__(16) float xs[RN_LDS];
    // the squares, padded with zeros to a multiple of 64 and one group past
    // that (the chain reads one group ahead)
    __shared__ __align__(16) float sq[MODE == WPCG_MODE_EXACT ? RN_LDS : 4];
    __shared__ float red[NW / 64];
    __shared__ float s_total;
    const bool staged = n <= RN_LDS;
    const float* src = staged ? xs : x;
    if (MODE == WPCG_MODE_EXACT && staged && (n & 3) == 0) {
        // every 16-byte load of x and of the weights first (range-checked,
        // none past n), the squares into LDS, x kept in registers for the
        // output: one memory round trip before the ordered chain
        constexpr int V = RN_LDS / 4 / NW;
        typedef float f4 __attribute__((ext_vector_type(4)));
        const auto xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), (short)0, n * 4, 0x00020000);
        const auto wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(w), (short)0, n * 4, 0x00020000);
        f4 xv[V], wv[V];
#pragma unroll
        for (int u = 0; u < V; u++) {
            xv[u] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(xr, (threadIdx.x + u * NW) * 16, 0, 0));
            wv[u] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(wr, (threadIdx.x + u * NW) * 16, 0, 0));
        }
#pragma unroll
        for (int u = 0; u < V; u++) {
            const int i = 4 * (threadIdx.x + u * NW);
            if (i < n) {
                const f4 v = xv[u];
                *reinterpret_cast<f4*>(&sq[i]) = f4{__fmul_rn(v.x, v.x), __fmul_rn(v.y, v.y),
                                                    __fmul_rn(v.z, v.z), __fmul_rn(v.w, v.w)};
            }
        }
        for (int i = n + threadIdx.x; i < os_padded(n); i += NW) sq[i] = 0.0f;
        __syncthreads();
        if (threadIdx.x == 0) s_total = ordered_sum_lds(sq, n);
        __syncthreads();
        const float mean_sq = __fdiv_rn(s_total, (float)n);
        const float scale = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(mean_sq, eps)));
#pragma unroll
        for (int u = 0; u < V; u++) {
            const int i = 4 * (threadIdx.x + u * NW);
            if (i < n) {
                out[i] = __fmul_rn(__fmul_rn(xv[u].x, scale), wv[u].x);
                out[i + 1] = __fmul_rn(__fmul_rn(xv[u].y, scale), wv[u].y);
                out[i + 2] = __fmul_rn(__fmul_rn(xv[u].z, scale), wv[u].z);
                out[i + 3] = __fmul_rn(__fmul_rn(xv[u].w, scale), wv[u].w);
            }
        }
        return;
    }
    float part = 0.0f;
    for (int i = threadIdx.x; i < n; i += NW) {
        const float v = x[i];
        if (staged) {
            xs[i] = v;
            if (MODE == WPCG_MODE_EXACT) sq[i] = __fmul_rn(v, v);
        }
        part = fmaf(v, v, part);
    }
    if (MODE == WPCG_MODE_EXACT) {
        if (staged)
            for (int i = n + threadIdx.x; i < os_padded(n); i += NW) sq[i] = 0.0f;
        __syncthreads();
        if (threadIdx.x == 0) s_total = staged ? ordered_sum_lds(sq, n) : ordered_sumsq(x, n);
    } else {
        part = wave_sum(part);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = part;
        __syncthreads();
        if (threadIdx.x == 0) s_total = (red[0] + red[1]) + (red[2] + red[3]);
    }
    __syncthreads();
    const float mean_sq = __fdiv_rn(s_total, (float)n);
    const float scale = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(mean_sq, eps)));
    for (int i = threadIdx.x; i < n; i += NW) out[i] = __fmul_rn(__fmul_rn(src[i], scale), w[i]);
}

// ---- attention step (model.rs:441-497) -------------------------------------
// One workgroup per query head h (kv head j = h / (nh/nkv)), all in one
// launch:
//   q_h, k_j: RMSNorm with q_norm / k_norm, then RoPE at `pos`
//     (rope.rs:24-39: out_i = x1*c - x2*s, out_{i+d/2} = x2*c + x1*s with c, s
//     the f32 casts of the host's f64 cos/sin, cos_t/sin_t [pos][d/2]);
//   the first query head of kv head j appends k_j and v_j to the caches;
//   scores_t = (sum_d q_h[d] * k_t[d]) * scale for t <= pos (k_pos taken from
//     LDS, earlier positions from the cache), softmax over them (norm.rs:28-43);
//   out_h[d] = sum_t w_t * v_t[d] in position order.
// Every workgroup recomputes k_j and v_j for `pos` itself, so no workgroup
// waits for another's cache write. Caches are [kv_head][max_pos][head_dim]
// of one layer. EXACT: index-order sums, separate roundings; FAST: fused
// multiply-adds and tree sums. head_dim <= 256, pos < max_pos <= AT_MAXPOS.
// 512 threads: at positions up to 512 every thread takes one position's
// score (with 256, two in turn, the second row's loads after the first
// row's chain): EXACT Qwen3-30B-A3B-shaped decode at positions 256..511
// 214 -> 220 tok/s
constexpr int AT_WG = 512;
constexpr int AT_MAXPOS = 4096;
constexpr int AT_VB = 32;  // value rows per LDS block of the output step
constexpr int AT_VD = 4;   // value blocks whose loads are in flight at once

template <int MODE>
__device__ void head_rms_rope(const float* x, const float* w, float* y, float* red, int hd,
                              float eps, const float* c, const float* sn)
{
    __shared__ float s_tmp[256];
    const float s = sum_squares<MODE>(x, hd, red);
    const float mean_sq = __fdiv_rn(s, (float)hd);
    const float scale = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(mean_sq, eps)));
    for (int i = threadIdx.x; i < hd; i += blockDim.x) s_tmp[i] = __fmul_rn(__fmul_rn(x[i], scale), w[i]);
    __syncthreads();
    const int half = hd / 2;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float x1 = s_tmp[i], x2 = s_tmp[i + half];
        y[i] = __fsub_rn(__fmul_rn(x1, c[i]), __fmul_rn(x2, sn[i]));
        y[i + half] = __fadd_rn(__fmul_rn(x2, c[i]), __fmul_rn(x1, sn[i]));
    }
    __syncthreads();
}

// EXACT q and k head norms + RoPE together: the two index-order sums of
// squares run at once, on lanes of different waves (one after the other,
// each was a chain behind two barriers).
__device__ void head_rms_rope_qk_exact(const float* xq, const float* wq, float* yq, const float* xk,
                                       const float* wk, float* yk, int hd, float eps, const float* c,
                                       const float* sn)
{
    __shared__ __align__(16) float sq[2][256];
    __shared__ float s_tot[2];
    __shared__ float s_tmp[2][256];
    for (int i = threadIdx.x; i < os_padded(hd); i += blockDim.x) {
        sq[0][i] = i < hd ? __fmul_rn(xq[i], xq[i]) : 0.0f;
        sq[1][i] = i < hd ? __fmul_rn(xk[i], xk[i]) : 0.0f;
    }
    __syncthreads();
    if (threadIdx.x == 0) s_tot[0] = ordered_sum_lds(sq[0], hd);
    if (threadIdx.x == 64) s_tot[1] = ordered_sum_lds(sq[1], hd);
    __syncthreads();
    const float scq = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(s_tot[0], (float)hd), eps)));
    const float sck = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(s_tot[1], (float)hd), eps)));
    for (int i = threadIdx.x; i < hd; i += blockDim.x) {
        s_tmp[0][i] = __fmul_rn(__fmul_rn(xq[i], scq), wq[i]);
        s_tmp[1][i] = __fmul_rn(__fmul_rn(xk[i], sck), wk[i]);
    }
    __syncthreads();
    const int half = hd / 2;
    for (int i = threadIdx.x; i < 2 * half; i += blockDim.x) {
        const int r = i / half, e = i - r * half;
        float* y = r ? yk : yq;
        const float x1 = s_tmp[r][e], x2 = s_tmp[r][e + half];
        y[e] = __fsub_rn(__fmul_rn(x1, c[e]), __fmul_rn(x2, sn[e]));
        y[e + half] = __fadd_rn(__fmul_rn(x2, c[e]), __fmul_rn(x1, sn[e]));
    }
    __syncthreads();
}

template <int MODE>
__global__ __launch_bounds__(AT_WG) void k_attention(const float* __restrict__ qp,
                                                     const float* __restrict__ kp,
                                                     const float* __restrict__ vp,
                                                     const float* __restrict__ qn,
                                                     const float* __restrict__ kn, int nh, int nkv,
                                                     int hd, float eps, float scale,
                                                     const float* __restrict__ cos_t,
                                                     const float* __restrict__ sin_t,
                                                     const DecodeState* __restrict__ st,
                                                     float* __restrict__ kc, float* __restrict__ vc,
                                                     float* __restrict__ out)
{
    __shared__ __align__(16) float qs[256], ks[256], vs[256];
    __shared__ __align__(16) float w[AT_MAXPOS + 128];  // zero padded for the ordered sum
    __shared__ __align__(16) float vsh[2][AT_VB * 256];
    __shared__ float red[AT_WG / 64];
    __shared__ float s_sum;
    const int h = blockIdx.x, n_rep = nh / nkv, j = h / n_rep;
    const uint32_t pos = st->pos, max_pos = st->max_pos;
    const int half = hd / 2;
    const float* c = cos_t + (size_t)pos * half;
    const float* sn = sin_t + (size_t)pos * half;
    if constexpr (MODE == WPCG_MODE_EXACT) {
        head_rms_rope_qk_exact(qp + (size_t)h * hd, qn, qs, kp + (size_t)j * hd, kn, ks, hd, eps, c, sn);
    } else {
        head_rms_rope<MODE>(qp + (size_t)h * hd, qn, qs, red, hd, eps, c, sn);
        head_rms_rope<MODE>(kp + (size_t)j * hd, kn, ks, red, hd, eps, c, sn);
    }
    for (int i = threadIdx.x; i < hd; i += AT_WG) vs[i] = vp[(size_t)j * hd + i];
    __syncthreads();
    const float* kb = kc + (size_t)j * max_pos * hd;
    const float* vb = vc + (size_t)j * max_pos * hd;
    // The cached value rows (t < pos) for the output step: blocks of AT_VB
    // positions, AT_VD of them in flight in registers; the first AT_VD are
    // requested here, before this workgroup's cache write (row pos, which
    // no block reads), so they arrive during the scores and the softmax.
    const int nv = (int)pos, nblk = (nv + AT_VB - 1) / AT_VB, f4 = AT_VB * hd / 4;
    constexpr int VPER = AT_VB * 256 / 4 / AT_WG;  // float4s per thread per block (hd <= 256)
    // Every block issues VPER range-checked loads per thread, so the count
    // in flight is fixed and each wait is for one block only: rows t >= pos,
    // blocks past the last and lanes past the block's f4 float4s read zeros
    // (their offsets are out of range, which moves no data).
    const auto vrs = buf_rsrc(vb, nv * hd * 4);
    u32x4 vr[AT_VD][VPER];
    auto vload = [&](int bk, u32x4(&r)[VPER]) {
#pragma unroll
        for (int u = 0; u < VPER; u++) {
            const int i = threadIdx.x + u * AT_WG;  // float4 of the block
            r[u] = __builtin_amdgcn_raw_buffer_load_b128(vrs, i < f4 ? (bk * AT_VB * hd + 4 * i) * 4 : 0x7ffffff0,
                                                         0, 0);
        }
    };
#pragma unroll
    for (int r = 0; r < AT_VD; r++) vload(r, vr[r]);
    if (h % n_rep == 0)
        for (int i = threadIdx.x; i < hd; i += AT_WG) {
            kc[((size_t)j * max_pos + pos) * hd + i] = ks[i];
            vc[((size_t)j * max_pos + pos) * hd + i] = vs[i];
        }
    // scores: thread t, one position at a time; a row's 128-value halves
    // read with all their 16-byte loads issued before the dot's chain
    const int n = (int)pos + 1;
    for (int t = threadIdx.x; t < n; t += AT_WG) {
        const float* kt = t == (int)pos ? ks : kb + (size_t)t * hd;
        float dot = 0.0f;
        for (int d0 = 0; d0 < hd; d0 += 128) {
            float4 kv[32];
#pragma unroll
            for (int u = 0; u < 32; u++)
                kv[u] = d0 + 4 * u < hd ? *reinterpret_cast<const float4*>(kt + d0 + 4 * u)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int u = 0; u < 32; u++) {
                if (d0 + 4 * u >= hd) break;  // uniform
                const float* q4 = qs + d0 + 4 * u;
                if (MODE == WPCG_MODE_EXACT) {
                    dot = __fadd_rn(dot, __fmul_rn(q4[0], kv[u].x));
                    dot = __fadd_rn(dot, __fmul_rn(q4[1], kv[u].y));
                    dot = __fadd_rn(dot, __fmul_rn(q4[2], kv[u].z));
                    dot = __fadd_rn(dot, __fmul_rn(q4[3], kv[u].w));
                } else {
                    dot = fmaf(q4[0], kv[u].x, dot);
                    dot = fmaf(q4[1], kv[u].y, dot);
                    dot = fmaf(q4[2], kv[u].z, dot);
                    dot = fmaf(q4[3], kv[u].w, dot);
                }
            }
        }
        w[t] = __fmul_rn(dot, scale);
    }
    __syncthreads();
    // softmax over w[0..n)
    float m = -INFINITY;
    for (int t = threadIdx.x; t < n; t += AT_WG) m = fmaxf(m, w[t]);
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int q = 1; q < AT_WG / 64; q++) m = fmaxf(m, red[q]);
    for (int t = threadIdx.x; t < n; t += AT_WG) w[t] = ref_expf(__fsub_rn(w[t], m));
    __syncthreads();
    if (MODE == WPCG_MODE_EXACT) {
        for (int t = n + threadIdx.x; t < os_padded(n); t += AT_WG) w[t] = 0.0f;
        __syncthreads();
        if (threadIdx.x == 0) s_sum = ordered_sum_lds(w, n);
    } else {
        float s = 0.0f;
        for (int t = threadIdx.x; t < n; t += AT_WG) s += w[t];
        s = wave_sum(s);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
        __syncthreads();
        if (threadIdx.x == 0) {  // a fixed order
            float t = red[0];
#pragma unroll
            for (int q = 1; q < AT_WG / 64; q++) t += red[q];
            s_sum = t;
        }
    }
    __syncthreads();
    const float ssum = s_sum;
    if (ssum > 0.0f)
        for (int t = threadIdx.x; t < n; t += AT_WG) w[t] = __fdiv_rn(w[t], ssum);
    __syncthreads();
    // out[d] = sum_t w_t v_t[d], position order; thread d. The value blocks
    // pass from the register ring through LDS, double buffered: block bk is
    // read from LDS while block bk + 1 is stored there and the loads of
    // block bk + AT_VD take the registers block bk held; t = pos comes
    // from vs.
    auto vstore = [&](int b, const u32x4(&r)[VPER]) {
#pragma unroll
        for (int u = 0; u < VPER; u++) {
            const int i = threadIdx.x + u * AT_WG;
            if (i < f4) *reinterpret_cast<u32x4*>(&vsh[b][4 * i]) = r[u];
        }
    };
    const int d = threadIdx.x;
    float acc = 0.0f;
    auto step = [&](float wt, float v) {
        acc = MODE == WPCG_MODE_EXACT ? __fadd_rn(acc, __fmul_rn(wt, v)) : fmaf(wt, v, acc);
    };
    if (nblk > 0) vstore(0, vr[0]);
    __syncthreads();
    for (int bk0 = 0; bk0 < nblk; bk0 += AT_VD) {
#pragma unroll
        for (int r = 0; r < AT_VD; r++) {  // block bk sits in vr[r], so the ring index is static
            const int bk = bk0 + r;
            if (bk >= nblk) break;  // uniform
            const int b = bk & 1, t0 = bk * AT_VB;
            vload(bk + AT_VD, vr[r]);
            if (d < hd) {
                if (t0 + AT_VB <= nv) {
#pragma unroll
                    for (int u = 0; u < AT_VB; u++) step(w[t0 + u], vsh[b][u * hd + d]);
                } else {
                    for (int u = 0; u < nv - t0; u++) step(w[t0 + u], vsh[b][u * hd + d]);
                }
            }
            if (bk + 1 < nblk) vstore(b ^ 1, vr[(r + 1) % AT_VD]);
            __syncthreads();
        }
    }
    if (d < hd) {
        step(w[pos], vs[d]);
        out[(size_t)h * hd + d] = acc;
    }
}

// ---- FAST attention step: positions split into chunks across workgroups ----
// Workgroup (j, c) takes kv head j's query heads (n_rep = nh/nkv of them)
// over chunk c of the n = pos + 1 positions: positions are dealt round
// robin, chunk c holding positions c, c + FA_NCH, c + 2 FA_NCH, ..., taken
// FA_C at a time as blocks (block b: positions c + FA_NCH (FA_C b + t),
// t < FA_C). The launch has a fixed shape (a HIP graph replays it at every
// position), no chunk holds more than ceil(n / FA_NCH) positions (the
// launch takes as long as its fullest chunk), and a chunk's first block
// does not depend on the position: its keys and values can be requested at
// entry, with the query rows, before the position is known (each row is
// one contiguous head_dim vector; see the FD_WG note below). The chunk's
// keys and values pass through LDS one block at a time,
// shared by all n_rep heads (the next block's loads are in flight while
// the current one is used), with a running (online) softmax: max m,
// sum l of exp(s - m), o = sum exp(s_t - m) v_t. Each workgroup applies
// q_norm + RoPE to its heads itself, with the step's RoPE row (cos, sin at
// the position, copied to a fixed buffer by the step's embedding launch);
// the chunk that holds `pos` computes the current key (k_norm + RoPE) and
// value and appends them to the caches. Each chunk leaves its state for
// the o_proj GEMV, which merges the chunks as it reads its input
// (attention_merge, XF_MERGE): o at part_o[c][h][d], (m, l) at
// part_ml[c][h][0..1], h the query head. Sums are fixed-order trees and
// fused multiply-adds: deterministic, not the reference's operation order.
// head_dim HD is 64 or 128, n_rep <= FA_MAXREP.
constexpr int FA_C = 32;
constexpr int FA_NCH = ATTN_CHUNKS;
constexpr int FA_MAXREP = 16;

// RMSNorm of one head row (w) then RoPE at the current position, by one
// wave: lane l < HD/2 holds elements l and l + HD/2, which are exactly the
// pair RoPE rotates. The result goes to y (LDS) and, if set, to g (global).
template <int HD>
__device__ __forceinline__ void fa_norm_rope(const float* x, const float* w, float eps, const float* c,
                                             const float* sn, float* y, float* g)
{
    constexpr int half = HD / 2;
    const int lane = threadIdx.x & 63;
    const bool on = lane < half;
    const float x1 = on ? x[lane] : 0.0f, x2 = on ? x[lane + half] : 0.0f;
    const float ss = wave_sum(fmaf(x1, x1, x2 * x2));
    const float scale = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)HD), eps)));
    if (on) {
        const float y1 = (x1 * scale) * w[lane], y2 = (x2 * scale) * w[lane + half];
        const float o1 = fmaf(y1, c[lane], -(y2 * sn[lane])), o2 = fmaf(y2, c[lane], y1 * sn[lane]);
        y[lane] = o1;
        y[lane + half] = o2;
        if (g) {
            g[lane] = o1;
            g[lane + half] = o2;
        }
    }
}

// FD_WG threads: 256, or 512 for at most 4 query heads per key head (two
// waves per SIMD instead of one; dense Qwen3-4B decode 694 -> 722 tok/s,
// while 8 heads per key head, Qwen3-30B-A3B, ran 1.5% slower at 512).
// The 256-thread launch requests its first block of keys and values before
// the position is known, every row of it (Qwen3-30B-A3B shape: 6.69 ->
// 6.34 us per launch); the 512-thread launch, with twice the key heads per
// query head and so twice the bytes per speculated row, requests only the
// rows before the position, once it is known (speculating took the dense
// Qwen3-4B-shaped launch from 5.21 to 5.42 us).
template <int HD, int FD_WG>
__global__ __launch_bounds__(FD_WG) void k_attention_fast(const float* __restrict__ qp,
                                                          const float* __restrict__ kp,
                                                          const float* __restrict__ vp,
                                                          const float* __restrict__ qn,
                                                          const float* __restrict__ kn, int nh, int nkv,
                                                          float eps, float scale,
                                                          const float* __restrict__ rope, int cache_pos,
                                                          const DecodeState* __restrict__ st,
                                                          float* __restrict__ kc, float* __restrict__ vc,
                                                          float* __restrict__ part_o, float* __restrict__ part_ml)
{
    constexpr int HD4 = HD / 4, KS = HD + 4;  // KS: key rows 16-byte aligned, offset by 4 banks
    constexpr int NOUT = FA_MAXREP * HD / FD_WG;   // outputs per thread
    constexpr int G = FD_WG / HD;                  // thread groups over head_dim
    constexpr int NKV = FA_C * HD4 / FD_WG;        // 16-byte key (and value) loads per thread and block
    __shared__ __align__(16) float qs[FA_MAXREP][HD];
    __shared__ __align__(16) float ks[FA_C][KS];
    __shared__ __align__(16) float vs[FA_C][HD];
    __shared__ __align__(16) float kcur[HD], vcur[HD];
    __shared__ float ps[FA_MAXREP][FA_C];                     // scores, head-major
    __shared__ __align__(16) float pt[FA_C][FA_MAXREP + 4];   // exp weights, position-major
    __shared__ float s_m[FA_MAXREP], s_l[FA_MAXREP], s_corr[FA_MAXREP];
    // every argument the loads below need, in one round trip (each read
    // where it is first used was a further dependent round trip)
    asm volatile("" ::"s"(qp), "s"(kp), "s"(vp), "s"(qn), "s"(kn), "s"(nh), "s"(nkv), "s"(rope), "s"(cache_pos),
                 "s"(st), "s"(kc), "s"(vc));
    const int j = blockIdx.x / FA_NCH, c = blockIdx.x % FA_NCH;
    const int n_rep = nh / nkv;
    // row t of this chunk's block b is position base(b) + FA_NCH t
    auto base = [&](int b) { return c + b * FA_C * FA_NCH; };
    auto row_pos = [&](int b, int t) { return base(b) + t * FA_NCH; };
    float* kb = kc + (size_t)j * cache_pos * HD;
    float* vb = vc + (size_t)j * cache_pos * HD;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;

    // The state (pos, n_prompt, max_pos, last), loaded first and through the
    // constant address space (nothing in the launch writes it), which lets
    // the compiler issue the loads below before using it: the test on the
    // position then waits for this load alone (vector loads return in
    // order). Read as an ordinary load, the compiler waited for it before
    // issuing any other.
    typedef const __attribute__((address_space(4))) u32x4* StatePtr;
    const u32x4 sv = *(StatePtr)st;
    // q heads (and the current key and value, in the chunk that holds pos):
    // wave w takes rows r = w, w + 4, ... (row n_rep is the key). Every load
    // of the wave's rows, the norm weights and the step's RoPE row is issued
    // before any is used (one memory round trip, in parallel with the
    // position's), then each row is RMS-normalised and rotated as
    // fa_norm_rope does it. These go out before the cached keys and values,
    // which vector loads return in order after them.
    constexpr int half = HD / 2, NWV = FD_WG / 64;
    constexpr int RW = (FA_MAXREP + NWV) / NWV;  // rows per wave at most
    const bool on = lane < half;
    const int li = on ? lane : 0;  // every address in bounds; off lanes' values are discarded
    float x1[RW], x2[RW];
#pragma unroll
    for (int i = 0; i < RW; i++) {
        const int r = wave + i * NWV;
        const float* src = r < n_rep ? qp + (size_t)(j * n_rep + r) * HD : kp + (size_t)j * HD;
        x1[i] = src[li];
        x2[i] = src[li + half];
    }
    const float c1 = rope[li], s1 = rope[half + li];
    const float qw1 = qn[li], qw2 = qn[li + half], kw1 = kn[li], kw2 = kn[li + half];
    float vv[HD / 64];
#pragma unroll
    for (int u = 0; u < HD / 64; u++) vv[u] = vp[(size_t)j * HD + lane + 64 * u];

    // A block's cached keys and values, rows t < lim: thread i, 16 bytes of
    // row i / HD4, through buffer loads over this head's cache, so that every
    // load may be unconditional: a row at or past lim gets an offset past
    // the range and reads zeros without a memory access, as does a row past
    // the cache; a speculated row past the step's position is read and never
    // used (the scores and the output take rows t < nt only); the current
    // position's row comes from kcur / vcur.
    constexpr bool SPEC = FD_WG == 256;
    const auto krs = buf_rsrc(kb, cache_pos * HD * 4), vrs = buf_rsrc(vb, cache_pos * HD * 4);
    u32x4 kr[NKV], vr[NKV];
    auto load_block = [&](int b, int lim) {
#pragma unroll
        for (int u = 0; u < NKV; u++) {
            const int i = threadIdx.x + u * FD_WG, t = i / HD4;
            const int off = t < lim ? (row_pos(b, t) * HD + 4 * (i % HD4)) * 4 : 0x40000000;
            kr[u] = __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0);
            vr[u] = __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0);
        }
    };
    if constexpr (SPEC) load_block(0, FA_C);

    const uint32_t pos = sv.x, max_pos = sv.z;
    const int n = (int)pos + 1;
    if ((c >= n) | (pos >= max_pos) | (pos >= (uint32_t)cache_pos)) {
        // An empty chunk leaves the neutral state (m = -inf, l = 0, o = 0),
        // so the merge in o_proj takes every chunk without knowing the
        // position: an empty chunk's weight exp(-inf - M) is 0. (Past the
        // cache, pos >= max_pos, every chunk is empty and chunk 0 leaves
        // m = 0, l = 1: the merged output is 0 rather than 0/0.)
        // The loads above are consumed here too (their bits into an empty
        // asm operand): with uses on both sides of this branch they stay
        // ahead of it; used on one side only, the compiler moved them into
        // the non-empty path, behind the position's round trip.
        uint32_t used = 0;
        if constexpr (SPEC) {
#pragma unroll
            for (int u = 0; u < NKV; u++) used |= kr[u].x | vr[u].x;
        }
#pragma unroll
        for (int i = 0; i < RW; i++) used |= __float_as_uint(x1[i]) | __float_as_uint(x2[i]);
#pragma unroll
        for (int u = 0; u < HD / 64; u++) used |= __float_as_uint(vv[u]);
        used |= __float_as_uint(c1) | __float_as_uint(s1) | __float_as_uint(qw1) | __float_as_uint(qw2) |
                __float_as_uint(kw1) | __float_as_uint(kw2);
        asm volatile("" ::"v"(used));
        const bool unit = c == 0;
        for (int i = threadIdx.x; i < n_rep * HD; i += FD_WG)
            part_o[((size_t)c * nh + j * n_rep) * HD + i] = 0.0f;
        if ((int)threadIdx.x < 2 * n_rep)
            part_ml[((size_t)c * nh + j * n_rep) * 2 + threadIdx.x] =
                (threadIdx.x & 1) ? (unit ? 1.0f : 0.0f) : (unit ? 0.0f : -INFINITY);
        return;
    }
    // the rows of block b before n (a prefix: positions grow with t)
    auto rows = [&](int b) { return min(FA_C, (n - base(b) + FA_NCH - 1) / FA_NCH); };
    if constexpr (!SPEC) load_block(0, rows(0));
    const bool has_pos = (int)(pos % FA_NCH) == c;
    {
        const int nrows = n_rep + (has_pos ? 1 : 0);
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const int r = wave + i * NWV;
            if (r < nrows) {
                const float a1 = on ? x1[i] : 0.0f, a2 = on ? x2[i] : 0.0f;
                const float ss = wave_sum(fmaf(a1, a1, a2 * a2));
                const float sc = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)HD), eps)));
                const bool isq = r < n_rep;
                const float y1 = (a1 * sc) * (isq ? qw1 : kw1), y2 = (a2 * sc) * (isq ? qw2 : kw2);
                const float o1 = fmaf(y1, c1, -(y2 * s1)), o2 = fmaf(y2, c1, y1 * s1);
                if (on) {
                    float* y = isq ? qs[r] : kcur;
                    y[lane] = o1;
                    y[lane + half] = o2;
                    if (!isq) {
                        kb[(size_t)pos * HD + lane] = o1;
                        kb[(size_t)pos * HD + lane + half] = o2;
                    }
                }
                if (!isq) {
#pragma unroll
                    for (int u = 0; u < HD / 64; u++) {
                        vcur[lane + 64 * u] = vv[u];
                        vb[(size_t)pos * HD + lane + 64 * u] = vv[u];
                    }
                }
            }
        }
    }
    if (threadIdx.x < FA_MAXREP) {
        s_m[threadIdx.x] = -INFINITY;
        s_l[threadIdx.x] = 0.0f;
    }
    // output (r0 + k, d) of thread (g, d): consecutive heads per thread, so
    // one 16-byte read of pt serves four of them
    const int g = threadIdx.x / HD, d = threadIdx.x % HD;
    const int nper = (n_rep + G - 1) / G, r0 = g * nper;
    float o[NOUT];
#pragma unroll
    for (int u = 0; u < NOUT; u++) o[u] = 0.0f;
    __syncthreads();  // qs, kcur, vcur, s_m, s_l written

    for (int b = 0; base(b) < n; b++) {
        const int nt = rows(b);
#pragma unroll
        for (int u = 0; u < NKV; u++) {
            const int i = threadIdx.x + u * FD_WG, t = i / HD4, d = 4 * (i % HD4);
            if (t < nt) {
                const bool cur = row_pos(b, t) == (int)pos;
                const u32x4 k4 = cur ? *reinterpret_cast<const u32x4*>(kcur + d) : kr[u];
                const u32x4 v4 = cur ? *reinterpret_cast<const u32x4*>(vcur + d) : vr[u];
                *reinterpret_cast<u32x4*>(&ks[t][d]) = k4;
                *reinterpret_cast<u32x4*>(&vs[t][d]) = v4;
            }
        }
        __syncthreads();
        if (base(b + 1) < n) load_block(b + 1, rows(b + 1));  // in flight during this block
        // scores s[r][t] = (q_r . k_t) * scale
        for (int i = threadIdx.x; i < n_rep * FA_C; i += FD_WG) {
            const int r = i / FA_C, t = i % FA_C;
            float dot = -INFINITY;
            if (t < nt) {
                float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
                for (int d = 0; d < HD; d += 4) {
                    const float4 q4 = *reinterpret_cast<const float4*>(&qs[r][d]);
                    const float4 k4 = *reinterpret_cast<const float4*>(&ks[t][d]);
                    a0 = fmaf(q4.x, k4.x, a0);
                    a1 = fmaf(q4.y, k4.y, a1);
                    a2 = fmaf(q4.z, k4.z, a2);
                    a3 = fmaf(q4.w, k4.w, a3);
                }
                dot = ((a0 + a1) + (a2 + a3)) * scale;
            }
            ps[r][t] = dot;
        }
        __syncthreads();
        // running softmax per head (one wave per head, lanes = positions)
        for (int r = wave; r < n_rep; r += FD_WG / 64) {
            const float v = lane < FA_C ? ps[r][lane] : -INFINITY;
            const float m = wave_max(v);
            const float mo = s_m[r], mn = fmaxf(mo, m);
            const float e = lane < nt ? __expf(v - mn) : 0.0f;
            const float l = wave_sum(e);
            const float corr = __expf(mo - mn);  // 0 on the first block (mo = -inf)
            if (lane < FA_C) pt[lane][r] = e;
            if (lane == 0) {
                s_m[r] = mn;
                s_l[r] = fmaf(s_l[r], corr, l);
                s_corr[r] = corr;
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < NOUT; u++)
            if (u < nper && r0 + u < n_rep) o[u] *= s_corr[r0 + u];
        if ((nper & 3) == 0) {
#pragma unroll 4
            for (int t = 0; t < nt; t++) {
                const float v = vs[t][d];
#pragma unroll
                for (int u = 0; u < NOUT; u += 4)
                    if (u < nper) {
                        const float4 w4 = *reinterpret_cast<const float4*>(&pt[t][r0 + u]);
                        o[u] = fmaf(w4.x, v, o[u]);
                        o[u + 1] = fmaf(w4.y, v, o[u + 1]);
                        o[u + 2] = fmaf(w4.z, v, o[u + 2]);
                        o[u + 3] = fmaf(w4.w, v, o[u + 3]);
                    }
            }
        } else {
            for (int t = 0; t < nt; t++) {
                const float v = vs[t][d];
#pragma unroll
                for (int u = 0; u < NOUT; u++)
                    if (u < nper) o[u] = fmaf(pt[t][r0 + u], v, o[u]);
            }
        }
        __syncthreads();  // before the next block overwrites ks, vs, ps, pt
    }

    // the chunk's state (the next launch, o_proj, reads it)
#pragma unroll
    for (int u = 0; u < NOUT; u++)
        if (u < nper && r0 + u < n_rep) part_o[((size_t)c * nh + j * n_rep + r0 + u) * HD + d] = o[u];
    if ((int)threadIdx.x < 2 * n_rep) {
        const int r = threadIdx.x >> 1;
        part_ml[((size_t)c * nh + j * n_rep + r) * 2 + (threadIdx.x & 1)] = (threadIdx.x & 1) ? s_l[r] : s_m[r];
    }
}

// ---- batched prefill: the n tokens at positions pos0 .. pos0+n-1 ----------
// Row t of Q [n][nh*HD], K and V [n][nkv*HD] is position pos0 + t. Workgroup
// t: q_norm + RoPE on every query head in place, k_norm + RoPE on every key
// head into the key cache, every value head into the value cache (one wave
// per head row, as fa_norm_rope does it for one position).
template <int HD>
__global__ __launch_bounds__(256) void k_pf_qk_rope(float* __restrict__ Q, const float* __restrict__ Kx,
                                                    const float* __restrict__ Vx, const float* __restrict__ qn,
                                                    const float* __restrict__ kn, int nh, int nkv, float eps,
                                                    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                                    int pos0, int max_pos, float* __restrict__ kc,
                                                    float* __restrict__ vc)
{
    const int t = blockIdx.x, pos = pos0 + t;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const float* cs = cos_t + (size_t)pos * (HD / 2);
    const float* sn = sin_t + (size_t)pos * (HD / 2);
    for (int r = wave; r < nh + 2 * nkv; r += 4) {
        if (r < nh) {
            float* q = Q + ((size_t)t * nh + r) * HD;
            fa_norm_rope<HD>(q, qn, eps, cs, sn, q, nullptr);
        } else if (r < nh + nkv) {
            const int j = r - nh;
            fa_norm_rope<HD>(Kx + ((size_t)t * nkv + j) * HD, kn, eps, cs, sn,
                             kc + ((size_t)j * max_pos + pos) * HD, nullptr);
        } else {
            const int j = r - nh - nkv;
            for (int d = lane; d < HD; d += 64)
                vc[((size_t)j * max_pos + pos) * HD + d] = Vx[((size_t)t * nkv + j) * HD + d];
        }
    }
}

// ---- the batched prefill's causal attention, on the fp32 matrix cores ----
// Query token t sits at position pos0 + t and sees positions 0..pos0 + t of
// the caches. Workgroup (NHW query heads of one key head, block of 16 query
// rows); its PA_W waves split the block's 16-position key tiles (wave w:
// tiles w, w + PA_W, ...), each with a running softmax per head, and merge
// their states pairwise through LDS at the end (a fixed tree: wave w takes
// wave w + PA_W/2, then w + PA_W/4, ...). Per tile a wave forms each head's scores
// transposed, S^T = K Q^T, in HD/4 steps of v_mfma_f32_16x16x4_f32: lane
// (kq, c) supplies key row c of the tile and query row c at the same dim in
// each step (read straight into registers). The product leaves lane (kq, c)
// the scores of query row c at tile positions 4kq..4kq+3, which, once
// exponentiated, are as they lie the second operand of O^T += V^T P^T (four
// steps of k = 4 positions; lane (kq, c) supplies V[position 4kq + i][a dim
// of column c] for each output tile): that product leaves lane (kq, c)
// holding query row c, so the softmax rescale is lane-local and only the
// row maximum crosses lanes (the row's four lane groups, by the 16- and
// 32-lane swaps). A wave serves NHW heads of one key head with each tile
// it loads; the launch uses one (NHW = 2 halves the loads, but doubles the
// matrix-core work per SIMD, and that, with the load latency, sets the
// time: 17.5 us for the 256-token, 32-head prefill against 12 with one).
// Scores are in the log2 domain (Q scaled by scale * log2 e on load) and
// exponentials are exp2. Rows of the last block past n are computed from
// row n - 1 and not stored; positions past the block's last are masked and
// their loads read row pos0 + n - 1. Deterministic; not the stepwise
// attention's operation order (FAST mode).
template <int HD, int NHW, int PA_W>
__global__ __launch_bounds__(PA_W * 64) void k_pf_attention(const float* __restrict__ Q, int nh, int nkv,
                                                            float scale, int pos0, int n, int max_pos,
                                                            const float* __restrict__ kc,
                                                            const float* __restrict__ vc, float* __restrict__ O,
                                                            uint32_t* __restrict__ xf, float* __restrict__ xsum,
                                                            int XT)
{
    constexpr int DL = HD / 4;    // dims per lane in the score product
    constexpr int NDT = HD / 16;  // output tiles of 16 dims
    constexpr int OS = HD + 4;    // LDS row stride of the merge
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    __shared__ float sm_m[PA_W / 2][NHW][16], sm_l[PA_W / 2][NHW][16];
    __shared__ __align__(16) float so[PA_W / 2][NHW][16][OS];
    // the longest blocks first, then the shortest: the second half of the
    // launch (which shares the CUs with the first) in the reverse order, so
    // that a CU's two workgroups hold about the same work
    const int ny = (int)gridDim.y, hy = (ny + 1) / 2, y = (int)blockIdx.y;
    const int h0 = blockIdx.x * NHW, qb = y < hy ? ny - 1 - y : y - hy;
    const int j = h0 / (nh / nkv);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, kq = lane >> 4, c = lane & 15;
    const int qpos = pos0 + 16 * qb + c;                   // this lane's query row's position
    const int last = pos0 + min(16 * qb + 15, n - 1);      // the block's last position
    const int plim = pos0 + n - 1;                         // last cache row the loads may read
    const int ntiles = last / 16 + 1;
    const float* kb = kc + (size_t)j * max_pos * HD;
    const float* vb = vc + (size_t)j * max_pos * HD;

    // Score step s = 4u + i of lane (kq, c) takes dim 16u + 4kq + i (query
    // and key alike), and output tile dt = 4u + jj row c dim 64u + 4c + jj,
    // so that one 16-byte load per lane covers 64 contiguous bytes of each
    // of 16 key rows, or 256 of each of 4 value rows (lanes reading 16 bytes
    // at a 128-byte stride cost a cache-line access each).
    float q[NHW][DL];
    {
        const float qs = scale * 1.44269504088896341f;
#pragma unroll
        for (int hh = 0; hh < NHW; hh++) {
            const float* qp = Q + ((size_t)min(16 * qb + c, n - 1) * nh + h0 + hh) * HD + 4 * kq;
#pragma unroll
            for (int u = 0; u < DL; u += 4) {
                const float4 v = *reinterpret_cast<const float4*>(qp + 4 * u);
                q[hh][u] = v.x * qs;
                q[hh][u + 1] = v.y * qs;
                q[hh][u + 2] = v.z * qs;
                q[hh][u + 3] = v.w * qs;
            }
        }
    }
    // Buffer loads: plain loads of a later tile were sunk by the compiler to
    // their uses. A tile's keys are requested once its scores are formed and
    // its values once its outputs are, each for the wave's next tile.
    const auto krs = buf_rsrc(kb, (plim + 1) * HD * 4), vrs = buf_rsrc(vb, (plim + 1) * HD * 4);
    u32x4 kr[DL / 4], vr[4][NDT / 4];
    auto load_k = [&](int tile) {
        const int ko = (min(tile * 16 + c, plim) * HD + 4 * kq) * 4;
#pragma unroll
        for (int u = 0; u < DL / 4; u++) kr[u] = __builtin_amdgcn_raw_buffer_load_b128(krs, ko + 64 * u, 0, 0);
    };
    auto load_v = [&](int tile) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int vo = (min(tile * 16 + 4 * kq + i, plim) * HD + 4 * c) * 4;
#pragma unroll
            for (int u = 0; u < NDT / 4; u++) vr[i][u] = __builtin_amdgcn_raw_buffer_load_b128(vrs, vo + 256 * u, 0, 0);
        }
    };
    f32x4 o[NHW][NDT];
    float m[NHW], l[NHW];
#pragma unroll
    for (int hh = 0; hh < NHW; hh++) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) o[hh][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (wave < ntiles) {
        load_k(wave);
        load_v(wave);
    }
    for (int tile = wave; tile < ntiles; tile += PA_W) {
        const bool more = tile + PA_W < ntiles;
        f32x4 s[NHW];
#pragma unroll
        for (int hh = 0; hh < NHW; hh++) s[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < DL / 4; u++)
#pragma unroll
            for (int hh = 0; hh < NHW; hh++) {
                s[hh] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(kr[u].x), q[hh][4 * u], s[hh], 0, 0, 0);
                s[hh] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(kr[u].y), q[hh][4 * u + 1], s[hh], 0, 0, 0);
                s[hh] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(kr[u].z), q[hh][4 * u + 2], s[hh], 0, 0, 0);
                s[hh] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(kr[u].w), q[hh][4 * u + 3], s[hh], 0, 0, 0);
            }
        if (more) load_k(tile + PA_W);
        __builtin_amdgcn_sched_barrier(0);
        const int pb = tile * 16 + 4 * kq;
        float e[NHW][4];
#pragma unroll
        for (int hh = 0; hh < NHW; hh++) {
            float sv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) sv[i] = pb + i <= qpos ? s[hh][i] : -INFINITY;
            float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
            const auto r1 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
            mt = fmaxf(__uint_as_float(r1[0]), __uint_as_float(r1[1]));
            const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
            mt = fmaxf(__uint_as_float(r2[0]), __uint_as_float(r2[1]));
            const float mn = fmaxf(m[hh], mt);
            const float mr = mn == -INFINITY ? 0.0f : mn;  // a row with every position so far masked
            const float corr = __builtin_amdgcn_exp2f(m[hh] - mr);
#pragma unroll
            for (int i = 0; i < 4; i++) e[hh][i] = __builtin_amdgcn_exp2f(sv[i] - mr);
            l[hh] = fmaf(l[hh], corr, (e[hh][0] + e[hh][1]) + (e[hh][2] + e[hh][3]));
            m[hh] = mn;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) o[hh][dt] *= corr;
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int u = 0; u < NDT / 4; u++)
#pragma unroll
                for (int hh = 0; hh < NHW; hh++) {
                    f32x4* oo = &o[hh][4 * u];
                    oo[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(vr[i][u].x), e[hh][i], oo[0], 0, 0, 0);
                    oo[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(vr[i][u].y), e[hh][i], oo[1], 0, 0, 0);
                    oo[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(vr[i][u].z), e[hh][i], oo[2], 0, 0, 0);
                    oo[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(vr[i][u].w), e[hh][i], oo[3], 0, 0, 0);
                }
        if (more) load_v(tile + PA_W);
        __builtin_amdgcn_sched_barrier(0);
    }
    // each row's sum over its four lane groups
#pragma unroll
    for (int hh = 0; hh < NHW; hh++) {
        const auto r1 = __builtin_amdgcn_permlane16_swap(__float_as_uint(l[hh]), __float_as_uint(l[hh]), false, false);
        l[hh] = __uint_as_float(r1[0]) + __uint_as_float(r1[1]);
        const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(l[hh]), __float_as_uint(l[hh]), false, false);
        l[hh] = __uint_as_float(r2[0]) + __uint_as_float(r2[1]);
    }
    // the waves' states merged pairwise: wave w + half into wave w, for
    // half = PA_W/2, ..., 1; lane (kq, c), output register i of tile dt = 4u + jj:
    // query row c, dim 64u + 4 (4kq + i) + jj
#pragma unroll
    for (int half = PA_W / 2; half >= 1; half >>= 1) {
        if (wave >= half && wave < 2 * half) {
            const int sl = wave - half;
#pragma unroll
            for (int hh = 0; hh < NHW; hh++) {
                if (kq == 0) {
                    sm_m[sl][hh][c] = m[hh];
                    sm_l[sl][hh][c] = l[hh];
                }
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int u = 0; u < NDT / 4; u++)
                        *reinterpret_cast<float4*>(&so[sl][hh][c][64 * u + 16 * kq + 4 * i]) =
                            make_float4(o[hh][4 * u][i], o[hh][4 * u + 1][i], o[hh][4 * u + 2][i],
                                        o[hh][4 * u + 3][i]);
            }
        }
        __syncthreads();
        if (wave < half) {
#pragma unroll
            for (int hh = 0; hh < NHW; hh++) {
                const float mb = sm_m[wave][hh][c], lb = sm_l[wave][hh][c];
                const float M = fmaxf(m[hh], mb);
                const float Mr = M == -INFINITY ? 0.0f : M;
                const float fa = __builtin_amdgcn_exp2f(m[hh] - Mr), fb = __builtin_amdgcn_exp2f(mb - Mr);
                m[hh] = M;
                l[hh] = fmaf(fa, l[hh], fb * lb);
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int u = 0; u < NDT / 4; u++) {
                        const float4 b = *reinterpret_cast<const float4*>(&so[wave][hh][c][64 * u + 16 * kq + 4 * i]);
                        o[hh][4 * u][i] = fmaf(fa, o[hh][4 * u][i], fb * b.x);
                        o[hh][4 * u + 1][i] = fmaf(fa, o[hh][4 * u + 1][i], fb * b.y);
                        o[hh][4 * u + 2][i] = fmaf(fa, o[hh][4 * u + 2][i], fb * b.z);
                        o[hh][4 * u + 3][i] = fmaf(fa, o[hh][4 * u + 3][i], fb * b.w);
                    }
            }
        }
        __syncthreads();
    }
    // wave 0 holds position 0 of every row, so the maximum is finite and l > 0
    const int t = 16 * qb + c;
    if constexpr (HD == 128 && NHW == 1 && PA_W == 4) {
        // a head is one 128-value block of o_proj's input: the workgroup
        // writes its 16 rows of it as the GEMM's packed X (block h0, column
        // tile qb) instead of fp32 rows for a packing launch
        __shared__ float pk_red[2][4][16];
        if (wave == 0) {
            const float rl = 1.0f / l[0];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int u = 0; u < NDT / 4; u++)
                    *reinterpret_cast<float4*>(&so[0][0][c][64 * u + 16 * kq + 4 * i]) =
                        make_float4(o[0][4 * u][i] * rl, o[0][4 * u + 1][i] * rl, o[0][4 * u + 2][i] * rl,
                                    o[0][4 * u + 3][i] * rl);
        }
        __syncthreads();
        pack_tile_split(&so[0][0][0][0], OS, min(16, n - 16 * qb), h0, qb, XT, xf, xsum, pk_red);
        return;
    }
    if (wave != 0 || t >= n) return;
#pragma unroll
    for (int hh = 0; hh < NHW; hh++) {
        const float rl = 1.0f / l[hh];
        float* op = O + ((size_t)t * nh + h0 + hh) * HD + 16 * kq;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int u = 0; u < NDT / 4; u++)
                *reinterpret_cast<float4*>(op + 64 * u + 4 * i) =
                    make_float4(o[hh][4 * u][i] * rl, o[hh][4 * u + 1][i] * rl, o[hh][4 * u + 2][i] * rl,
                                o[hh][4 * u + 3][i] * rl);
    }
}

// x[i] += y[i] (residual updates the GEMV epilogues do not cover)
__global__ __launch_bounds__(256) void k_add(float* __restrict__ x, const float* __restrict__ y, int n)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = __fadd_rn(x[i], y[i]);
}

// ---- the FAST attention's chunk states merged into its output -------------
// out[h][d] = sum_c e^(m_c - M) o_c[h][d] / sum_c e^(m_c - M) l_c[h] with
// M = max_c m_c: the merge the o_proj GEMV's XF_MERGE prep does as it reads
// x, with the same operations in the same order (chunk order, fused
// multiply-adds, one correctly rounded reciprocal), done once per head for
// a plain GEMV that follows. Workgroup h, thread d < hd.
__global__ __launch_bounds__(128) void k_attention_merge(const float* __restrict__ part_o,
                                                         const float* __restrict__ part_ml, int nh, int hd,
                                                         float* __restrict__ out)
{
    const int h = blockIdx.x, d = threadIdx.x;
    if (d >= hd) return;
    const size_t stride = (size_t)nh * hd;
    float m[ATTN_CHUNKS], l[ATTN_CHUNKS], o[ATTN_CHUNKS];
#pragma unroll
    for (int cc = 0; cc < ATTN_CHUNKS; cc++) {
        m[cc] = part_ml[((size_t)cc * nh + h) * 2];
        l[cc] = part_ml[((size_t)cc * nh + h) * 2 + 1];
        o[cc] = part_o[cc * stride + (size_t)h * hd + d];
    }
    float M = -INFINITY;
#pragma unroll
    for (int cc = 0; cc < ATTN_CHUNKS; cc++) M = fmaxf(M, m[cc]);
    float L = 0.0f, a = 0.0f;
#pragma unroll
    for (int cc = 0; cc < ATTN_CHUNKS; cc++) {
        const float w = __expf(m[cc] - M);  // 0 for a chunk that held no position
        L = fmaf(w, l[cc], L);
        a = fmaf(w, o[cc], a);
    }
    out[(size_t)h * hd + d] = a * __fdiv_rn(1.0f, L);
}

// ---- argmax (sampling.rs:3-14) and the next step's input -------------------
// First index of the largest logit (strict >, so NaN never wins; 0 when no
// logit beats -inf).
constexpr int AM_WG = 1024;
// The first index of the largest of logits[0..n) by the whole workgroup
// (AM_WG threads), valid in thread 0; -1 when no value beats -inf.
__device__ int block_argmax(const float* __restrict__ logits, int n)
{
    __shared__ float sv[AM_WG / 64];
    __shared__ int si[AM_WG / 64];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    // thread t scans 16-byte chunks t, t+AM_WG, ... in increasing index
    // order (strict >, so its first maximum stays), four chunks in flight
    const int n4 = n >> 2;
    const float4* l4 = reinterpret_cast<const float4*>(logits);
    int c = threadIdx.x;
    for (; c + 3 * AM_WG < n4; c += 4 * AM_WG) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = l4[c + u * AM_WG];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = 4 * (c + u * AM_WG);
            if (v[u].x > bv) { bv = v[u].x; bi = i; }
            if (v[u].y > bv) { bv = v[u].y; bi = i + 1; }
            if (v[u].z > bv) { bv = v[u].z; bi = i + 2; }
            if (v[u].w > bv) { bv = v[u].w; bi = i + 3; }
        }
    }
    for (; c < n4; c += AM_WG) {
        const float4 v = l4[c];
        const int i = 4 * c;
        if (v.x > bv) { bv = v.x; bi = i; }
        if (v.y > bv) { bv = v.y; bi = i + 1; }
        if (v.z > bv) { bv = v.z; bi = i + 2; }
        if (v.w > bv) { bv = v.w; bi = i + 3; }
    }
    for (int i = 4 * n4 + threadIdx.x; i < n; i += AM_WG)
        if (logits[i] > bv) { bv = logits[i]; bi = i; }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < AM_WG / 64; w++)  // wave 0's result is already in bv, bi
            if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) { bv = sv[w]; bi = si[w]; }
    return bv > -INFINITY ? bi : -1;
}

// Then the position advances; a position at or past the prompt gets the
// argmax (0 when no logit beats -inf) as its token.
__global__ __launch_bounds__(AM_WG) void k_argmax_next(const float* __restrict__ logits, int n,
                                                       DecodeState* __restrict__ st,
                                                       uint32_t* __restrict__ tokens)
{
    const int bi = block_argmax(logits, n);
    if (threadIdx.x == 0) {
        const uint32_t next = bi >= 0 ? (uint32_t)bi : 0u;
        const uint32_t p = st->pos + 1;
        st->last = next;
        if (p >= st->n_prompt && p <= st->max_pos) tokens[p] = next;
        st->pos = p;
    }
}

// The same from the keys of a FAST GEMV's workgroups (GemvJob::amax): the
// largest key names the first largest logit (0 when no logit beat -inf).
__global__ __launch_bounds__(AM_WG) void k_argmax_keys_next(const uint64_t* __restrict__ keys, int n,
                                                            DecodeState* __restrict__ st,
                                                            uint32_t* __restrict__ tokens)
{
    __shared__ uint64_t sk[AM_WG / 64];
    uint64_t k = 0;
    for (int i = threadIdx.x; i < n; i += AM_WG) k = max(k, keys[i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t k2 = ((uint64_t)(uint32_t)__shfl_xor((int)(k >> 32), o) << 32) |
                            (uint32_t)__shfl_xor((int)(uint32_t)k, o);
        k = max(k, k2);
    }
    if ((threadIdx.x & 63) == 0) sk[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < AM_WG / 64; w++) k = max(k, sk[w]);
        const uint32_t next = k ? 0xFFFFFFFFu - (uint32_t)k : 0u;
        const uint32_t p = st->pos + 1;
        st->last = next;
        if (p >= st->n_prompt && p <= st->max_pos) tokens[p] = next;
        st->pos = p;
    }
}

// out[r] = argmax of row r of logits [rows][n] (0 when none beats -inf).
__global__ __launch_bounds__(AM_WG) void k_argmax_rows(const float* __restrict__ logits, int n,
                                                       uint32_t* __restrict__ out)
{
    const int bi = block_argmax(logits + (size_t)blockIdx.x * n, n);
    if (threadIdx.x == 0) out[blockIdx.x] = bi >= 0 ? (uint32_t)bi : 0u;
}

// EXACT: the MoE layer's weighted combine folded into the next RMSNorm of
// the residual. x (the residual) becomes x + sum_k w_k y_k, the sum taken
// in chosen order from 0 over the slots that ran (ids[k] >= 0), each
// product and sum rounded (qwen3_moe_model.rs:526-533, as k_combine); the
// kernel writes it back to x, then RMSNorms it into out exactly as
// k_rms_norm<EXACT> does. One workgroup; n % 4 == 0, n <= RC_MAXN,
// top_k <= RC_MAXK. (In place of a combine launch before the norm.)
constexpr int RC_MAXN = 4096, RC_MAXK = 8;
__global__ __launch_bounds__(NW) void k_rms_norm_combine(float* __restrict__ x, const float* __restrict__ w,
                                                         int n, float eps, float* __restrict__ out,
                                                         const float* __restrict__ ys,
                                                         const int32_t* __restrict__ ids,
                                                         const float* __restrict__ cw, int top_k)
{
    constexpr int V = RC_MAXN / 4 / NW;
    typedef float f4 __attribute__((ext_vector_type(4)));
    __shared__ __align__(16) float sq[RC_MAXN];
    __shared__ float s_total;
    // every load first: x, the norm weights, the slots' outputs (range
    // checked, none past n), then the slots' ids and weights
    const auto xr = buf_rsrc(x, n * 4), wr = buf_rsrc(w, n * 4);
    f4 xv[V], wv[V], yv[RC_MAXK][V];
#pragma unroll
    for (int u = 0; u < V; u++) {
        xv[u] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(xr, (threadIdx.x + u * NW) * 16, 0, 0));
        wv[u] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(wr, (threadIdx.x + u * NW) * 16, 0, 0));
    }
#pragma unroll
    for (int k = 0; k < RC_MAXK; k++) {
        const auto yr = buf_rsrc(ys + (size_t)k * n, k < top_k ? n * 4 : 0);
#pragma unroll
        for (int u = 0; u < V; u++)
            yv[k][u] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(yr, (threadIdx.x + u * NW) * 16, 0, 0));
    }
    int idk[RC_MAXK];
    float wk[RC_MAXK];
#pragma unroll
    for (int k = 0; k < RC_MAXK; k++) {
        idk[k] = k < top_k ? ids[k] : -1;
        wk[k] = k < top_k ? cw[k] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < V; u++) {
        f4 acc = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < RC_MAXK; k++)
            if (idk[k] >= 0) {
                acc.x = __fadd_rn(acc.x, __fmul_rn(wk[k], yv[k][u].x));
                acc.y = __fadd_rn(acc.y, __fmul_rn(wk[k], yv[k][u].y));
                acc.z = __fadd_rn(acc.z, __fmul_rn(wk[k], yv[k][u].z));
                acc.w = __fadd_rn(acc.w, __fmul_rn(wk[k], yv[k][u].w));
            }
        xv[u] = f4{__fadd_rn(xv[u].x, acc.x), __fadd_rn(xv[u].y, acc.y), __fadd_rn(xv[u].z, acc.z),
                   __fadd_rn(xv[u].w, acc.w)};
        const int i = 4 * (threadIdx.x + u * NW);
        if (i < n) {
            *reinterpret_cast<f4*>(&x[i]) = xv[u];
            *reinterpret_cast<f4*>(&sq[i]) = f4{__fmul_rn(xv[u].x, xv[u].x), __fmul_rn(xv[u].y, xv[u].y),
                                                __fmul_rn(xv[u].z, xv[u].z), __fmul_rn(xv[u].w, xv[u].w)};
        }
    }
    for (int i = n + threadIdx.x; i < os_padded(n); i += NW) sq[i] = 0.0f;
    __syncthreads();
    if (threadIdx.x == 0) s_total = ordered_sum_lds(sq, n);
    __syncthreads();
    const float mean_sq = __fdiv_rn(s_total, (float)n);
    const float scale = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(mean_sq, eps)));
#pragma unroll
    for (int u = 0; u < V; u++) {
        const int i = 4 * (threadIdx.x + u * NW);
        if (i < n) {
            out[i] = __fmul_rn(__fmul_rn(xv[u].x, scale), wv[u].x);
            out[i + 1] = __fmul_rn(__fmul_rn(xv[u].y, scale), wv[u].y);
            out[i + 2] = __fmul_rn(__fmul_rn(xv[u].z, scale), wv[u].z);
            out[i + 3] = __fmul_rn(__fmul_rn(xv[u].w, scale), wv[u].w);
        }
    }
}

}  // namespace

// ---- launchers ---------------------------------------------------------------
hipError_t launch_rms_norm(int mode, const float* x, const float* w, int n, float eps, float* out,
                           hipStream_t s)
{
    (void)hipGetLastError();
    if (mode == WPCG_MODE_EXACT)
        hipLaunchKernelGGL(k_rms_norm<WPCG_MODE_EXACT>, dim3(1), dim3(NW), 0, s, x, w, n, eps, out);
    else
        hipLaunchKernelGGL(k_rms_norm<WPCG_MODE_FAST>, dim3(1), dim3(NW), 0, s, x, w, n, eps, out);
    return hipGetLastError();
}

bool rms_norm_combine_ok(int n, int top_k) { return n > 0 && n % 4 == 0 && n <= RC_MAXN && top_k >= 1 && top_k <= RC_MAXK; }

hipError_t launch_rms_norm_combine(float* x, const float* w, int n, float eps, float* out, const float* ys,
                                   const int32_t* ids, const float* cw, int top_k, hipStream_t s)
{
    if (!rms_norm_combine_ok(n, top_k)) return hipErrorInvalidValue;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_rms_norm_combine, dim3(1), dim3(NW), 0, s, x, w, n, eps, out, ys, ids, cw, top_k);
    return hipGetLastError();
}

hipError_t launch_rms_norm_rows(int mode, const float* x, const float* w, int n, int rows, float eps, float* out,
                                hipStream_t s)
{
    (void)hipGetLastError();
    if (mode == WPCG_MODE_EXACT)
        hipLaunchKernelGGL(k_rms_norm<WPCG_MODE_EXACT>, dim3(rows), dim3(NW), 0, s, x, w, n, eps, out);
    else
        hipLaunchKernelGGL(k_rms_norm<WPCG_MODE_FAST>, dim3(rows), dim3(NW), 0, s, x, w, n, eps, out);
    return hipGetLastError();
}

int attention_max_pos() { return AT_MAXPOS; }

bool attention_fast_ok(int nh, int nkv, int hd) { return (hd == 64 || hd == 128) && nh / nkv <= FA_MAXREP; }

hipError_t launch_attention(int mode, const float* q, const float* k, const float* v, const float* qn,
                            const float* kn, int nh, int nkv, int hd, float eps, float scale,
                            const float* cos_t, const float* sin_t, const DecodeState* st, float* kc,
                            float* vc, float* out, hipStream_t s)
{
    (void)hipGetLastError();
    if (mode == WPCG_MODE_EXACT)
        hipLaunchKernelGGL(k_attention<WPCG_MODE_EXACT>, dim3(nh), dim3(AT_WG), 0, s, q, k, v, qn, kn,
                           nh, nkv, hd, eps, scale, cos_t, sin_t, st, kc, vc, out);
    else
        hipLaunchKernelGGL(k_attention<WPCG_MODE_FAST>, dim3(nh), dim3(AT_WG), 0, s, q, k, v, qn, kn,
                           nh, nkv, hd, eps, scale, cos_t, sin_t, st, kc, vc, out);
    return hipGetLastError();
}

hipError_t launch_attention_chunks(const float* q, const float* k, const float* v, const float* qn,
                                   const float* kn, int nh, int nkv, int hd, float eps, float scale,
                                   const float* rope, int cache_pos, const DecodeState* st, float* kc,
                                   float* vc, float* part_o, float* part_ml, hipStream_t s)
{
    if (!attention_fast_ok(nh, nkv, hd) || !rope || cache_pos < 1 || (size_t)cache_pos * hd * 4 > 0x7fffffffu)
        return hipErrorInvalidValue;
    (void)hipGetLastError();
#define WPCG_ATT(HD, WG)                                                                                  \
    hipLaunchKernelGGL((k_attention_fast<HD, WG>), dim3(nkv * FA_NCH), dim3(WG), 0, s, q, k, v, qn, kn, nh, nkv, \
                       eps, scale, rope, cache_pos, st, kc, vc, part_o, part_ml)
    const bool wide = nh / nkv <= 4;
    if (hd == 128) {
        if (wide) WPCG_ATT(128, 512);
        else WPCG_ATT(128, 256);
    } else {
        if (wide) WPCG_ATT(64, 512);
        else WPCG_ATT(64, 256);
    }
#undef WPCG_ATT
    return hipGetLastError();
}

// one head per wave, four waves per workgroup (grid: heads x query blocks)
constexpr int PA_W = 4;
template <int HD>
void launch_pf_attention_t(const float* Q, int nh, int nkv, float scale, int pos0, int n, int max_pos,
                           const float* kc, const float* vc, float* out, void* xf, float* xsum, hipStream_t s)
{
    hipLaunchKernelGGL((k_pf_attention<HD, 1, PA_W>), dim3(nh, (n + 15) / 16), dim3(PA_W * 64), 0, s, Q, nh, nkv,
                       scale, pos0, n, max_pos, kc, vc, out, static_cast<uint32_t*>(xf), xsum, gemm_rows_tiles(n));
}

hipError_t launch_prefill_attention(float* Q, const float* Kx, const float* Vx, const float* qn, const float* kn,
                                    int nh, int nkv, int hd, float eps, float scale, const float* cos_t,
                                    const float* sin_t, int pos0, int n, int max_pos, float* kc, float* vc,
                                    float* out, void* xf, float* xsum, hipStream_t s, bool qk_done)
{
    if (!attention_fast_ok(nh, nkv, hd) || n < 1 || pos0 + n > max_pos) return hipErrorInvalidValue;
    if (hd == 128 ? !xf || !xsum : !out || qk_done) return hipErrorInvalidValue;
    (void)hipGetLastError();
    if (hd == 128) {
        if (!qk_done)
            hipLaunchKernelGGL(k_pf_qk_rope<128>, dim3(n), dim3(256), 0, s, Q, Kx, Vx, qn, kn, nh, nkv, eps, cos_t,
                               sin_t, pos0, max_pos, kc, vc);
        launch_pf_attention_t<128>(Q, nh, nkv, scale, pos0, n, max_pos, kc, vc, out, xf, xsum, s);
    } else {
        hipLaunchKernelGGL(k_pf_qk_rope<64>, dim3(n), dim3(256), 0, s, Q, Kx, Vx, qn, kn, nh, nkv, eps, cos_t,
                           sin_t, pos0, max_pos, kc, vc);
        launch_pf_attention_t<64>(Q, nh, nkv, scale, pos0, n, max_pos, kc, vc, out, xf, xsum, s);
    }
    return hipGetLastError();
}

hipError_t launch_attention_merge(const float* part_o, const float* part_ml, int nh, int hd, float* out,
                                  hipStream_t s)
{
    if (nh < 1 || hd < 1 || hd > 128) return hipErrorInvalidValue;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_attention_merge, dim3(nh), dim3(128), 0, s, part_o, part_ml, nh, hd, out);
    return hipGetLastError();
}

hipError_t launch_add(float* x, const float* y, int n, hipStream_t s)
{
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_add, dim3((n + 255) / 256), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

hipError_t launch_argmax_rows(const float* logits, int n, int rows, uint32_t* out, hipStream_t s)
{
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_argmax_rows, dim3(rows), dim3(AM_WG), 0, s, logits, n, out);
    return hipGetLastError();
}

hipError_t launch_argmax_keys_next(const uint64_t* keys, int n, DecodeState* st, uint32_t* tokens,
                                   hipStream_t s)
{
    if (n < 1) return hipErrorInvalidValue;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_argmax_keys_next, dim3(1), dim3(AM_WG), 0, s, keys, n, st, tokens);
    return hipGetLastError();
}

hipError_t launch_argmax_next(const float* logits, int n, DecodeState* st, uint32_t* tokens,
                              hipStream_t s)
{
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_argmax_next, dim3(1), dim3(AM_WG), 0, s, logits, n, st, tokens);
    return hipGetLastError();
}

}  // namespace wpcg
