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

namespace wpcg {
namespace {

// Correctly rounded square root (IEEE, as f32::sqrt): the plain builtin
// expands to the hardware estimate plus a rounding fixup; __fsqrt_rn, without
// OCML's rounded-operation mode, is the bare estimate (up to 1 ulp off).
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }

// ---- rms_norm (wpc-runtime/src/norm.rs:4-13) -------------------------------
// mean_sq = (sum x_i^2) / n; scale = 1 / sqrt(mean_sq + eps);
// out_i = x_i * scale * w_i. One workgroup of NW threads.
constexpr int NW = 256;

template <int MODE>
__device__ float sum_squares(const float* x, int n, float* red)
{
    __shared__ float s_total;
    if (MODE == WPCG_MODE_EXACT) {
        if (threadIdx.x == 0) {
            float s = 0.0f;
            for (int i = 0; i < n; i++) s = __fadd_rn(s, __fmul_rn(x[i], x[i]));
            s_total = s;
        }
    } else {
        float s = 0.0f;
        for (int i = threadIdx.x; i < n; i += blockDim.x) s = fmaf(x[i], x[i], s);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
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
// memory twice): EXACT's index-order sum of squares then runs from LDS in one
// thread, FAST's from registers as a tree.
constexpr int RN_LDS = 8192;
template <int MODE>
__global__ __launch_bounds__(NW) void k_rms_norm(const float* __restrict__ x,
                                                 const float* __restrict__ w, int n, float eps,
                                                 float* __restrict__ out)
{
    __shared__ float xs[RN_LDS];
    __shared__ float red[NW / 64];
    __shared__ float s_total;
    const bool staged = n <= RN_LDS;
    const float* src = staged ? xs : x;
    float part = 0.0f;
    for (int i = threadIdx.x; i < n; i += NW) {
        const float v = x[i];
        if (staged) xs[i] = v;
        part = fmaf(v, v, part);
    }
    if (MODE == WPCG_MODE_EXACT) {
        __syncthreads();
        if (threadIdx.x == 0) {
            float s = 0.0f;
            for (int i = 0; i < n; i++) s = __fadd_rn(s, __fmul_rn(src[i], src[i]));
            s_total = s;
        }
    } else {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o);
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
constexpr int AT_WG = 256;
constexpr int AT_MAXPOS = 4096;

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
    __shared__ float w[AT_MAXPOS];
    __shared__ float red[AT_WG / 64];
    __shared__ float s_sum;
    const int h = blockIdx.x, n_rep = nh / nkv, j = h / n_rep;
    const uint32_t pos = st->pos, max_pos = st->max_pos;
    const int half = hd / 2;
    const float* c = cos_t + (size_t)pos * half;
    const float* sn = sin_t + (size_t)pos * half;
    head_rms_rope<MODE>(qp + (size_t)h * hd, qn, qs, red, hd, eps, c, sn);
    head_rms_rope<MODE>(kp + (size_t)j * hd, kn, ks, red, hd, eps, c, sn);
    for (int i = threadIdx.x; i < hd; i += AT_WG) vs[i] = vp[(size_t)j * hd + i];
    __syncthreads();
    const float* kb = kc + (size_t)j * max_pos * hd;
    const float* vb = vc + (size_t)j * max_pos * hd;
    if (h % n_rep == 0)
        for (int i = threadIdx.x; i < hd; i += AT_WG) {
            kc[((size_t)j * max_pos + pos) * hd + i] = ks[i];
            vc[((size_t)j * max_pos + pos) * hd + i] = vs[i];
        }
    // scores: thread t, one position at a time; rows read as float4 chunks
    const int n = (int)pos + 1;
    for (int t = threadIdx.x; t < n; t += AT_WG) {
        const float* kt = t == (int)pos ? ks : kb + (size_t)t * hd;
        float dot = 0.0f;
        for (int d0 = 0; d0 < hd; d0 += 32) {
            float4 kv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) kv[u] = *reinterpret_cast<const float4*>(kt + d0 + 4 * u);
#pragma unroll
            for (int u = 0; u < 8; u++) {
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
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int t = threadIdx.x; t < n; t += AT_WG) w[t] = ref_expf(__fsub_rn(w[t], m));
    __syncthreads();
    if (MODE == WPCG_MODE_EXACT) {
        if (threadIdx.x == 0) {
            float s = 0.0f;
            for (int t = 0; t < n; t++) s = __fadd_rn(s, w[t]);
            s_sum = s;
        }
    } else {
        float s = 0.0f;
        for (int t = threadIdx.x; t < n; t += AT_WG) s += w[t];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
        __syncthreads();
        if (threadIdx.x == 0) s_sum = (red[0] + red[1]) + (red[2] + red[3]);
    }
    __syncthreads();
    const float ssum = s_sum;
    if (ssum > 0.0f)
        for (int t = threadIdx.x; t < n; t += AT_WG) w[t] = __fdiv_rn(w[t], ssum);
    __syncthreads();
    // out[d] = sum_t w_t v_t[d], position order; thread d, loads 8 ahead
    for (int d = threadIdx.x; d < hd; d += AT_WG) {
        float acc = 0.0f;
        int t = 0;
        for (; t + 8 <= (int)pos; t += 8) {
            float vv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) vv[u] = vb[(size_t)(t + u) * hd + d];
#pragma unroll
            for (int u = 0; u < 8; u++)
                acc = MODE == WPCG_MODE_EXACT ? __fadd_rn(acc, __fmul_rn(w[t + u], vv[u]))
                                              : fmaf(w[t + u], vv[u], acc);
        }
        for (; t < (int)pos; t++)
            acc = MODE == WPCG_MODE_EXACT ? __fadd_rn(acc, __fmul_rn(w[t], vb[(size_t)t * hd + d]))
                                          : fmaf(w[t], vb[(size_t)t * hd + d], acc);
        acc = MODE == WPCG_MODE_EXACT ? __fadd_rn(acc, __fmul_rn(w[pos], vs[d])) : fmaf(w[pos], vs[d], acc);
        out[(size_t)h * hd + d] = acc;
    }
}

// x[i] += y[i] (residual updates the GEMV epilogues do not cover)
__global__ __launch_bounds__(256) void k_add(float* __restrict__ x, const float* __restrict__ y, int n)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = __fadd_rn(x[i], y[i]);
}

// ---- argmax (sampling.rs:3-14) and the next step's input -------------------
// First index of the largest logit (strict >, so NaN never wins; 0 when no
// logit beats -inf). Then the position advances; a position at or past the
// prompt gets the argmax as its token.
constexpr int AM_WG = 1024;
__global__ __launch_bounds__(AM_WG) void k_argmax_next(const float* __restrict__ logits, int n,
                                                       DecodeState* __restrict__ st,
                                                       uint32_t* __restrict__ tokens)
{
    __shared__ float sv[AM_WG / 64];
    __shared__ int si[AM_WG / 64];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += AM_WG)
        if (logits[i] > bv) { bv = logits[i]; bi = i; }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < AM_WG / 64; w++)  // wave 0's result is already in bv, bi
            if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) { bv = sv[w]; bi = si[w]; }
        const uint32_t next = bv > -INFINITY ? (uint32_t)bi : 0u;
        const uint32_t p = st->pos + 1;
        st->last = next;
        if (p >= st->n_prompt && p <= st->max_pos) tokens[p] = next;
        st->pos = p;
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

int attention_max_pos() { return AT_MAXPOS; }

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

hipError_t launch_add(float* x, const float* y, int n, hipStream_t s)
{
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_add, dim3((n + 255) / 256), dim3(256), 0, s, x, y, n);
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
