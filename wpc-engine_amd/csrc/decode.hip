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

template <int MODE>
__global__ __launch_bounds__(NW) void k_rms_norm(const float* __restrict__ x,
                                                 const float* __restrict__ w, int n, float eps,
                                                 float* __restrict__ out)
{
    __shared__ float red[NW / 64];
    const float s = sum_squares<MODE>(x, n, red);
    const float mean_sq = __fdiv_rn(s, (float)n);
    const float scale = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(mean_sq, eps)));
    for (int i = threadIdx.x; i < n; i += NW) out[i] = __fmul_rn(__fmul_rn(x[i], scale), w[i]);
}

// ---- per-head q/k RMSNorm, RoPE, KV-cache append ---------------------------
// Workgroup h < nh: query head h, normed with q_norm and rotated in place.
// Workgroup nh + j: key head j, normed with k_norm, rotated and stored at the
// current position of the layer's K cache; value head j copied to the V
// cache. RoPE (rope.rs:24-39): out_i = x1*c - x2*s, out_{i+d/2} = x2*c + x1*s
// with c, s the f32 casts of the host's f64 cos/sin (cos_t/sin_t, [pos][d/2]).
// Caches are [layer][kv_head][max_pos][head_dim].
template <int MODE>
__global__ __launch_bounds__(128) void k_head_norm_rope(float* __restrict__ q,
                                                        const float* __restrict__ k,
                                                        const float* __restrict__ v,
                                                        const float* __restrict__ qn,
                                                        const float* __restrict__ kn, int nh,
                                                        int hd, float eps,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t,
                                                        const DecodeState* __restrict__ st,
                                                        float* __restrict__ kc,
                                                        float* __restrict__ vc, int nkv)
{
    __shared__ float red[2];
    __shared__ float y[256];  // head_dim <= 256
    const int h = blockIdx.x;
    const bool is_q = h < nh;
    const float* x = is_q ? q + (size_t)h * hd : k + (size_t)(h - nh) * hd;
    const float* w = is_q ? qn : kn;
    const float s = sum_squares<MODE>(x, hd, red);
    const float mean_sq = __fdiv_rn(s, (float)hd);
    const float scale = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(mean_sq, eps)));
    for (int i = threadIdx.x; i < hd; i += blockDim.x) y[i] = __fmul_rn(__fmul_rn(x[i], scale), w[i]);
    __syncthreads();
    const uint32_t pos = st->pos;
    const int half = hd / 2;
    const float* c = cos_t + (size_t)pos * half;
    const float* sn = sin_t + (size_t)pos * half;
    float* dst = is_q ? q + (size_t)h * hd
                      : kc + ((size_t)(h - nh) * st->max_pos + pos) * hd;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float x1 = y[i], x2 = y[i + half];
        dst[i] = __fsub_rn(__fmul_rn(x1, c[i]), __fmul_rn(x2, sn[i]));
        dst[i + half] = __fadd_rn(__fmul_rn(x2, c[i]), __fmul_rn(x1, sn[i]));
    }
    if (!is_q) {
        const int j = h - nh;
        float* vd = vc + ((size_t)j * st->max_pos + pos) * hd;
        for (int i = threadIdx.x; i < hd; i += blockDim.x) vd[i] = v[(size_t)j * hd + i];
    }
    (void)nkv;
}

// ---- attention over positions 0..pos (model.rs:466-490) --------------------
// scores[h][t] = (sum_d q_h[d] * k_t[d]) * scale, index order; the head's
// kv head is h / (nh / nkv). One thread per (head, position).
template <int MODE>
__global__ __launch_bounds__(64) void k_attn_scores(const float* __restrict__ q,
                                                    const float* __restrict__ kc, int nh, int nkv,
                                                    int hd, float scale,
                                                    const DecodeState* __restrict__ st,
                                                    float* __restrict__ scores)
{
    __shared__ float qs[256];
    const int h = blockIdx.y;
    const int t = blockIdx.x * 64 + threadIdx.x;
    const uint32_t pos = st->pos, max_pos = st->max_pos;
    if (blockIdx.x * 64 > pos) return;  // whole workgroup past the sequence
    for (int i = threadIdx.x; i < hd; i += 64) qs[i] = q[(size_t)h * hd + i];
    __syncthreads();
    if (t > (int)pos) return;
    const int kvh = h / (nh / nkv);
    const float* kt = kc + ((size_t)kvh * max_pos + t) * hd;
    float dot = 0.0f;
    if (MODE == WPCG_MODE_EXACT) {
        for (int d = 0; d < hd; d++) dot = __fadd_rn(dot, __fmul_rn(qs[d], kt[d]));
    } else {
        for (int d = 0; d < hd; d++) dot = fmaf(qs[d], kt[d], dot);
    }
    scores[(size_t)h * max_pos + t] = __fmul_rn(dot, scale);
}

// softmax_inplace over scores[h][0..pos] (norm.rs:28-43), one workgroup per head
__global__ __launch_bounds__(NW) void k_attn_softmax(float* __restrict__ scores,
                                                     const DecodeState* __restrict__ st)
{
    __shared__ float red[NW / 64];
    __shared__ float s_sum;
    const int n = (int)st->pos + 1;
    float* x = scores + (size_t)blockIdx.x * st->max_pos;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += NW) m = fmaxf(m, x[i]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int i = threadIdx.x; i < n; i += NW) x[i] = ref_expf(__fsub_rn(x[i], m));
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (int i = 0; i < n; i++) s = __fadd_rn(s, x[i]);
        s_sum = s;
    }
    __syncthreads();
    const float s = s_sum;
    if (s > 0.0f)
        for (int i = threadIdx.x; i < n; i += NW) x[i] = __fdiv_rn(x[i], s);
}

// out[h][d] = sum_t scores[h][t] * v_t[d] in position order, from 0.
// One thread per (head, d).
template <int MODE>
__global__ __launch_bounds__(128) void k_attn_out(const float* __restrict__ scores,
                                                  const float* __restrict__ vc, int nh, int nkv,
                                                  int hd, const DecodeState* __restrict__ st,
                                                  float* __restrict__ out)
{
    const int h = blockIdx.x;
    const uint32_t pos = st->pos, max_pos = st->max_pos;
    const int kvh = h / (nh / nkv);
    const float* w = scores + (size_t)h * max_pos;
    const float* vb = vc + (size_t)kvh * max_pos * hd;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.0f;
        if (MODE == WPCG_MODE_EXACT) {
            for (uint32_t t = 0; t <= pos; t++) acc = __fadd_rn(acc, __fmul_rn(w[t], vb[(size_t)t * hd + d]));
        } else {
            for (uint32_t t = 0; t <= pos; t++) acc = fmaf(w[t], vb[(size_t)t * hd + d], acc);
        }
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

hipError_t launch_head_norm_rope(int mode, float* q, const float* k, const float* v, const float* qn,
                                 const float* kn, int nh, int nkv, int hd, float eps,
                                 const float* cos_t, const float* sin_t, const DecodeState* st,
                                 float* kc, float* vc, hipStream_t s)
{
    (void)hipGetLastError();
    if (mode == WPCG_MODE_EXACT)
        hipLaunchKernelGGL(k_head_norm_rope<WPCG_MODE_EXACT>, dim3(nh + nkv), dim3(128), 0, s, q, k,
                           v, qn, kn, nh, hd, eps, cos_t, sin_t, st, kc, vc, nkv);
    else
        hipLaunchKernelGGL(k_head_norm_rope<WPCG_MODE_FAST>, dim3(nh + nkv), dim3(128), 0, s, q, k,
                           v, qn, kn, nh, hd, eps, cos_t, sin_t, st, kc, vc, nkv);
    return hipGetLastError();
}

hipError_t launch_attention(int mode, const float* q, const float* kc, const float* vc, int nh,
                            int nkv, int hd, int max_pos, float scale, const DecodeState* st,
                            float* scores, float* out, hipStream_t s)
{
    (void)hipGetLastError();
    const dim3 g((max_pos + 63) / 64, nh);
    if (mode == WPCG_MODE_EXACT)
        hipLaunchKernelGGL(k_attn_scores<WPCG_MODE_EXACT>, g, dim3(64), 0, s, q, kc, nh, nkv, hd, scale,
                           st, scores);
    else
        hipLaunchKernelGGL(k_attn_scores<WPCG_MODE_FAST>, g, dim3(64), 0, s, q, kc, nh, nkv, hd, scale,
                           st, scores);
    hipLaunchKernelGGL(k_attn_softmax, dim3(nh), dim3(NW), 0, s, scores, st);
    if (mode == WPCG_MODE_EXACT)
        hipLaunchKernelGGL(k_attn_out<WPCG_MODE_EXACT>, dim3(nh), dim3(128), 0, s, scores, vc, nh, nkv,
                           hd, st, out);
    else
        hipLaunchKernelGGL(k_attn_out<WPCG_MODE_FAST>, dim3(nh), dim3(128), 0, s, scores, vc, nh, nkv,
                           hd, st, out);
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
