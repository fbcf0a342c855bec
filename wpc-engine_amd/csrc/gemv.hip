// Dequant-GEMV kernels for gfx950 (CDNA4, wave64) over WPC blocks of 128
// weights (v4: 4-bit codes, v3: 6-bit codes in two planes).
//
// Device layout (see wpcg_internal.hpp): per block a u32 params word
// (zp f16 | scale f16 << 16) and 64 lane-major code bytes, dev[l*8+g] =
// ref[g*8+l], plus (v3) 32 lane-major high-plane bytes.
//
// EXACT mode reproduces the reference's AVX2 row kernels bit for bit:
//   matvec_v4_fused (wpc-eval/src/fused_kernel.rs:237-271)
//   matvec_v3_fused (wpc-eval/src/fused_kernel.rs:163-189)
// Eight threads own one output row; thread l is AVX2 lane l. For every block
// in order it runs the lane's chain w = fma(code, scale, zp),
// acc = fma(w, x, acc) over the same weights in the same order, and the
// eight accumulators are combined in hsum_avx2's order
// ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) with xor-shuffles 4, 1, 2.
//
// x is staged in LDS per segment of blocks in the layout
//   xs[s*XS_BLK + l*XS_LANE + G] = x[(b0+s)*128 + G*8 + l]   (G < 16)
// so each thread reads its sixteen activations with four 16-byte LDS loads;
// XS_LANE = 20 floats spreads the eight lanes over distinct LDS banks.
#include <hip/hip_runtime.h>

#include "wpcg_internal.hpp"

namespace wpcg {
namespace {

constexpr int XS_LANE = 20;
constexpr int XS_BLK = 8 * XS_LANE;
constexpr int SEG = 32;  // blocks of x staged per LDS pass (20 KiB)
constexpr int WG = 256;  // threads per workgroup: 32 rows x 8 lanes

__device__ __forceinline__ float h2f(uint32_t bits)
{
    _Float16 h;
    uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

__device__ __forceinline__ void stage_x(float* xs, const float* __restrict__ x, int b0, int nbs)
{
    for (int i = threadIdx.x; i < nbs * 128; i += WG) {
        int s = i >> 7, r = i & 127;
        xs[s * XS_BLK + (r & 7) * XS_LANE + (r >> 3)] = x[(size_t)b0 * 128 + i];
    }
}

// One block of AVX2 lane l of matvec_v4_fused: for g in 0..8, low nibble of
// byte g*8+l (activation G = g) then its high nibble (G = 8+g).
__device__ __forceinline__ float v4_exact_block(uint2 c, uint32_t p, const float* xl, float acc)
{
    const float zp = h2f(p & 0xFFFFu), sc = h2f(p >> 16);
    float xv[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float4 v = reinterpret_cast<const float4*>(xl)[q];
        xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const uint32_t w = g < 4 ? c.x : c.y;
        const uint32_t byte = (w >> (8 * (g & 3))) & 0xFFu;
        const float lo = (float)(byte & 15u), hi = (float)(byte >> 4);
        acc = __builtin_fmaf(__builtin_fmaf(lo, sc, zp), xv[g], acc);
        acc = __builtin_fmaf(__builtin_fmaf(hi, sc, zp), xv[8 + g], acc);
    }
    return acc;
}

// One block of AVX2 lane l of matvec_v3_fused: codes k = g*8+l for g in
// 0..16 in natural order. Low 4 bits: low-plane byte g (g < 8, low nibble)
// or byte g-8 (high nibble); top 2 bits: high-plane byte g&3, bits 2*(g>>2).
__device__ __forceinline__ float v3_exact_block(uint2 c, uint32_t h, uint32_t p, const float* xl,
                                                float acc)
{
    const float zp = h2f(p & 0xFFFFu), sc = h2f(p >> 16);
    float xv[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float4 v = reinterpret_cast<const float4*>(xl)[q];
        xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int g = 0; g < 16; g++) {
        const int gb = g & 7;
        const uint32_t w = gb < 4 ? c.x : c.y;
        const uint32_t byte = (w >> (8 * (gb & 3))) & 0xFFu;
        const uint32_t nib = g < 8 ? (byte & 15u) : (byte >> 4);
        const uint32_t top = (h >> (8 * (g & 3) + 2 * (g >> 2))) & 3u;
        const float code = (float)(nib | (top << 4));
        acc = __builtin_fmaf(__builtin_fmaf(code, sc, zp), xv[g], acc);
    }
    return acc;
}

template <int SCHEME>
__global__ __launch_bounds__(WG) void k_gemv_exact(const uint8_t* __restrict__ codes,
                                                   const uint8_t* __restrict__ hp,
                                                   const uint32_t* __restrict__ params,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ y, int rows, int nb)
{
    __shared__ __align__(16) float xs[SEG * XS_BLK];
    const int l = threadIdx.x & 7;
    const int row = blockIdx.x * (WG / 8) + (threadIdx.x >> 3);
    const bool active = row < rows;
    const size_t rb = (size_t)(active ? row : 0) * (size_t)nb;
    float acc = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += SEG) {
        const int nbs = min(SEG, nb - b0);
        __syncthreads();
        stage_x(xs, x, b0, nbs);
        __syncthreads();
        if (active) {
            const uint8_t* cp = codes + (rb + b0) * 64 + l * 8;
            const uint32_t* pp = params + rb + b0;
            const float* xl = xs + l * XS_LANE;
            if constexpr (SCHEME == 4) {
#pragma unroll 4
                for (int s = 0; s < nbs; s++) {
                    const uint2 c = *reinterpret_cast<const uint2*>(cp + (size_t)s * 64);
                    acc = v4_exact_block(c, pp[s], xl + s * XS_BLK, acc);
                }
            } else {
                const uint8_t* hq = hp + (rb + b0) * 32 + l * 4;
#pragma unroll 4
                for (int s = 0; s < nbs; s++) {
                    const uint2 c = *reinterpret_cast<const uint2*>(cp + (size_t)s * 64);
                    const uint32_t h = *reinterpret_cast<const uint32_t*>(hq + (size_t)s * 32);
                    acc = v3_exact_block(c, h, pp[s], xl + s * XS_BLK, acc);
                }
            }
        }
    }
    // hsum_avx2: s_l = a_l + a_{l^4}; t = s_l + s_{l^1}; r = t_l + t_{l^2}.
    // Float addition is commutative bit for bit, so lane 0 ends with
    // ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)).
    const float s4 = acc + __shfl_xor(acc, 4);
    const float s1 = s4 + __shfl_xor(s4, 1);
    const float r = s1 + __shfl_xor(s1, 2);
    if (active && l == 0) y[row] = bias ? r + bias[row] : r;
}

// Natural-order decode of row `row` (token), with the reference's two
// roundings: out[k] = zp + code*scale (wpc_weights_v4.rs:103-115).
template <int SCHEME>
__global__ __launch_bounds__(WG) void k_embed(const uint8_t* __restrict__ codes,
                                              const uint8_t* __restrict__ hp,
                                              const uint32_t* __restrict__ params,
                                              float* __restrict__ out, size_t row, int nb)
{
    const int k = blockIdx.x * WG + threadIdx.x;
    if (k >= nb * 128) return;
    const size_t blk = row * (size_t)nb + (size_t)(k >> 7);
    const int kk = k & 127;
    const uint32_t p = params[blk];
    // natural index kk -> lane l = kk & 7, group G = kk >> 3
    const int l = kk & 7, G = kk >> 3;
    const uint8_t byte = codes[blk * 64 + l * 8 + (G & 7)];
    uint32_t code = G < 8 ? (byte & 15u) : (byte >> 4);
    if (SCHEME == 3) {
        const uint8_t hb = hp[blk * 32 + l * 4 + (G & 3)];
        code |= ((hb >> (2 * (G >> 2))) & 3u) << 4;
    }
    out[k] = __fadd_rn(h2f(p & 0xFFFFu), __fmul_rn((float)code, h2f(p >> 16)));
}

template <int SCHEME>
__global__ __launch_bounds__(WG) void k_dequant(const uint8_t* __restrict__ codes,
                                                const uint8_t* __restrict__ hp,
                                                const uint32_t* __restrict__ params,
                                                float* __restrict__ w, size_t n, int nb,
                                                int rounding)
{
    const size_t i = (size_t)blockIdx.x * WG + threadIdx.x;
    if (i >= n) return;
    const size_t blk = i >> 7;
    const int kk = (int)(i & 127);
    const uint32_t p = params[blk];
    const int l = kk & 7, G = kk >> 3;
    const uint8_t byte = codes[blk * 64 + l * 8 + (G & 7)];
    uint32_t code = G < 8 ? (byte & 15u) : (byte >> 4);
    if (SCHEME == 3) {
        const uint8_t hb = hp[blk * 32 + l * 4 + (G & 3)];
        code |= ((hb >> (2 * (G >> 2))) & 3u) << 4;
    }
    const float zp = h2f(p & 0xFFFFu), sc = h2f(p >> 16);
    w[i] = rounding == WPCG_ROUND_FMA ? __builtin_fmaf((float)code, sc, zp)
                                      : __fadd_rn(zp, __fmul_rn((float)code, sc));
    (void)nb;
}

}  // namespace

hipError_t launch_gemv(const DeviceMatrix& m, int mode, const float* x, const float* bias,
                       float* y, hipStream_t s)
{
    (void)mode;
    const int rows = (int)m.rows, nb = (int)m.nb;
    dim3 grid((unsigned)((m.rows + WG / 8 - 1) / (WG / 8)));
    if (m.scheme == 4)
        hipLaunchKernelGGL(k_gemv_exact<4>, grid, dim3(WG), 0, s, m.codes, m.hp, m.params, x,
                           bias, y, rows, nb);
    else
        hipLaunchKernelGGL(k_gemv_exact<3>, grid, dim3(WG), 0, s, m.codes, m.hp, m.params, x,
                           bias, y, rows, nb);
    return hipGetLastError();
}

hipError_t launch_embed(const DeviceMatrix& m, uint32_t row, float* out, hipStream_t s)
{
    dim3 grid((unsigned)((m.cols + WG - 1) / WG));
    if (m.scheme == 4)
        hipLaunchKernelGGL(k_embed<4>, grid, dim3(WG), 0, s, m.codes, m.hp, m.params, out,
                           (size_t)row, (int)m.nb);
    else
        hipLaunchKernelGGL(k_embed<3>, grid, dim3(WG), 0, s, m.codes, m.hp, m.params, out,
                           (size_t)row, (int)m.nb);
    return hipGetLastError();
}

hipError_t launch_dequant(const DeviceMatrix& m, int rounding, float* w, hipStream_t s)
{
    const size_t n = (size_t)m.rows * m.cols;
    dim3 grid((unsigned)((n + WG - 1) / WG));
    if (m.scheme == 4)
        hipLaunchKernelGGL(k_dequant<4>, grid, dim3(WG), 0, s, m.codes, m.hp, m.params, w, n,
                           (int)m.nb, rounding);
    else
        hipLaunchKernelGGL(k_dequant<3>, grid, dim3(WG), 0, s, m.codes, m.hp, m.params, w, n,
                           (int)m.nb, rounding);
    return hipGetLastError();
}

}  // namespace wpcg
