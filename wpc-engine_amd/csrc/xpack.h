// The batched GEMM's packed X: bf16 fragments in the matrix cores' k order
// plus per-block column sums (the format k_gemm_pack writes and k_gemm
// reads). Shared by the GEMM and by the prefill kernels that produce a
// GEMM's X and write it packed themselves.
//
// k order: for kstep i (0..3) the lanes of group g (lanes 16g..16g+15) feed
// the eight values k(i, g, s) = 8s + g + 4(i & 1) + 64(i >> 1), s = 0..7, of
// a 128-value block; fragment (block b, column tile n, kstep i) is 64 lanes
// x 8 bf16, lane g*16 + c holding column n*16 + c. In the SPLIT form a
// group of four column tiles holds two tiles of hi = bf16(x) and then the
// same two columns' lo = bf16(x - hi).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace wpcg {

__device__ __forceinline__ int gk(int i, int g, int s) { return 8 * s + g + 4 * (i & 1) + 64 * (i >> 1); }

// Two floats to packed bf16 (round to nearest even), low half first.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b)
{
    typedef float xp_f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 xp_bf16x2 __attribute__((ext_vector_type(2)));
    const xp_f32x2 f = {a, b};
    const xp_bf16x2 h = __builtin_convertvector(f, xp_bf16x2);
    uint32_t r;
    __builtin_memcpy(&r, &h, 4);
    return r;
}
__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }
// x rounded to bf16 (nearest even), as a float
__device__ __forceinline__ float bf16_round(float v) { return bf16_lo(pk_bf16(v, 0.0f)); }

// One 16-column tile of fp32 X, staged in LDS as tile[c * stride + k]
// (column c, k < 128 of block b), to the SPLIT packed form: column tile t16
// of the block is hi tile 4 (t16 / 2) + t16 % 2 and lo tile + 2, of the XT
// tiles per block. Columns c >= valid are written as zeros. Called by all
// 256 threads of the workgroup (thread 64i + 16g + c: kstep i, lane group g,
// column c); red is 2 x 4 x 16 floats of LDS; ends with a barrier.
__device__ __forceinline__ void pack_tile_split(const float* tile, int stride, int valid, int b, int t16, int XT,
                                                uint32_t* xf, float* xsum, float (*red)[4][16])
{
    const int i = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const int n_hi = 4 * (t16 >> 1) + (t16 & 1), n_lo = n_hi + 2;
    float v[8], w[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        v[s] = c < valid ? tile[c * stride + gk(i, g, s)] : 0.0f;
        w[s] = v[s] - bf16_round(v[s]);  // exact in fp32
    }
    const uint32_t h0 = pk_bf16(v[0], v[1]), h1 = pk_bf16(v[2], v[3]), h2 = pk_bf16(v[4], v[5]),
                   h3 = pk_bf16(v[6], v[7]);
    const uint32_t l0 = pk_bf16(w[0], w[1]), l1 = pk_bf16(w[2], w[3]), l2 = pk_bf16(w[4], w[5]),
                   l3 = pk_bf16(w[6], w[7]);
    typedef unsigned xp_u32x4 __attribute__((ext_vector_type(4)));
    reinterpret_cast<xp_u32x4*>(xf)[((size_t)(b * XT + n_hi) * 4 + i) * 64 + lane] = xp_u32x4{h0, h1, h2, h3};
    reinterpret_cast<xp_u32x4*>(xf)[((size_t)(b * XT + n_lo) * 4 + i) * 64 + lane] = xp_u32x4{l0, l1, l2, l3};
    float sh = ((bf16_lo(h0) + bf16_hi(h0)) + (bf16_lo(h1) + bf16_hi(h1))) +
               ((bf16_lo(h2) + bf16_hi(h2)) + (bf16_lo(h3) + bf16_hi(h3)));
    float sl = ((bf16_lo(l0) + bf16_hi(l0)) + (bf16_lo(l1) + bf16_hi(l1))) +
               ((bf16_lo(l2) + bf16_hi(l2)) + (bf16_lo(l3) + bf16_hi(l3)));
    sh += __shfl_xor(sh, 16);
    sh += __shfl_xor(sh, 32);
    sl += __shfl_xor(sl, 16);
    sl += __shfl_xor(sl, 32);
    if (g == 0) {
        red[0][i][c] = sh;
        red[1][i][c] = sl;
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        const int p = threadIdx.x >> 4, cc = threadIdx.x & 15;
        xsum[(size_t)b * XT * 16 + (p ? n_lo : n_hi) * 16 + cc] =
            (red[p][0][cc] + red[p][1][cc]) + (red[p][2][cc] + red[p][3][cc]);
    }
    __syncthreads();
}

}  // namespace wpcg
