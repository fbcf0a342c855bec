// Dequant-GEMV kernels for gfx950 (CDNA4, wave64) over WPC blocks of 128
// weights (v4: 4-bit codes, v3: 6-bit codes in two planes). Device layout:
// see wpcg_internal.hpp (per 16-row tile and block, one contiguous record of
// code bytes in paired-lane order, one of high bits, one of parameters).
//
// EXACT mode reproduces the reference's AVX2 row kernels bit for bit:
//   matvec_v4_fused (wpc-eval/src/fused_kernel.rs:237-271)
//   matvec_v3_fused (wpc-eval/src/fused_kernel.rs:163-189)
// Eight threads own one output row; thread L is AVX2 lane L. For every block
// in order it runs the lane's chain w = fma(code, scale, zp),
// acc = fma(w, x, acc) over the same weights in the same order, and the
// eight accumulators are combined in hsum_avx2's order
// ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) with xor-shuffles 4, 1, 2.
//
// FAST mode puts the dot products on the matrix cores. Codes are exact int8
// (0..15 or 0..63). Each 128-value block b of x is written as
//   x ~= s_b * Q / 2^21,  s_b = max|x_b| / 127,  Q = rint(x * 127*2^21 / max|x_b|)
// and Q = d0*2^21 + d1*2^14 + d2*2^7 + d3 with int8 digits d0 = Q >> 21 in
// [-128,127], d1..d3 in [0,127]. v_mfma_i32_16x16x64_i8 then gives the exact integer
// dots D_j = sum(code * d_j) of the four digits with each row of a 16-row
// tile (the digits are the first operand, so one lane receives all four
// of its row), and each block adds
//   scale * s_b * (D0 + D1*2^-7 + D2*2^-14 + D3*2^-21) + zp * sum(x_b)
// to the row's fp32 accumulators (the digit sum by Horner's rule). The
// only approximation is x's representation: the fp32 product x*127*2^21/m
// (relative 6e-8, as fp32 itself) plus 0.5*s_b*2^-21 = 1.9e-9 * max|x_b|,
// which keeps the small values of a block that holds an outlier accurate.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "route_exact.h"
#include "wpcg_internal.hpp"
#include "wave.h"

namespace wpcg {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Byte of row r (of its tile) that AVX2 lane L reads first, within a block's
// code record (1 KiB) or high-plane record (512 B).
__device__ __forceinline__ int dcode_pos(int r, int L) { return ((L & 3) * 16 + r) * 16 + (L >> 2) * 8; }
__device__ __forceinline__ int dhp_pos(int r, int L) { return ((L & 3) * 16 + r) * 8 + (L >> 2) * 4; }
__device__ __forceinline__ size_t param_idx(size_t row, size_t nb, size_t blk)
{
    return ((row / TILE_ROWS) * nb + blk) * TILE_ROWS + row % TILE_ROWS;
}

__device__ __forceinline__ float h2f(uint32_t bits)
{
    _Float16 h;
    uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// A pointer that is the same in every lane, as a wave-uniform value.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p)
{
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// Buffer resource over [base, base + bytes): raw buffer loads at offsets
// past `bytes` return zeros and access no memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
constexpr int CPOL_NT = 2;  // non-temporal: streamed weights are read once

// ============================================================ EXACT mode
constexpr int XS_LANE = 20;  // floats per AVX lane in LDS (bank spread)
constexpr int XS_BLK = 8 * XS_LANE;
constexpr int EX_SEG = 32;   // blocks of x per LDS pass (20 KiB)
constexpr int EX_WG = 128;   // 16 rows x 8 lanes

// x staged as xs[s*XS_BLK + L*XS_LANE + G] = x[(b0+s)*128 + G*8 + L]: the 16
// activations AVX lane L uses, in the order it uses them. Every 16-byte load
// of the segment is issued before the first store (range-checked: none past
// the segment's nbs blocks).
__device__ __forceinline__ void stage_x(float* xs, const float* __restrict__ x, int b0, int nbs)
{
    constexpr int PER = EX_SEG * 128 / 4 / EX_WG;  // float4s per thread
    const auto xr = buf_rsrc(x + (size_t)b0 * 128, nbs * 512);
    u32x4 v[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) v[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, (threadIdx.x + u * EX_WG) * 16, 0, 0);
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = 4 * (threadIdx.x + u * EX_WG);  // first of four consecutive values
        if (i < nbs * 128) {
            const int s = i >> 7, r = i & 127;
            float* d = xs + s * XS_BLK + (r >> 3);
            d[((r + 0) & 7) * XS_LANE] = __uint_as_float(v[u].x);
            d[((r + 1) & 7) * XS_LANE] = __uint_as_float(v[u].y);
            d[((r + 2) & 7) * XS_LANE] = __uint_as_float(v[u].z);
            d[((r + 3) & 7) * XS_LANE] = __uint_as_float(v[u].w);
        }
    }
}

__device__ __forceinline__ void load16(const float* xl, float xv[16])
{
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float4 v = reinterpret_cast<const float4*>(xl)[q];
        xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
    }
}

// float of byte B of w (one v_cvt_f32_ubyteB)
template <int B>
__device__ __forceinline__ float byte_f(uint32_t w) { return (float)((w >> (8 * B)) & 0xFFu); }
// the same as one instruction the compiler keeps: from a masked word it
// would otherwise extract each nibble again (bit-field extract + convert)
template <int B>
__device__ __forceinline__ float byte_cvt(uint32_t w)
{
    float r;
    if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
    else if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
    else if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w));
    return r;
}

// AVX2 lane L of matvec_v4_fused over one block: for g in 0..8, the low
// nibble of ref byte g*8+L (activation G = g), then its high nibble (G = 8+g).
// The nibbles are masked four at a time into bytes, each then one byte
// conversion (per block 22 instructions for the 16 codes instead of 28
// bit-field extracts and conversions).
__device__ __forceinline__ float v4_exact_block(uint2 c, uint32_t p, const float* xl, float acc)
{
    const float zp = h2f(p & 0xFFFFu), sc = h2f(p >> 16);
    float xv[16];
    load16(xl, xv);
    const uint32_t M = 0x0F0F0F0Fu;
    const uint32_t lx = c.x & M, ly = c.y & M, hx = (c.x >> 4) & M, hy = (c.y >> 4) & M;
    const float lo[8] = {byte_cvt<0>(lx), byte_cvt<1>(lx), byte_cvt<2>(lx), byte_cvt<3>(lx),
                         byte_cvt<0>(ly), byte_cvt<1>(ly), byte_cvt<2>(ly), byte_cvt<3>(ly)};
    const float hi[8] = {byte_cvt<0>(hx), byte_cvt<1>(hx), byte_cvt<2>(hx), byte_cvt<3>(hx),
                         byte_cvt<0>(hy), byte_cvt<1>(hy), byte_cvt<2>(hy), byte_cvt<3>(hy)};
#pragma unroll
    for (int g = 0; g < 8; g++) {
        acc = __builtin_fmaf(__builtin_fmaf(lo[g], sc, zp), xv[g], acc);
        acc = __builtin_fmaf(__builtin_fmaf(hi[g], sc, zp), xv[8 + g], acc);
    }
    return acc;
}

// AVX2 lane L of matvec_v3_fused over one block: codes k = G*8+L for G in
// 0..16, natural order. Low 4 bits: low-plane byte G (G < 8, low nibble) or
// G-8 (high nibble); top 2 bits: high-plane byte G&3, bits 2*(G>>2). Four
// codes are assembled per dword (nibbles masked, top bits shifted into bits
// 4-5 of each byte), each then one byte conversion.
__device__ __forceinline__ float v3_exact_block(uint2 c, uint32_t h, uint32_t p, const float* xl,
                                                float acc)
{
    const float zp = h2f(p & 0xFFFFu), sc = h2f(p >> 16);
    float xv[16];
    load16(xl, xv);
    const uint32_t M = 0x0F0F0F0Fu, T = 0x30303030u;
    // G = 0..3, 4..7, 8..11, 12..15
    const uint32_t d0 = (c.x & M) | ((h << 4) & T), d1 = (c.y & M) | ((h << 2) & T);
    const uint32_t d2 = ((c.x >> 4) & M) | (h & T), d3 = ((c.y >> 4) & M) | ((h >> 2) & T);
    const float code[16] = {byte_f<0>(d0), byte_f<1>(d0), byte_f<2>(d0), byte_f<3>(d0),
                            byte_f<0>(d1), byte_f<1>(d1), byte_f<2>(d1), byte_f<3>(d1),
                            byte_f<0>(d2), byte_f<1>(d2), byte_f<2>(d2), byte_f<3>(d2),
                            byte_f<0>(d3), byte_f<1>(d3), byte_f<2>(d3), byte_f<3>(d3)};
#pragma unroll
    for (int G = 0; G < 16; G++) acc = __builtin_fmaf(__builtin_fmaf(code[G], sc, zp), xv[G], acc);
    return acc;
}

// One 16-row tile (workgroup-local index `tile`) of an EXACT GEMV. With
// `sel` set, the planes stack experts of rows_pad rows each and the GEMV is
// expert sel[sel_k]'s (a negative id writes y = 0).
template <int SCHEME>
__device__ __forceinline__ void gemv_exact_tile(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ hp,
                                                const uint32_t* __restrict__ params, const float* __restrict__ x,
                                                const float* __restrict__ bias, float* __restrict__ y, int rows,
                                                int nb, const int32_t* __restrict__ sel, int sel_k, int rows_pad,
                                                int tile, float* xs)
{
    if (sel) {
        const int e = __builtin_amdgcn_readfirstlane(sel[sel_k]);
        if (e < 0) {
            const int r = tile * (EX_WG / 8) + (threadIdx.x >> 3);
            if (r < rows && (threadIdx.x & 7) == 0) y[r] = 0.0f;
            return;
        }
        const size_t t0 = (size_t)e * (rows_pad / TILE_ROWS) * nb;
        codes += t0 * CODE_REC;
        if (SCHEME == 3) hp += t0 * HP_REC;
        params += t0 * TILE_ROWS;
    }
    // The planes' addresses are the same for every lane, but the early exit
    // above (a store by some lanes, then return) makes the compiler carry
    // them in lane registers; buffer resources built from those made every
    // load of the batched kernel a loop over lanes (q/k/v: 4.8 us to issue
    // them). Taken from the first lane they are uniform again.
    codes = uniform_ptr(codes);
    hp = uniform_ptr(hp);
    params = uniform_ptr(params);
    const int L = threadIdx.x & 7;
    const int r16 = threadIdx.x >> 3;  // row within the tile
    const int row = tile * (EX_WG / 8) + r16;
    const bool active = row < rows;
    const size_t tb = (size_t)tile * (size_t)nb;  // this tile's first block record
    // the tile's records: per block, the workgroup reads one contiguous 1 KiB
    // code record (v3: and a 512 B high-plane record) and 64 B of parameters
    const auto crs = buf_rsrc(codes + tb * CODE_REC, nb * (int)CODE_REC);
    const auto hrs = buf_rsrc((SCHEME == 3 ? hp : codes) + tb * HP_REC, SCHEME == 3 ? nb * (int)HP_REC : 0);
    const auto prs = buf_rsrc(params + tb * TILE_ROWS, nb * TILE_ROWS * 4);
    const int coff = dcode_pos(r16, L), hoff = dhp_pos(r16, L), poff = r16 * 4;
    float acc = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += EX_SEG) {
        const int nbs = min(EX_SEG, nb - b0);
        // every load of the segment first (range-checked: none past the
        // row), so their latency overlaps the staging of x and each other
        uint2 c[EX_SEG];
        uint32_t h[EX_SEG], p[EX_SEG];
#pragma unroll
        for (int s = 0; s < EX_SEG; s++) {
            if (s < nbs) {  // uniform
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(crs, (b0 + s) * (int)CODE_REC + coff, 0, CPOL_NT);
                c[s] = make_uint2(v.x, v.y);
                if constexpr (SCHEME == 3)
                    h[s] = __builtin_amdgcn_raw_buffer_load_b32(hrs, (b0 + s) * (int)HP_REC + hoff, 0, CPOL_NT);
                p[s] = __builtin_amdgcn_raw_buffer_load_b32(prs, (b0 + s) * TILE_ROWS * 4 + poff, 0, CPOL_NT);
            }
        }
        __syncthreads();
        stage_x(xs, x, b0, nbs);
        __syncthreads();
        const float* xl = xs + L * XS_LANE;
#pragma unroll
        for (int s = 0; s < EX_SEG; s++) {
            if (s < nbs) {  // uniform
                if constexpr (SCHEME == 4)
                    acc = v4_exact_block(c[s], p[s], xl + s * XS_BLK, acc);
                else
                    acc = v3_exact_block(c[s], h[s], p[s], xl + s * XS_BLK, acc);
            }
        }
    }
    // hsum_avx2: s_L = a_L + a_{L^4}; t = s_L + s_{L^1}; r = t_L + t_{L^2}.
    // Float addition is commutative bit for bit, so lane 0 ends with
    // ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)).
    const float s4 = acc + __shfl_xor(acc, 4);
    const float s1 = s4 + __shfl_xor(s4, 1);
    const float r = s1 + __shfl_xor(s1, 2);
    if (active && L == 0) y[row] = bias ? r + bias[row] : r;
}

template <int SCHEME>
__global__ __launch_bounds__(EX_WG) void k_gemv_exact(const uint8_t* __restrict__ codes,
                                                      const uint8_t* __restrict__ hp,
                                                      const uint32_t* __restrict__ params,
                                                      const float* __restrict__ x,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, int rows, int nb,
                                                      const int32_t* __restrict__ sel, int sel_k,
                                                      int rows_pad)
{
    __shared__ __align__(16) float xs[EX_SEG * XS_BLK];
    gemv_exact_tile<SCHEME>(codes, hp, params, x, bias, y, rows, nb, sel, sel_k, rows_pad, blockIdx.x, xs);
}

// Several EXACT GEMVs (same scheme) in one launch: workgroup (x, y) runs
// tile x of problem y exactly as k_gemv_exact would (x < the problem's nwg;
// the grid is as wide as the largest problem). The problem index comes from
// the grid, so a workgroup reads its problem's fields in one round trip.
struct ExactProblem {
    const uint8_t* codes;
    const uint8_t* hp;
    const uint32_t* params;
    const float* x;
    const float* bias;
    float* y;
    const int32_t* sel;
    int rows, nb, sel_k, rows_pad, nwg;
    // With scores set the workgroup routes itself (softmax and top_k of the
    // n_exp router scores, the reference's arithmetic) and takes slot sel_k
    // of the result as its expert; workgroup (0, 0) also stores the ids and
    // weights at ids_out / w_out for the launches after it.
    const float* scores;
    int32_t* ids_out;
    float* w_out;
    int n_exp, top_k, norm_topk;
};
struct ExactBatch {
    ExactProblem p[MAX_JOBS];
    int n;
};
static_assert(sizeof(ExactBatch) <= 4096, "kernel arguments of a batched EXACT launch");

template <int SCHEME>
__global__ __launch_bounds__(EX_WG) void k_gemv_exact_multi(const ExactBatch B)
{
    __shared__ __align__(16) float xs[EX_SEG * XS_BLK];
    __shared__ __align__(16) float route_e[64 * RT_PER];
    __shared__ int32_t route_ids[MAX_JOBS];
    __shared__ float route_w[MAX_JOBS];
    __shared__ double route_tab[32];
    // (the problem is read through the kernel-argument segment: indexing the
    // by-value argument with a variable would copy it to scratch memory)
    typedef const __attribute__((address_space(4))) ExactBatch* KargPtr;
    const KargPtr kargs = (KargPtr)__builtin_amdgcn_kernarg_segment_ptr();
    const auto& P = kargs->p[blockIdx.y];
    const uint8_t* const codes = P.codes;
    const uint32_t* const params = P.params;
    const float* const x = P.x;
    const int nb = P.nb, rows_pad = P.rows_pad, nwg = P.nwg;
    // these loads go out together, before the exit test below needs nwg
    asm volatile("" ::"s"(codes), "s"(params), "s"(x), "s"(nb), "s"(rows_pad), "s"(nwg));
    if ((int)blockIdx.x >= nwg) return;  // past this problem's tiles
    const int32_t* sel = P.sel;
    if (const float* scores = P.scores) {  // uniform: this workgroup routes itself
        // (in place of a routing launch before this one, 8.6 us per MoE
        // layer; here it runs before the weight loads can be addressed)
        if (threadIdx.x < 64)
            softmax_route_wave(scores, P.n_exp, P.top_k, P.norm_topk, route_ids, route_w, route_e, route_tab);
        __syncthreads();
        if (blockIdx.x == 0 && blockIdx.y == 0 && (int)threadIdx.x < P.top_k) {
            P.ids_out[threadIdx.x] = route_ids[threadIdx.x];
            P.w_out[threadIdx.x] = route_w[threadIdx.x];
        }
        sel = route_ids;
    }
    gemv_exact_tile<SCHEME>(codes, P.hp, params, x, P.bias, P.y, P.rows, nb, sel, P.sel_k, rows_pad, blockIdx.x,
                            xs);
}

// ============================================================ FAST mode

struct FastProblem {
    const uint8_t* codes;
    const uint8_t* hp;
    const uint32_t* params;
    const float* x;      // x; for XF_SILU the gate values g
    const float* x2;     // XF_SILU: the up values u
    const float* nw;     // XF_NORM: the RMSNorm weights
    float* y;
    const float* bias;
    float* part;
    uint32_t* counters;
    // Expert selection: with sel set, the matrix stacks experts of rows_pad
    // rows each and this problem is expert sel[sel_k] (its rows only; a
    // negative id gives y = 0). With `scores` set instead, the workgroup
    // routes itself (softmax and top_k of the n_exp router scores) and takes
    // slot sel_k of the result; workgroup 0 of the launch also stores the
    // ids and weights at ids_out / w_out.
    const int32_t* sel;
    const float* rw;     // routed: the routing weight of each slot
    const float* scores;
    int32_t* ids_out;
    float* w_out;
    int rows, rows_pad, nb, kg, nwg, tw;  // nwg: workgroups; tw: 16-row tiles per workgroup
    const DecodeState* st;  // XF_MERGE: the decode position
    int sel_k, xform, routed, n_exp, top_k, norm_topk;
    float eps;
    int enb;  // routed: blocks per row of one expert (nb = top_k * enb)
    int head_dim, n_heads;  // XF_MERGE
    // set by the host so that the kernel divides nothing: blocks per K-slice
    // ceil(nb / kg), log2 of tw, and ceil(2^32 / kg) (0 when kg = 1) for
    // workgroup / kg as a multiply-high (exact for workgroups < 2^16)
    int nbk, ltw;
    uint32_t kg_inv;
    // deferred K-split: slice k >= 1 writes its sum to y2 + (k-1)*rows;
    // XF_NORM adds the n_xa vectors at x_add (stride nb*128) to x; the bias
    // is bias + the n_b2 vectors at bias2 (stride rows)
    float* y2;
    const float* x_add;
    const float* bias2;
    int n_xa, n_b2;
    uint64_t* amax;  // one K-slice: workgroup w's key of its first largest row
};
struct FastBatch {
    FastProblem p[MAX_JOBS];
    int n;
};
static_assert(sizeof(FastBatch) <= 4096, "kernel arguments of a FAST launch");

constexpr int FAST_WG = 512;        // 8 waves
constexpr int QB = 8;               // most blocks one wave puts through the matrix cores
constexpr int MG = 2;               // blocks per branch-free group of the matrix-core loop
constexpr int NDIG = 4;             // int8 digits per x value
constexpr int HALF = 4 * NDIG * 16; // fragment bytes per MFMA half: 4 groups x digits x 16
constexpr int FRAG = 2 * HALF;      // per block
constexpr int MAXBK = FAST_MAXBK;   // most blocks of one K-slice (one tile per workgroup)
static_assert(MAXBK == QB * 8, "slice = 8 waves x QB blocks");

// Byte position of digit 0 of x index k (0..127) in a block's fragment area.
// MFMA half h = k>>6 covers 64 k; lane group g = k&3; byte (k>>3)&7 + 8*((k>>2)&1).
// This is the inverse of the A-operand packing below, in which lane group g
// holds AVX lanes g and g+4 of a block (16 packed bytes). Digit j of the same
// value sits 16*j bytes further.
__device__ __forceinline__ int frag_pos(int k)
{
    return (k >> 6) * HALF + (k & 3) * (NDIG * 16) + ((k >> 3) & 7) + 8 * ((k >> 2) & 1);
}


// DPP lane exchange inside rows of 16 lanes (full row and bank masks).
template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <-> 7-i within each 8
constexpr int DPP_MIRROR = 0x140;      // lane i <-> 15-i within each 16


__device__ __forceinline__ float lane_of(float v, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Softmax of n <= PER*64 router scores and the top-k selection of route()
// (qwen3_moe_model.rs:376-402) by the workgroup, into LDS: ids[k], w[k] for
// k < top_k (id -1, weight 0 for a slot no selectable expert fills); every
// thread calls it. Wave 0 computes the probabilities (softmax_inplace's
// steps, norm.rs:28-43, in FAST arithmetic like the router scores
// themselves: the hardware exp of x log2(e) and one reciprocal of the tree
// sum; EXACT's k_softmax_route keeps the reference's arithmetic) and a key
// per expert, bits(p) << 32 | ~index (p >= 0: larger p first, then the lower
// index; NaN never chosen, key 0); the rank of a key is how many keys beat
// it, which is the order of route()'s repeated strict-`>` scans. Each wave
// ranks an eighth of the keys: a lane counts the keys of one part of the
// array that beat its key (LDS reads every lane of a group shares), the
// parts' counts are added across lanes, and a selectable key of rank
// r < top_k writes slot r. Returns the number of selectable experts
// (wave 0; others 0). LDS: key (PER*64 keys).
template <int PER>
__device__ __forceinline__ int route_wg(const float* __restrict__ scores, int n, int top_k, uint64_t* key_lds,
                                        int32_t* ids, float* w)
{
    constexpr int N = PER * 64, KPW = N / 8, G = 64 / KPW;  // keys per wave, lane groups
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int selectable = 0;
    if (wave == 0) {
        float v[PER];
#pragma unroll
        for (int q = 0; q < PER; q++) v[q] = scores[min(lane + 64 * q, n - 1)];
        float m = -INFINITY;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            if (lane + 64 * q >= n) v[q] = -INFINITY;
            m = fmaxf(m, v[q]);
        }
        m = wave_max(m);
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            v[q] = lane + 64 * q < n ? __expf(__fsub_rn(v[q], m)) : 0.0f;
            sum += v[q];
        }
        sum = wave_sum(sum);
        const float rs = sum > 0.0f ? __builtin_amdgcn_rcpf(sum) : 1.0f;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int i = lane + 64 * q;
            v[q] *= rs;
            const bool ok = i < n && v[q] > -INFINITY;  // NaN fails
            key_lds[i] = ok ? ((uint64_t)__float_as_uint(v[q]) << 32) | (0xFFFFFFFFu - (uint32_t)i) : 0ull;
            selectable += __popcll(__ballot(ok));
        }
        if (lane < top_k) {
            ids[lane] = -1;
            w[lane] = 0.0f;
        }
    }
    __syncthreads();
    {
        const int i = wave * KPW + lane % KPW;
        const uint64_t mine = key_lds[i];
        const uint64_t* part = key_lds + (lane / KPW) * (N / G);
        int cnt = 0;
#pragma unroll
        for (int u = 0; u < N / G; u += 2) {
            const ulonglong2 pr = *reinterpret_cast<const ulonglong2*>(part + u);
            cnt += (pr.x > mine ? 1 : 0) + (pr.y > mine ? 1 : 0);
        }
        if constexpr (G >= 4) cnt += __shfl_xor(cnt, 16);
        if constexpr (G >= 2) cnt += __shfl_xor(cnt, 32);
        if (lane < KPW && mine && cnt < top_k) {
            ids[cnt] = i;
            w[cnt] = __uint_as_float((uint32_t)(mine >> 32));
        }
    }
    __syncthreads();
    return selectable;
}

// A workgroup of 8 waves computes tw (1, 2 or 4) 16-row tiles over one K-slice
// of nbl <= 8*QB/tw blocks.
//   prep:  the slice's x becomes int8 digit fragments in LDS, shared by all
//          waves; a wave takes two blocks at a time (32 lanes, 4 values each).
//   dots:  wave w works on tile w / kw (kw = 8/tw waves per tile) over the
//          contiguous kq-th part of the slice (kq = w % kw), in branch-free
//          groups of MG blocks: a block past the part's end reads zeros
//          everywhere and adds exactly 0, and the groups' LDS reads, MFMAs
//          and scaling overlap (groups of two waste fewer slots on a part
//          of 5 or 7 blocks than groups of four and measured faster).
//   sum:   the kw parts of a tile are added in part order (deterministic).
// Input transforms, applied to x in the prep (FAST mode only):
//   XF_NORM  x' = x * nw, and the row's result is scaled by
//            1 / sqrt(mean(x^2) + eps): RMSNorm (norm.rs:4-13) folded into
//            the GEMV (a single K-slice holds the whole row);
//   XF_SILU  x' = silu(g) * u (qwen3_moe_model.rs:518-522), times the
//            slot's routing weight in a routed problem;
//   XF_MERGE x' = the attention output of head h = k / head_dim, merged
//            from the chunk states the FAST attention left:
//            sum_c e^(m_c - M) o_c[k] / sum_c e^(m_c - M) l_c, M = max_c m_c,
//            over the chunks that held positions at this step.
// A routed problem (the MoE down projection of all chosen experts) has the
// chosen experts' rows side by side: its K is top_k * enb blocks, block b
// being block b % enb of expert sel[b / enb] with x from slot b / enb's g,
// u and routing weight. One K-slice holds them all, so the row sum is the
// weighted combine sum_k w_k W_k h_k of the chosen experts
// (qwen3_moe_model.rs:526-533) with no cross-workgroup handoff.
// KIND: FK_PLAIN (a stacked matrix's expert may still come from sel),
// FK_ROUTE (the workgroup routes itself from router scores) or FK_ROUTED
// (the routed down projection); all problems of a launch share it.
// XF: the input transform (XF_NONE, XF_NORM, XF_SILU), also shared by the
// launch's problems.
constexpr int FK_PLAIN = 0, FK_ROUTE = 1, FK_ROUTED = 2;
// XPN: x pairs (two blocks) per wave the registers hold, MAXBK / 16 for a
// full slice; the norm-folding plain GEMV of slices of at most 32 blocks
// (the decode's q/k/v, gate/up and lm_head) uses 2, which fits six waves per
// SIMD (three workgroups per CU) without spilling.
template <int SCHEME, int KIND, int XF, int XPN = MAXBK / 16>
// The plain GEMV asks for 6 waves per SIMD (at most 80 VGPRs): three
// workgroups per CU instead of two, so a launch of up to 768 workgroups
// runs in one round (2x9728x2560 v3: 12.5 -> 11.1 us). The routing kinds
// keep their registers (their routing state would spill).
__global__ __launch_bounds__(FAST_WG, KIND == FK_PLAIN && (XF == XF_NONE || (XF == XF_NORM && XPN == 2)) ? 6 : 1) void k_gemv_fast(const FastBatch B)
{
    // A wave's last group of MG may reach up to MG-1 blocks past the slice:
    // those blocks' codes are zero, their digits are never written (any
    // int8 is harmless) and their scales are zeroed below (a stale NaN is not).
    __shared__ __align__(16) int8_t xq[(MAXBK + 4) * FRAG];     // digits of the slice
    __shared__ __align__(8) float2 xs[MAXBK + 4];              // {s_b, sum(x_b)}
    __shared__ __align__(16) uint32_t spar[8][QB * TILE_ROWS]; // parameters, per wave
    __shared__ float red[8][TILE_ROWS];
    __shared__ float ssq[8];                                    // XF_NORM: sum of x^2 per wave
    __shared__ int32_t route_ids[MAX_JOBS];                     // FK_ROUTE: the routing
    __shared__ float route_w[MAX_JOBS];
    __shared__ int s_last;
    // FK_ROUTE's keys live in xq, which routing finishes with before the
    // barrier that ends it (the x prep writes xq after it)
    uint64_t* const route_key = reinterpret_cast<uint64_t*>(xq);

    // Workgroup (x, y) is workgroup x of problem y: the problem index comes
    // from the grid, so the problem's fields are read in one round trip (a
    // search over the problems' workgroup ranges cost two more, ~0.85 us per
    // launch). The problem is read through the kernel-argument segment
    // (indexing the by-value argument with a variable would copy it to
    // scratch memory). The grid is as wide as the largest problem.
    typedef const __attribute__((address_space(4))) FastBatch* KargPtr;
    const KargPtr kargs = (KargPtr)__builtin_amdgcn_kernarg_segment_ptr();
    const auto& P = kargs->p[blockIdx.y];
    const int local = blockIdx.x;
    const int nb = P.nb, kg = P.kg, tw = P.tw, nwg = P.nwg, rows_pad = P.rows_pad;
    constexpr int xform = XF;
    const uint8_t* codes = P.codes;
    const uint8_t* hplane = SCHEME == 3 ? P.hp : P.codes;
    const uint32_t* params = P.params;
    const float* const x0 = P.x;
    // these loads go out together, before the exit test below needs nwg
    const int nbk_ = P.nbk, ltw_ = P.ltw;
    const uint32_t kg_inv_ = P.kg_inv;
    // The fields the end phase reads. The plain GEMV requests them with the
    // others (read at the end, each was a dependent scalar round trip in the
    // launch's tail: cfg1 step 29.59 -> 29.40 us); the transform kinds, which
    // hold more fields already, read them at the end (requested here too,
    // they made the dense Qwen3-4B-shaped decode 739 -> 724 tok/s).
    float* const out_y = P.y;
    const float* const out_bias = P.bias;
    float* const out_y2 = P.y2;
    const float* const out_bias2 = P.bias2;
    const int out_rows = P.rows, out_nb2 = P.n_b2;
    uint64_t* const out_amax = P.amax;
    // With them, the fields each kind reads before its weight loads (read
    // where they are used, each was a further dependent round trip): one
    // statement, so that one wait covers them all.
    {
        const float* f0 = XF == XF_NORM ? P.x_add : XF == XF_SILU || XF == XF_MERGE ? P.x2 : nullptr;
        const float* f1 = XF == XF_NORM ? P.nw : KIND == FK_ROUTE ? P.scores : KIND == FK_ROUTED ? P.rw : nullptr;
        const int32_t* f2 = KIND != FK_ROUTE ? P.sel : nullptr;
        const int i0 = XF == XF_MERGE ? P.head_dim : KIND == FK_ROUTE ? P.n_exp : KIND == FK_ROUTED ? P.enb : 0;
        const int i1 = XF == XF_MERGE ? P.n_heads : KIND != FK_PLAIN ? P.top_k : 0;
        const int i2 = KIND == FK_ROUTE ? P.norm_topk : 0, i3 = KIND == FK_ROUTE ? P.sel_k : 0;
        const int i4 = XF == XF_NORM ? P.n_xa : 0;
        if constexpr (XF == XF_NONE)
            asm volatile("" ::"s"(nb), "s"(kg), "s"(tw), "s"(nwg), "s"(rows_pad), "s"(codes), "s"(hplane),
                         "s"(params), "s"(x0), "s"(nbk_), "s"(ltw_), "s"(kg_inv_), "s"(f0), "s"(f1), "s"(f2),
                         "s"(i0), "s"(i1), "s"(i2), "s"(i3), "s"(i4), "s"(out_y), "s"(out_bias), "s"(out_y2),
                         "s"(out_bias2), "s"(out_rows), "s"(out_nb2), "s"(out_amax));
        else
            asm volatile("" ::"s"(nb), "s"(kg), "s"(tw), "s"(nwg), "s"(rows_pad), "s"(codes), "s"(hplane),
                         "s"(params), "s"(x0), "s"(nbk_), "s"(ltw_), "s"(kg_inv_), "s"(f0), "s"(f1), "s"(f2),
                         "s"(i0), "s"(i1), "s"(i2), "s"(i3), "s"(i4));
    }
    if (local >= nwg) return;  // past this problem's workgroups
    const int tg = kg == 1 ? local : (int)__umulhi((uint32_t)local, kg_inv_), kgi = local - tg * kg;  // tile group, K-slice
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    // the slice: blocks [b0, b0 + nbl) of the matrix (of expert sel[kgi] in
    // a routed problem), its x (g) and u at xp / x2p
    int b0, nbl;
    const float* xp;
    const float* x2p = nullptr;
    int e = 0;
    bool live = true;
    if constexpr (KIND == FK_ROUTED) {
        b0 = 0;
        nbl = nb;
        xp = x0;
        x2p = P.x2;
    } else {
        const int nbk = nbk_;
        b0 = kgi * nbk;
        nbl = max(0, min(nb, b0 + nbk) - b0);
        xp = x0 + (size_t)b0 * 128;
        if constexpr (xform == XF_SILU) x2p = P.x2 + (size_t)b0 * 128;
    }
    // Loads, all issued before any use: x (L2-resident), then parameters,
    // then weights (HBM): one memory round trip. Each is a buffer load over
    // exactly the bytes it may touch, so a load past the end returns zeros
    // without a memory access and every load can be unconditional. (With
    // FK_ROUTE, routing runs between the x loads and the weight loads.)
    // x pair p = wave + 8*i: blocks 2p, 2p+1; lane l holds x[4(l&31) .. +3]
    // of block 2p + (l>>5).
    constexpr int XP = XPN;  // x pairs per wave at most
    // The plain GEMV loads XP0 pairs up front and the rest only when its
    // slice has them (slices of more than 32 blocks): fewer registers held
    // across the memory round trip.
    constexpr int XP0 = 2;
    const auto xrs = buf_rsrc(xp, nbl * 512);
    u32x4 xv[XP], x2v[XP], xav[XP], xav2[XP];
    if constexpr (xform != XF_MERGE) {
#pragma unroll
        for (int i = 0; i < XP; i++)
            if (XF != XF_NONE || i < XP0)
                xv[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (wave + 8 * i) * 1024 + lane * 16, 0, 0);
    }
    // the deferred slices, with x's loads
    const bool has_xa = XF == XF_NORM && P.x_add, has_xa2 = has_xa && P.n_xa > 1;
    if constexpr (XF == XF_NORM) {
        if (has_xa) {
            const auto ars = buf_rsrc(P.x_add + (size_t)b0 * 128, nbl * 512);
#pragma unroll
            for (int i = 0; i < XP; i++)
                xav[i] = __builtin_amdgcn_raw_buffer_load_b128(ars, (wave + 8 * i) * 1024 + lane * 16, 0, 0);
        }
        if (has_xa2) {
            const auto ars = buf_rsrc(P.x_add + (size_t)nb * 128 + (size_t)b0 * 128, nbl * 512);
#pragma unroll
            for (int i = 0; i < XP; i++)
                xav2[i] = __builtin_amdgcn_raw_buffer_load_b128(ars, (wave + 8 * i) * 1024 + lane * 16, 0, 0);
        }
    }
    // XF_MERGE: the chunk states of x pair p = wave + 8i: for every chunk
    // c, (m, l) of the head of this lane's four values and their four
    // unnormalised outputs. Chunks that held no position carry the neutral
    // state (m = -inf, l = 0, o = 0), so every chunk is read and the position
    // is not needed. Lanes of a block past the slice (blocks 2p+1 = nbl of an
    // odd slice, or a whole pair past it) load nothing (an out-of-range
    // offset: their head index may lie past n_heads) and their values are
    // replaced by zeros after the merge. Pair 0's loads go out
    // here, with the kernel's first loads and before the weights (its inputs
    // are the attention's outputs, an L2 or memory round trip away).
    struct MergeIn { float m[ATTN_CHUNKS], l[ATTN_CHUNKS]; float4 o[ATTN_CHUNKS]; };
    auto merge_load = [&](int i, MergeIn& in) {
        const int p = wave + 8 * i, hi = lane >> 5, k0 = 4 * (lane & 31);
        const bool blk_ok = 2 * p + hi < nbl;
        const int k = (b0 + 2 * p + hi) * 128 + k0, h = k / P.head_dim;
        const int stride = P.n_heads * P.head_dim;
        // buffer loads: the chunk's offset is a scalar, the lane's a vector
        // offset; a lane past the slice reads out of range (zeros, no access)
        const auto ors = buf_rsrc(P.x, ATTN_CHUNKS * stride * 4);
        const auto mrs = buf_rsrc(P.x2, ATTN_CHUNKS * P.n_heads * 8);
        const int vo = blk_ok ? k * 4 : 0x40000000, vm = blk_ok ? h * 8 : 0x40000000;
#pragma unroll
        for (int cc = 0; cc < ATTN_CHUNKS; cc++) {
            const u32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(mrs, vm, cc * P.n_heads * 8, 0);
            const u32x4 o = __builtin_amdgcn_raw_buffer_load_b128(ors, vo, cc * stride * 4, 0);
            in.m[cc] = __uint_as_float(ml.x);
            in.l[cc] = __uint_as_float(ml.y);
            in.o[cc] = make_float4(__uint_as_float(o.x), __uint_as_float(o.y), __uint_as_float(o.z), __uint_as_float(o.w));
        }
    };
    // Pair 1 too when the slice has it (an unsplit o_proj: dense Qwen3-4B
    // decode 685 -> 699 tok/s); v3's extra weight registers leave no room
    // for its states, which it loads in the prep.
    MergeIn mg0, mg1;
    if constexpr (xform == XF_MERGE) {
        merge_load(0, mg0);
        if (SCHEME == 4 && 2 * (wave + 8) < nbl) merge_load(1, mg1);
    }
    float wkv[XP];  // routed: the routing weight of each x pair's block
    auto load_x2 = [&]() {  // the second operand of the transform: nw or u
        const auto x2rs = buf_rsrc(xform == XF_NORM ? P.nw + (size_t)b0 * 128 : x2p, nbl * 512);
#pragma unroll
        for (int i = 0; i < XP; i++)
            x2v[i] = __builtin_amdgcn_raw_buffer_load_b128(x2rs, (wave + 8 * i) * 1024 + lane * 16, 0, 0);
    };
    // (with routing too: requested after routing, the norm weights were a
    // memory round trip on the critical path, ~1 us; the registers this holds
    // across routing leave one routing workgroup per CU, which is what a
    // top-8 gate/up launch of 192 workgroups uses)
    if constexpr (xform == XF_NORM || xform == XF_SILU) load_x2();
    if constexpr (KIND == FK_ROUTED) {
        // blk / enb as (blk * minv) >> 20: exact for blk < 2^20 / enb, and
        // blk < FAST_MAXBK here
        const uint32_t minv = (1u << 20) / (uint32_t)P.enb + 1;
#pragma unroll
        for (int i = 0; i < XP; i++) {
            const int blk = 2 * (wave + 8 * i) + (lane >> 5);
            wkv[i] = blk < nbl ? P.rw[((uint32_t)blk * minv) >> 20] : 0.0f;
        }
    }
    if constexpr (KIND == FK_ROUTE) {  // this workgroup routes itself
        const int selectable =
            P.n_exp <= 128 ? route_wg<2>(P.scores, P.n_exp, P.top_k, route_key, route_ids, route_w)
                           : route_wg<4>(P.scores, P.n_exp, P.top_k, route_key, route_ids, route_w);
        e = route_ids[P.sel_k];
        if (local == 0 && blockIdx.y == 0 && wave == 0) {
            // the routing for the down projection: slot k on lane k, the
            // weights divided by their sum in chosen order (norm_topk)
            const int got = __builtin_amdgcn_readfirstlane(min(P.top_k, selectable));
            float wk = lane < got ? route_w[lane] : 0.0f;
            if (P.norm_topk) {
                float sw = 0.0f;
                for (int k = 0; k < got; k++) sw = __fadd_rn(sw, lane_of(wk, k));
                if (sw > 0.0f) wk = __fdiv_rn(wk, sw);
            }
            if (lane < P.top_k) {
                P.ids_out[lane] = lane < got ? route_ids[lane] : -1;
                P.w_out[lane] = wk;
            }
        }
    } else if constexpr (KIND == FK_PLAIN) {
        if (P.sel) e = P.sel[P.sel_k];
    }
    if (KIND == FK_ROUTE || (KIND == FK_PLAIN && P.sel)) {  // the expert's rows of a stacked matrix
        live = e >= 0;
        const size_t t0 = (size_t)max(e, 0) * (rows_pad / TILE_ROWS) * nb;  // tile-block records
        codes += t0 * CODE_REC;
        hplane += t0 * HP_REC;
        params += t0 * TILE_ROWS;
    }
    const int ntiles = rows_pad / TILE_ROWS;
    const int ltw = ltw_, lkw = 3 - ltw, kw = 1 << lkw;  // kw = 8 / tw waves per tile
    const int T = (tg << ltw) + (wave >> lkw), kq = wave & (kw - 1);
    const int q = (nbl + kw - 1) >> lkw;             // blocks per part (<= QB)
    const int qw = live && T < ntiles ? max(0, min(q, nbl - kq * q)) : 0;  // this wave's blocks
    const int wb = b0 + kq * q;                      // its first block
    const int g = lane >> 4, j = lane & 15;

    u32x4 pv;
    u32x4 c[QB];
    u32x2 h[QB];
    if constexpr (KIND != FK_ROUTED) {
        const size_t rec = (size_t)min(T, ntiles - 1) * nb + wb;
        // lane l: rows 4(l&3)..+3 of block l>>2 (blocks past QB are not kept)
        const auto prs = buf_rsrc(params + rec * TILE_ROWS, qw * 64);
        pv = __builtin_amdgcn_raw_buffer_load_b128(prs, lane * 16, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        const auto crs = buf_rsrc(codes + rec * CODE_REC, qw * (int)CODE_REC);
        const auto hrs = buf_rsrc(hplane + rec * HP_REC, SCHEME == 3 ? qw * (int)HP_REC : 0);
#pragma unroll
        for (int i = 0; i < QB; i++) {
            c[i] = __builtin_amdgcn_raw_buffer_load_b128(crs, i * (int)CODE_REC + lane * 16, 0, CPOL_NT);
            if constexpr (SCHEME == 3)
                h[i] = __builtin_amdgcn_raw_buffer_load_b64(hrs, i * (int)HP_REC + lane * 8, 0, CPOL_NT);
        }
    } else {
        // block i of this wave's part is block (wb+i) % enb of expert
        // sel[(wb+i) / enb]; a block past the part or of an unfilled slot
        // (id < 0) reads zeros (a record range of 0 bytes)
        const int enb = P.enb, tiles_e = ntiles;  // the stack's experts have rows_pad rows each
        const int Tc = min(T, ntiles - 1), top_k = P.top_k;
        // the chosen experts' ids, slot l in lane l (one load for every
        // block; reading them block by block cost a round trip each)
        const int selv = (int)__builtin_amdgcn_raw_buffer_load_b32(buf_rsrc(P.sel, top_k * 4), (lane & 15) * 4, 0, 0);
        size_t recs[QB];
        int ok[QB];
        // block wb + i is block r of slot `slot`, stepped without a division
        int slot = wb / enb, r = wb - slot * enb;
#pragma unroll
        for (int i = 0; i < QB; i++) {
            const int ei = i < qw ? __builtin_amdgcn_readlane(selv, min(slot, top_k - 1)) : -1;
            ok[i] = ei >= 0;
            recs[i] = ((size_t)max(ei, 0) * tiles_e + Tc) * enb + r;
            if (++r == enb) {
                r = 0;
                slot++;
            }
        }
        {
            const int bi = lane >> 2;  // params: lane l, rows 4(l&3)..+3 of block l>>2
            size_t rb = recs[0];
            int okb = ok[0];
#pragma unroll
            for (int i = 1; i < QB; i++)
                if (bi == i) { rb = recs[i]; okb = ok[i]; }
            // one resource over the stack's parameters (its size is checked
            // below 2^31 bytes when the routed path is chosen) and a lane
            // offset: a resource per lane group made the load a loop over
            // the lane groups; a lane without a block reads past the range
            const auto prs = buf_rsrc(params, 0x7FFFFFF0);
            const uint32_t po = bi < QB && okb ? (uint32_t)(rb * TILE_ROWS * 4) + (lane & 3) * 16 : 0x7FFFFFF0u;
            pv = __builtin_amdgcn_raw_buffer_load_b128(prs, po, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < QB; i++) {
            const auto crs = buf_rsrc(codes + recs[i] * CODE_REC, ok[i] ? (int)CODE_REC : 0);
            c[i] = __builtin_amdgcn_raw_buffer_load_b128(crs, lane * 16, 0, CPOL_NT);
            if constexpr (SCHEME == 3) {
                const auto hrs = buf_rsrc(hplane + recs[i] * HP_REC, ok[i] ? (int)HP_REC : 0);
                h[i] = __builtin_amdgcn_raw_buffer_load_b64(hrs, lane * 8, 0, CPOL_NT);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- x -> int8 digits. x ~= s_b * Q / 2^21 with s_b = M/127; the scale
    // and its inverse need only agree to fp32 rounding, so both come from one
    // reciprocal. A wave digitises its pairs two at a time in one straight
    // run of code, so the two pairs' dependent chains (reductions, reciprocal,
    // rounding) overlap; the prep is latency-bound, one wave per SIMD at a
    // time. A wave's last pair, when it has an odd number, goes alone.
    {
        const int hi = lane >> 5, k0 = 4 * (lane & 31);
        const int pos0 = frag_pos(k0), pos1 = frag_pos(k0 + 1), pos2 = frag_pos(k0 + 2), pos3 = frag_pos(k0 + 3);
        float sq = 0.0f;
        // x' of pair i (after the transform) as four values per lane
        auto pair_values = [&](int i, float (&v)[4]) {
            if constexpr (xform == XF_MERGE) {
                // sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c, M = max_c m_c
                MergeIn later;
                constexpr int early = SCHEME == 4 ? 2 : 1;  // pairs loaded at entry
                if (i >= early) merge_load(i, later);
                const MergeIn& in = i == 0 ? mg0 : i < early ? mg1 : later;
                float M = -INFINITY;
#pragma unroll
                for (int cc = 0; cc < ATTN_CHUNKS; cc++) M = fmaxf(M, in.m[cc]);
                float L = 0.0f;
                float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int cc = 0; cc < ATTN_CHUNKS; cc++) {
                    const float w = __expf(in.m[cc] - M);  // 0 for a neutral chunk
                    L = fmaf(w, in.l[cc], L);
                    a.x = fmaf(w, in.o[cc].x, a.x);
                    a.y = fmaf(w, in.o[cc].y, a.y);
                    a.z = fmaf(w, in.o[cc].z, a.z);
                    a.w = fmaf(w, in.o[cc].w, a.w);
                }
                // a block past the slice read zeros (L = 0): its values are zeros
                const bool blk_ok = 2 * (wave + 8 * i) + hi < nbl;
                const float rl = __fdiv_rn(1.0f, L);
                xv[i] = blk_ok ? u32x4{__float_as_uint(a.x * rl), __float_as_uint(a.y * rl),
                                       __float_as_uint(a.z * rl), __float_as_uint(a.w * rl)}
                               : u32x4{0u, 0u, 0u, 0u};
            }
            v[0] = __uint_as_float(xv[i].x); v[1] = __uint_as_float(xv[i].y);
            v[2] = __uint_as_float(xv[i].z); v[3] = __uint_as_float(xv[i].w);
            if constexpr (xform == XF_NORM) {
                if (has_xa) {
                    v[0] += __uint_as_float(xav[i].x); v[1] += __uint_as_float(xav[i].y);
                    v[2] += __uint_as_float(xav[i].z); v[3] += __uint_as_float(xav[i].w);
                }
                if (has_xa2) {
                    v[0] += __uint_as_float(xav2[i].x); v[1] += __uint_as_float(xav2[i].y);
                    v[2] += __uint_as_float(xav2[i].z); v[3] += __uint_as_float(xav2[i].w);
                }
#pragma unroll
                for (int e = 0; e < 4; e++) sq = fmaf(v[e], v[e], sq);
                v[0] *= __uint_as_float(x2v[i].x); v[1] *= __uint_as_float(x2v[i].y);
                v[2] *= __uint_as_float(x2v[i].z); v[3] *= __uint_as_float(x2v[i].w);
            } else if constexpr (xform == XF_SILU) {
                const float wk = KIND == FK_ROUTED ? wkv[i] : 1.0f;
                const uint32_t u[4] = {x2v[i].x, x2v[i].y, x2v[i].z, x2v[i].w};
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = __fdividef(v[e], 1.0f + __expf(-v[e])) * __uint_as_float(u[e]) * wk;
            }
        };
        // block max |x| and sum of two pairs' values, step by step for both
        // so that the two dependent chains interleave: lane-local, the 16
        // lanes of a row by DPP exchanges (max on the bits of non-negative
        // floats), then the two rows of a block by a row swap; every lane of a
        // block ends with the same values, the sums added in one fixed order.
        // Then the 28-bit Q of each value.
        struct Dig { int Q[4]; float M, S; };
        auto digitize = [&](auto npairs, const float (&v)[2][4], Dig (&d)[2]) {
            constexpr int NP = decltype(npairs)::value;
            uint32_t mb[2];
            float sm[2];
#pragma unroll
            for (int u = 0; u < NP; u++) {
                mb[u] = __float_as_uint(fmaxf(fmaxf(fabsf(v[u][0]), fabsf(v[u][1])), fmaxf(fabsf(v[u][2]), fabsf(v[u][3]))));
                sm[u] = (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
            }
#pragma unroll
            for (int u = 0; u < NP; u++) mb[u] = max(mb[u], (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb[u], DPP_XOR1, 0xF, 0xF, false));
#pragma unroll
            for (int u = 0; u < NP; u++) sm[u] += dpp<DPP_XOR1>(sm[u]);
#pragma unroll
            for (int u = 0; u < NP; u++) mb[u] = max(mb[u], (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb[u], DPP_XOR2, 0xF, 0xF, false));
#pragma unroll
            for (int u = 0; u < NP; u++) sm[u] += dpp<DPP_XOR2>(sm[u]);
#pragma unroll
            for (int u = 0; u < NP; u++) mb[u] = max(mb[u], (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb[u], DPP_HALF_MIRROR, 0xF, 0xF, false));
#pragma unroll
            for (int u = 0; u < NP; u++) sm[u] += dpp<DPP_HALF_MIRROR>(sm[u]);
#pragma unroll
            for (int u = 0; u < NP; u++) mb[u] = max(mb[u], (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb[u], DPP_MIRROR, 0xF, 0xF, false));
#pragma unroll
            for (int u = 0; u < NP; u++) sm[u] += dpp<DPP_MIRROR>(sm[u]);
            float inv[2];
#pragma unroll
            for (int u = 0; u < NP; u++) {
                const auto mr = __builtin_amdgcn_permlane16_swap(mb[u], mb[u], false, false);
                d[u].M = __uint_as_float(max((uint32_t)mr[0], (uint32_t)mr[1]));
                inv[u] = d[u].M > 0.0f ? (127.0f * 2097152.0f) * __builtin_amdgcn_rcpf(d[u].M) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < NP; u++) {
                const auto sr = __builtin_amdgcn_permlane16_swap(__float_as_uint(sm[u]), __float_as_uint(sm[u]), false, false);
                d[u].S = __uint_as_float(sr[0]) + __uint_as_float(sr[1]);
            }
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int u = 0; u < NP; u++) d[u].Q[e] = (int)rintf(v[u][e] * inv[u]);
        };
        // pair i's digit bytes and {s_b, sum} into LDS (pairs inside the
        // slice): Q = d0*2^21 + d1*2^14 + d2*2^7 + d3 with |Q| <= 127*2^21 (+
        // rounding), d0 = Q >> 21 (arithmetic) in [-128, 127] and d1, d2, d3
        // the three 7-bit fields of Q mod 2^21; digit j of index k at
        // frag_pos(k) + 16*j
        auto put_pair = [&](int i, const Dig& d) {
            const int p = wave + 8 * i;
            if (2 * p >= nbl) return;
            int8_t* dst = xq + (2 * p + hi) * FRAG;
            const int pos[4] = {pos0, pos1, pos2, pos3};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int8_t* b = dst + pos[e];
                b[0] = (int8_t)(d.Q[e] >> 21);
                b[16] = (int8_t)((d.Q[e] >> 14) & 127);
                b[32] = (int8_t)((d.Q[e] >> 7) & 127);
                b[48] = (int8_t)(d.Q[e] & 127);
            }
            if ((lane & 31) == 0) xs[2 * p + hi] = make_float2(d.M * (1.0f / 127.0f), d.S);
        };
#pragma unroll
        for (int i = 0; i < XP; i += 2) {
            if (2 * (wave + 8 * i) < nbl) {
                if constexpr (XF == XF_NONE)
                    if (i >= XP0) {
                        xv[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (wave + 8 * i) * 1024 + lane * 16, 0, 0);
                        xv[i + 1] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (wave + 8 * (i + 1)) * 1024 + lane * 16, 0, 0);
                    }
                float v2[2][4];
                Dig d2[2];
                pair_values(i, v2[0]);
                if (2 * (wave + 8 * (i + 1)) < nbl) {
                    pair_values(i + 1, v2[1]);
                    digitize(std::integral_constant<int, 2>(), v2, d2);
                    put_pair(i, d2[0]);
                    put_pair(i + 1, d2[1]);
                } else {  // the wave's last pair
                    digitize(std::integral_constant<int, 1>(), v2, d2);
                    put_pair(i, d2[0]);
                }
            }
        }
        if constexpr (xform == XF_NORM) {
            sq = wave_sum(sq);
            if (lane == 0) ssq[wave] = sq;
        }
    }
    if (lane < QB * 4) *reinterpret_cast<u32x4*>(spar[wave] + lane * 4) = pv;
    if (threadIdx.x < 4) xs[nbl + threadIdx.x] = make_float2(0.0f, 0.0f);  // == prep's value if written
    __syncthreads();

    // XF_NORM: RMSNorm's scale of the row x, 1 / sqrt(mean(x^2) + eps), taken
    // here so that its dependent divisions and square root overlap the
    // matrix-core phase rather than follow the final sum (the empty asm keeps
    // the compiler from sinking it there)
    float rscale = 1.0f;
    if constexpr (xform == XF_NORM) {
        const float s2 = ((ssq[0] + ssq[1]) + (ssq[2] + ssq[3])) + ((ssq[4] + ssq[5]) + (ssq[6] + ssq[7]));
        rscale = __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(__fdiv_rn(s2, (float)(nb * 128)), P.eps)));
        asm volatile("" ::"v"(rscale));
    }

    // ---- matrix-core phase
    float acc = 0.f, zacc = 0.f;
    {
        const int lb = kq * q;  // the part's first block within the slice
        // lane (g, j) supplies digit row j&3 of the x operand, so its rows
        // 4..15 repeat digits 0..3 and every lane group of the result alike
        const int8_t* xf = xq + lb * FRAG + g * (NDIG * 16) + (j & 3) * 16;
        const float2* xsp = xs + lb;
        const uint32_t* sp = spar[wave] + j;
        const uint32_t M = 0x0F0F0F0Fu;
#pragma unroll
        for (int i0 = 0; i0 < QB; i0 += MG) {
            if (i0 < qw) {
                // this group's LDS operands first, so their latencies overlap
                v4i B0[MG], B1[MG];
                uint32_t pr[MG];
                float2 sc[MG];
#pragma unroll
                for (int u = 0; u < MG; u++) {
                    B0[u] = *reinterpret_cast<const v4i*>(xf + (i0 + u) * FRAG);
                    B1[u] = *reinterpret_cast<const v4i*>(xf + (i0 + u) * FRAG + HALF);
                    pr[u] = sp[(i0 + u) * TILE_ROWS];
                    sc[u] = xsp[i0 + u];
                }
#pragma unroll
                for (int i = i0; i < i0 + MG; i++) {
                    const int u = i - i0;
                    v4i A0, A1;
                    A0.x = c[i].x & M; A0.y = c[i].y & M; A0.z = c[i].z & M; A0.w = c[i].w & M;
                    A1.x = (c[i].x >> 4) & M; A1.y = (c[i].y >> 4) & M;
                    A1.z = (c[i].z >> 4) & M; A1.w = (c[i].w >> 4) & M;
                    if constexpr (SCHEME == 3) {
                        // top two bits: group g holds AVX lanes g (h.x) and g+4 (h.y)
                        const uint32_t T6 = 0x30303030u, hx = h[i].x, hy = h[i].y;
                        A0.x |= (hx << 4) & T6; A0.y |= (hx << 2) & T6;
                        A0.z |= (hy << 4) & T6; A0.w |= (hy << 2) & T6;
                        A1.x |= hx & T6;        A1.y |= (hx >> 2) & T6;
                        A1.z |= hy & T6;        A1.w |= (hy >> 2) & T6;
                    }
                    // x digits as the first operand: lane (g, j) gets digits
                    // 0..3 of row j's dot (every lane group alike)
                    v4i d = {0, 0, 0, 0};
                    d = __builtin_amdgcn_mfma_i32_16x16x64_i8(B0[u], A0, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_i32_16x16x64_i8(B1[u], A1, d, 0, 0, 0);
                    float cd = fmaf((float)d.w, 0x1p-7f, (float)d.z);
                    cd = fmaf(cd, 0x1p-7f, (float)d.y);
                    cd = fmaf(cd, 0x1p-7f, (float)d.x);
                    acc = __builtin_fmaf(cd * sc[u].x, h2f(pr[u] >> 16), acc);
                    zacc = __builtin_fmaf(h2f(pr[u] & 0xFFFFu), sc[u].y, zacc);
                }
            }
        }
    }
    // lane (g, j) holds row j's sum over its blocks
    if (g == 0) red[wave][j] = acc + zacc;
    __syncthreads();

    const int t = threadIdx.x;
    const int tt = t >> 4, rr = t & 15;
    const bool mine = t < tw * TILE_ROWS && tg * tw + tt < ntiles;
    const size_t orow = (size_t)(tg * tw + tt) * TILE_ROWS + rr;
    float sum = 0.0f;
    if (mine) {  // the tile's parts in order
        sum = red[tt * kw][rr];
        for (int k = 1; k < kw; k++) sum += red[tt * kw + k][rr];
        if constexpr (xform == XF_NORM) sum *= rscale;
    }
    if (kg == 1 || out_y2) {  // one slice, or the deferred split: slices k >= 1 to y2
        const bool row_ok = mine && orow < (size_t)out_rows;
        if (row_ok) {
            if (kgi == 0) {
                if (out_bias) {
                    float b = out_bias[orow];
                    if (out_bias2) {
                        b += out_bias2[orow];
                        if (out_nb2 > 1) b += out_bias2[(size_t)out_rows + orow];
                    }
                    sum += b;
                }
                out_y[orow] = sum;
            } else {
                out_y2[(size_t)(kgi - 1) * out_rows + orow] = sum;
            }
        }
        // the argmax key of this workgroup's rows (one slice: every output
        // row is a thread of wave 0, rows growing with the lane):
        // (order-preserving bits of the largest value, -0 read as +0) << 32 |
        // ~(its first row), 0 when no value beats -inf (NaN never does). The
        // largest value by a DPP maximum and its first row by a ballot: a
        // 64-bit maximum by lane exchanges (twelve LDS-crossbar round trips)
        // cost the 2374-workgroup lm_head 1.7 us.
        if (out_amax && wave == 0) {
            const float v = row_ok && sum > -INFINITY ? sum : -INFINITY;
            const float vmax = wave_max(v);
            uint64_t key = 0;
            if (vmax > -INFINITY) {
                const uint64_t at = __ballot(v == vmax);  // -0 == +0: the first of them
                const uint32_t row = (uint32_t)__builtin_amdgcn_readlane((int)orow, __ffsll((long long)at) - 1);
                const uint32_t b = __float_as_uint(__fadd_rn(vmax, 0.0f));
                key = ((uint64_t)((b & 0x80000000u) ? ~b : (b | 0x80000000u)) << 32) | (0xFFFFFFFFu - row);
            }
            if (lane == 0) out_amax[tg] = key;
        }
        return;
    }
    // Split K: publish this slice's partials; the last workgroup of the tile
    // group adds the kg slices in slice order (deterministic) and resets the
    // counter for the next launch.
    //
    // The handoff needs no cache-wide write-back or invalidate. Partials are
    // published with device-scope atomic exchanges, which are performed at
    // the device's coherence point and return only once performed; each
    // thread consumes the returned value (the empty asm makes the compiler
    // wait for it) before the barrier, so every partial of this workgroup
    // is performed before thread 0 increments the counter. The workgroup that
    // sees kg-1 then reads the partials with device-scope atomic loads, which
    // are coherent per location across all XCDs.
    if (mine) {
        const float prev = __hip_atomic_exchange(P.part + (size_t)kgi * P.rows_pad + orow, sum,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::"v"(prev));
    }
    __syncthreads();
    if (t == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(P.counters + tg, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (uint32_t)(kg - 1);
    }
    __syncthreads();
    if (!s_last) return;
    if (mine && orow < (size_t)out_rows) {
        float acc = __hip_atomic_load(P.part + orow, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int k = 1; k < kg; k++)
            acc += __hip_atomic_load(P.part + (size_t)k * P.rows_pad + orow, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        out_y[orow] = out_bias ? acc + out_bias[orow] : acc;
    }
    if (t == 0) __hip_atomic_store(P.counters + tg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ============================================================ FAST mode, vector-ALU variant
// k_gemv_valu: the plain FAST GEMV (no input transform, no routing) with the
// dot products on the vector ALU in fp32 instead of the matrix cores: x is
// read as fp32 and never digitised, so the prep has no block maximum, no
// reciprocal and no rounding, only a transposing copy into LDS. Same
// problems, launch shape, plan (tiles per workgroup, K-slices) and end phase
// as k_gemv_fast<S, FK_PLAIN, XF_NONE>; the reference's row kernel it
// restates with another summation order is matvec_v{4,3}_fused
// (wpc-eval/src/fused_kernel.rs:237-271, 163-189).
//   prep:  the slice's x goes to LDS transposed by lane group: value k of a
//          block at xv[blk][k & 3][k >> 2] (groups padded to 36 floats so
//          that the four groups' 16-byte reads fall in distinct banks), and
//          each group's sum of its 32 values at xg[blk][k & 3].
//   dots:  lane (g, j) of a wave holds, per block, the 16 code bytes of row
//          j that AVX2 lanes g and g+4 read (32 codes, every k = g mod 4),
//          turns them into floats with shift/mask in registers (v3: the high
//          plane's two bits or-ed in) and multiplies them with its group's
//          32 x values: P = sum code*x in fp32, then
//          acc += scale*P + zp*sum(x of the group).
//   sum:   the four lane groups of a row by two row swaps, then the waves of
//          a tile in part order (deterministic).
constexpr int VX_G = 36;          // floats per lane group of a block in LDS
constexpr int VX_BLK = 4 * VX_G;  // floats per block

// float of byte b of w (v_cvt_f32_ubyte{0..3})
template <int B>
__device__ __forceinline__ float ub(uint32_t w) { return (float)((w >> (8 * B)) & 0xFFu); }

// P += the 8 products of word w's four bytes with x values m0, m0+2, m0+4, m0+6
__device__ __forceinline__ float dot4(uint32_t w, const float* X, int m0, float P)
{
    P = __builtin_fmaf(ub<0>(w), X[m0], P);
    P = __builtin_fmaf(ub<1>(w), X[m0 + 2], P);
    P = __builtin_fmaf(ub<2>(w), X[m0 + 4], P);
    P = __builtin_fmaf(ub<3>(w), X[m0 + 6], P);
    return P;
}

template <int SCHEME>
__global__ __launch_bounds__(FAST_WG, 4) void k_gemv_valu(const FastBatch B)
{
    __shared__ __align__(16) float xv[MAXBK * VX_BLK];  // the slice's x, transposed
    __shared__ __align__(16) float xg[MAXBK * 4];       // per block and lane group: sum of its x
    __shared__ __align__(16) uint32_t spar[8][QB * TILE_ROWS];
    __shared__ float red[8][TILE_ROWS];
    __shared__ int s_last;

    typedef const __attribute__((address_space(4))) FastBatch* KargPtr;
    const KargPtr kargs = (KargPtr)__builtin_amdgcn_kernarg_segment_ptr();
    const auto& P = kargs->p[blockIdx.y];
    const int local = blockIdx.x;
    const int nb = P.nb, kg = P.kg, tw = P.tw, nwg = P.nwg, rows_pad = P.rows_pad;
    const uint8_t* codes = P.codes;
    const uint8_t* hplane = SCHEME == 3 ? P.hp : P.codes;
    const uint32_t* params = P.params;
    const float* const x0 = P.x;
    const int nbk_ = P.nbk, ltw_ = P.ltw;
    const uint32_t kg_inv_ = P.kg_inv;
    float* const out_y = P.y;
    const float* const out_bias = P.bias;
    const int out_rows = P.rows;
    const int32_t* const sel = P.sel;
    asm volatile("" ::"s"(nb), "s"(kg), "s"(tw), "s"(nwg), "s"(rows_pad), "s"(codes), "s"(hplane), "s"(params),
                 "s"(x0), "s"(nbk_), "s"(ltw_), "s"(kg_inv_), "s"(out_y), "s"(out_bias), "s"(out_rows), "s"(sel));
    if (local >= nwg) return;  // past this problem's workgroups
    const int tg = kg == 1 ? local : (int)__umulhi((uint32_t)local, kg_inv_), kgi = local - tg * kg;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int b0 = kgi * nbk_, nbl = max(0, min(nb, b0 + nbk_) - b0);
    const float* xp = x0 + (size_t)b0 * 128;

    // Loads, all issued before any use, as in k_gemv_fast: x, parameters, weights.
    // float4 f = threadIdx.x + FAST_WG*u of the slice: block f >> 5, values 4(f & 31) .. +3
    constexpr int XU = MAXBK * 32 / FAST_WG;
    const auto xrs = buf_rsrc(xp, nbl * 512);
    u32x4 xl[XU];
#pragma unroll
    for (int u = 0; u < XU; u++) xl[u] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (threadIdx.x + FAST_WG * u) * 16, 0, 0);

    int e = 0;
    if (sel) e = sel[P.sel_k];
    const bool live = !sel || e >= 0;
    if (sel) {
        const size_t t0 = (size_t)max(e, 0) * (rows_pad / TILE_ROWS) * nb;
        codes += t0 * CODE_REC;
        hplane += t0 * HP_REC;
        params += t0 * TILE_ROWS;
    }
    const int ntiles = rows_pad / TILE_ROWS;
    const int ltw = ltw_, lkw = 3 - ltw, kw = 1 << lkw;
    const int T = (tg << ltw) + (wave >> lkw), kq = wave & (kw - 1);
    const int q = (nbl + kw - 1) >> lkw;
    const int qw = live && T < ntiles ? max(0, min(q, nbl - kq * q)) : 0;
    const int wb = b0 + kq * q;
    const int g = lane >> 4, j = lane & 15;

    u32x4 pv;
    u32x4 c[QB];
    u32x2 h[QB];
    {
        const size_t rec = (size_t)min(T, ntiles - 1) * nb + wb;
        const auto prs = buf_rsrc(params + rec * TILE_ROWS, qw * 64);
        pv = __builtin_amdgcn_raw_buffer_load_b128(prs, lane * 16, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        const auto crs = buf_rsrc(codes + rec * CODE_REC, qw * (int)CODE_REC);
        const auto hrs = buf_rsrc(hplane + rec * HP_REC, SCHEME == 3 ? qw * (int)HP_REC : 0);
#pragma unroll
        for (int i = 0; i < QB; i++) {
            c[i] = __builtin_amdgcn_raw_buffer_load_b128(crs, i * (int)CODE_REC + lane * 16, 0, CPOL_NT);
            if constexpr (SCHEME == 3)
                h[i] = __builtin_amdgcn_raw_buffer_load_b64(hrs, i * (int)HP_REC + lane * 8, 0, CPOL_NT);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- x -> LDS, transposed by lane group; each group's sum over a block
    // by DPP within rows and a row swap (the 32 lanes holding a block are
    // rows 0-1 or 2-3 of the wave); a fixed tree, the same on every call.
#pragma unroll
    for (int u = 0; u < XU; u++) {
        const int f = threadIdx.x + FAST_WG * u, blk = f >> 5, m = f & 31;
        if (blk >= nbl) break;  // uniform per half-wave; past the slice from here on
        float v[4] = {__uint_as_float(xl[u].x), __uint_as_float(xl[u].y), __uint_as_float(xl[u].z),
                      __uint_as_float(xl[u].w)};
        float* d = xv + blk * VX_BLK + m;
#pragma unroll
        for (int gg = 0; gg < 4; gg++) d[gg * VX_G] = v[gg];
#pragma unroll
        for (int gg = 0; gg < 4; gg++) v[gg] += dpp<DPP_XOR1>(v[gg]);
#pragma unroll
        for (int gg = 0; gg < 4; gg++) v[gg] += dpp<DPP_XOR2>(v[gg]);
#pragma unroll
        for (int gg = 0; gg < 4; gg++) v[gg] += dpp<DPP_HALF_MIRROR>(v[gg]);
#pragma unroll
        for (int gg = 0; gg < 4; gg++) v[gg] += dpp<DPP_MIRROR>(v[gg]);
#pragma unroll
        for (int gg = 0; gg < 4; gg++) {  // every lane of the half-wave takes part in the swap
            const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[gg]), __float_as_uint(v[gg]), false, false);
            v[gg] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
        if (m == 0) {
#pragma unroll
            for (int gg = 0; gg < 4; gg++) xg[blk * 4 + gg] = v[gg];
        }
    }
    if (lane < QB * 4) *reinterpret_cast<u32x4*>(spar[wave] + lane * 4) = pv;
    __syncthreads();

    // ---- dots
    float acc = 0.0f, zacc = 0.0f;
    {
        const int lb = kq * q;
        const float* xw = xv + lb * VX_BLK + g * VX_G;
        const float* xgw = xg + lb * 4 + g;
        const uint32_t* sp = spar[wave] + j;
        const uint32_t M = 0x0F0F0F0Fu;
#pragma unroll
        for (int i = 0; i < QB; i++) {
            if (i < qw) {
                float X[32];
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const float4 v = *reinterpret_cast<const float4*>(xw + i * VX_BLK + 4 * t);
                    X[4 * t] = v.x; X[4 * t + 1] = v.y; X[4 * t + 2] = v.z; X[4 * t + 3] = v.w;
                }
                const uint32_t pr = sp[i * TILE_ROWS];
                const float sgrp = xgw[i * 4];
                // low nibbles: codes k (k < 64), high nibbles: k + 64 (x index m + 16)
                uint32_t L0 = c[i].x & M, L1 = c[i].y & M, L2 = c[i].z & M, L3 = c[i].w & M;
                uint32_t H0 = (c[i].x >> 4) & M, H1 = (c[i].y >> 4) & M;
                uint32_t H2 = (c[i].z >> 4) & M, H3 = (c[i].w >> 4) & M;
                if constexpr (SCHEME == 3) {
                    const uint32_t T6 = 0x30303030u, hx = h[i].x, hy = h[i].y;
                    L0 |= (hx << 4) & T6; L1 |= (hx << 2) & T6;
                    L2 |= (hy << 4) & T6; L3 |= (hy << 2) & T6;
                    H0 |= hx & T6;        H1 |= (hx >> 2) & T6;
                    H2 |= hy & T6;        H3 |= (hy >> 2) & T6;
                }
                // byte b of word 0 is k = 8b + g (m = 2b), of word 1 k = 8(b+4) + g
                // (m = 8 + 2b), of word 2 k = 8b + g + 4 (m = 2b + 1), of word 3
                // m = 9 + 2b; two chains, added at the end
                float Pa = 0.0f, Pb = 0.0f;
                Pa = dot4(L0, X, 0, Pa);
                Pb = dot4(L2, X, 1, Pb);
                Pa = dot4(L1, X, 8, Pa);
                Pb = dot4(L3, X, 9, Pb);
                Pa = dot4(H0, X, 16, Pa);
                Pb = dot4(H2, X, 17, Pb);
                Pa = dot4(H1, X, 24, Pa);
                Pb = dot4(H3, X, 25, Pb);
                acc = __builtin_fmaf(Pa + Pb, h2f(pr >> 16), acc);
                zacc = __builtin_fmaf(h2f(pr & 0xFFFFu), sgrp, zacc);
            }
        }
    }
    // the four lane groups of row j: rows 0+1 and 2+3 by a 16-lane swap, then the halves
    float r = acc + zacc;
    {
        const auto s1 = __builtin_amdgcn_permlane16_swap(__float_as_uint(r), __float_as_uint(r), false, false);
        r = __uint_as_float(s1[0]) + __uint_as_float(s1[1]);
        const auto s2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(r), __float_as_uint(r), false, false);
        r = __uint_as_float(s2[0]) + __uint_as_float(s2[1]);
    }
    if (g == 0) red[wave][j] = r;
    __syncthreads();

    const int t = threadIdx.x;
    const int tt = t >> 4, rr = t & 15;
    const bool mine = t < tw * TILE_ROWS && tg * tw + tt < ntiles;
    const size_t orow = (size_t)(tg * tw + tt) * TILE_ROWS + rr;
    float sum = 0.0f;
    if (mine) {
        sum = red[tt * kw][rr];
        for (int k = 1; k < kw; k++) sum += red[tt * kw + k][rr];
    }
    if (kg == 1) {
        if (mine && orow < (size_t)out_rows) out_y[orow] = out_bias ? sum + out_bias[orow] : sum;
        return;
    }
    // split K: the handoff of k_gemv_fast (device-scope exchanges, a counter
    // per tile group, the last workgroup adding the slices in slice order)
    if (mine) {
        const float prev = __hip_atomic_exchange(P.part + (size_t)kgi * P.rows_pad + orow, sum,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::"v"(prev));
    }
    __syncthreads();
    if (t == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(P.counters + tg, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (uint32_t)(kg - 1);
    }
    __syncthreads();
    if (!s_last) return;
    if (mine && orow < (size_t)out_rows) {
        float a = __hip_atomic_load(P.part + orow, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int k = 1; k < kg; k++)
            a += __hip_atomic_load(P.part + (size_t)k * P.rows_pad + orow, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        out_y[orow] = out_bias ? a + out_bias[orow] : a;
    }
    if (t == 0) __hip_atomic_store(P.counters + tg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ============================================================ decode helpers
__device__ __forceinline__ uint32_t code_at(const uint8_t* codes, const uint8_t* hp, size_t row,
                                            size_t b, int nb, int kk, int scheme)
{
    const int L = kk & 7, G = kk >> 3, r = (int)(row % TILE_ROWS);
    const size_t rec = (row / TILE_ROWS) * (size_t)nb + b;
    const uint8_t byte = codes[rec * CODE_REC + dcode_pos(r, L) + (G & 7)];
    uint32_t code = G < 8 ? (byte & 15u) : (byte >> 4);
    if (scheme == 3) {
        const uint8_t hb = hp[rec * HP_REC + dhp_pos(r, L) + (G & 3)];
        code |= ((hb >> (2 * (G >> 2))) & 3u) << 4;
    }
    return code;
}

// Natural-order decode of row `row`, two roundings: out[k] = zp + code*scale
// (row_decode_into_v4, wpc_weights_v4.rs:103-115).
template <int SCHEME>
__global__ __launch_bounds__(256) void k_embed(const uint8_t* __restrict__ codes,
                                               const uint8_t* __restrict__ hp,
                                               const uint32_t* __restrict__ params,
                                               float* __restrict__ out, size_t row, int nb)
{
    const int k = blockIdx.x * 256 + threadIdx.x;
    if (k >= nb * 128) return;
    const uint32_t code = code_at(codes, hp, row, (size_t)(k >> 7), nb, k & 127, SCHEME);
    const uint32_t p = params[param_idx(row, nb, k >> 7)];
    out[k] = __fadd_rn(h2f(p & 0xFFFFu), __fmul_rn((float)code, h2f(p >> 16)));
}

// The embedding row of the decode step's input token, tokens[st->pos].
template <int SCHEME>
__global__ __launch_bounds__(256) void k_embed_tok(const uint8_t* __restrict__ codes,
                                                   const uint8_t* __restrict__ hp,
                                                   const uint32_t* __restrict__ params,
                                                   float* __restrict__ out,
                                                   const uint32_t* __restrict__ tokens,
                                                   const DecodeState* __restrict__ st, int nb,
                                                   uint32_t rows, const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t, int half,
                                                   float* __restrict__ rope)
{
    // The step's RoPE row, cos then sin at the position, for the FAST
    // attention launches of the step (a fixed address they read at entry).
    if (rope && blockIdx.x == 0 && (int)threadIdx.x < 2 * half) {
        const uint32_t p = st->pos, i = threadIdx.x;
        if (p < st->max_pos) rope[i] = (int)i < half ? cos_t[(size_t)p * half + i] : sin_t[(size_t)p * half + i - half];
    }
    const int k = blockIdx.x * 256 + threadIdx.x;
    if (k >= nb * 128) return;
    const uint32_t row = min(tokens[st->pos], rows - 1);  // ids are checked on the host
    const uint32_t code = code_at(codes, hp, row, (size_t)(k >> 7), nb, k & 127, SCHEME);
    const uint32_t p = params[param_idx(row, nb, k >> 7)];
    out[k] = __fadd_rn(h2f(p & 0xFFFFu), __fmul_rn((float)code, h2f(p >> 16)));
}

// Embedding rows of a batch of tokens: out[t] = row tokens[t] (blockIdx.y = t).
template <int SCHEME>
__global__ __launch_bounds__(256) void k_embed_rows(const uint8_t* __restrict__ codes,
                                                    const uint8_t* __restrict__ hp,
                                                    const uint32_t* __restrict__ params,
                                                    float* __restrict__ out,
                                                    const uint32_t* __restrict__ tokens, int nb, uint32_t rows)
{
    const int k = blockIdx.x * 256 + threadIdx.x;
    if (k >= nb * 128) return;
    const uint32_t row = min(tokens[blockIdx.y], rows - 1);  // ids are checked on the host
    const uint32_t code = code_at(codes, hp, row, (size_t)(k >> 7), nb, k & 127, SCHEME);
    const uint32_t p = params[param_idx(row, nb, k >> 7)];
    out[(size_t)blockIdx.y * nb * 128 + k] = __fadd_rn(h2f(p & 0xFFFFu), __fmul_rn((float)code, h2f(p >> 16)));
}

template <int SCHEME>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ codes,
                                                 const uint8_t* __restrict__ hp,
                                                 const uint32_t* __restrict__ params,
                                                 float* __restrict__ w, size_t n, int nb,
                                                 int rounding)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const size_t blk = i >> 7;
    const size_t row = blk / nb, b = blk % nb;
    const uint32_t code = code_at(codes, hp, row, b, nb, (int)(i & 127), SCHEME);
    const uint32_t p = params[param_idx(row, nb, b)];
    const float zp = h2f(p & 0xFFFFu), sc = h2f(p >> 16);
    w[i] = rounding == WPCG_ROUND_FMA ? __builtin_fmaf((float)code, sc, zp)
                                      : __fadd_rn(zp, __fmul_rn((float)code, sc));
}

// FAST routing of a batch of score rows (the batched prefill): workgroup t
// routes row t exactly as a FAST one-token projection's FK_ROUTE workgroup
// does (route_wg, then the chosen weights divided by their sum in chosen
// order when norm_topk), so each prompt token gets the routing a FAST step
// would give it from the same scores. ids/w: [rows][top_k].
__global__ __launch_bounds__(512) void k_route_rows(const float* __restrict__ scores, int n, int top_k,
                                                    int norm_topk, int32_t* __restrict__ ids,
                                                    float* __restrict__ w)
{
    __shared__ uint64_t key[ROUTE_MAXN];
    __shared__ int32_t rid[MAX_JOBS];
    __shared__ float rw[MAX_JOBS];
    scores += (size_t)blockIdx.x * n;
    const int selectable = n <= 128 ? route_wg<2>(scores, n, top_k, key, rid, rw)
                                    : route_wg<4>(scores, n, top_k, key, rid, rw);
    if (threadIdx.x < 64) {  // wave 0 holds the count
        const int lane = threadIdx.x;
        const int got = __builtin_amdgcn_readfirstlane(min(top_k, selectable));
        float wk = lane < got ? rw[lane] : 0.0f;
        if (norm_topk) {
            float sw = 0.0f;
            for (int k = 0; k < got; k++) sw = __fadd_rn(sw, lane_of(wk, k));
            if (sw > 0.0f) wk = __fdiv_rn(wk, sw);
        }
        if (lane < top_k) {
            ids[(size_t)blockIdx.x * top_k + lane] = lane < got ? rid[lane] : -1;
            w[(size_t)blockIdx.x * top_k + lane] = wk;
        }
    }
}

}  // namespace

// ============================================================ launchers
int fast_kslices(uint64_t rows, uint64_t nb)
{
    if (nb == 0) return 1;
    // As few K-slices as fit: a split costs a cross-workgroup handoff. When
    // a split is needed anyway, slices of at most half the largest slice
    // (measured on 2560x9728: 3 slices of 26 blocks beat 2 of 38 at one
    // tile per workgroup, and at two tiles 3 slices beat 5).
    const uint64_t mb = fast_max_slice(rows, nb);
    uint64_t kg = (nb + mb - 1) / mb;
    if (kg > 1) {
        const uint64_t cap = std::min<uint64_t>(mb, FAST_MAXBK / 2);
        kg = (nb + cap - 1) / cap;
    }
    return fast_normalize_kslices(nb, (int)kg);
}

hipError_t launch_gemv_exact(const DeviceMatrix& m, const float* x, const float* bias, float* y,
                             hipStream_t s, const int32_t* sel, int sel_k)
{
    const int rows = (int)m.rows, nb = (int)m.nb;
    dim3 grid((unsigned)(m.rows_pad / (EX_WG / 8)));
    (void)hipGetLastError();  // report only this launch
    if (m.scheme == 4)
        hipLaunchKernelGGL(k_gemv_exact<4>, grid, dim3(EX_WG), 0, s, m.codes, m.hp, m.params, x,
                           bias, y, rows, nb, sel, sel_k, (int)m.rows_pad);
    else
        hipLaunchKernelGGL(k_gemv_exact<3>, grid, dim3(EX_WG), 0, s, m.codes, m.hp, m.params, x,
                           bias, y, rows, nb, sel, sel_k, (int)m.rows_pad);
    return hipGetLastError();
}

hipError_t launch_gemv_exact_multi(const GemvJob* jobs, int n, hipStream_t s)
{
    if (n <= 0 || n > MAX_JOBS) return hipErrorInvalidValue;
    ExactBatch B{};
    B.n = n;
    int wgs = 0;
    const int scheme = jobs[0].m->scheme;
    for (int i = 0; i < n; i++) {
        const DeviceMatrix& m = *jobs[i].m;
        if (m.scheme != scheme || m.nb == 0) return hipErrorInvalidValue;
        ExactProblem& P = B.p[i];
        P.codes = m.codes;
        P.hp = m.hp;
        P.params = m.params;
        P.x = jobs[i].x;
        P.bias = jobs[i].bias;
        P.y = jobs[i].y;
        P.sel = jobs[i].sel;
        P.sel_k = jobs[i].sel_k;
        P.rows = (int)m.rows;
        P.nb = (int)m.nb;
        P.rows_pad = (int)m.rows_pad;
        P.nwg = (int)(m.rows_pad / (EX_WG / 8));
        const GemvJob& J = jobs[i];
        if (J.scores) {  // routing reads at most 64 * RT_PER scores into MAX_JOBS slots
            if (J.n_exp < 1 || J.n_exp > 64 * RT_PER || J.top_k < 1 || J.top_k > MAX_JOBS ||
                J.sel_k >= J.top_k || !J.ids_out || !J.w_out || J.sel)
                return hipErrorInvalidValue;
            P.scores = J.scores;
            P.ids_out = J.ids_out;
            P.w_out = J.w_out;
            P.n_exp = J.n_exp;
            P.top_k = J.top_k;
            P.norm_topk = J.norm_topk;
        }
        wgs = std::max(wgs, P.nwg);
    }
    if (wgs == 0) return hipSuccess;
    (void)hipGetLastError();  // report only this launch
    if (scheme == 4)
        hipLaunchKernelGGL(k_gemv_exact_multi<4>, dim3(wgs, n), dim3(EX_WG), 0, s, B);
    else
        hipLaunchKernelGGL(k_gemv_exact_multi<3>, dim3(wgs, n), dim3(EX_WG), 0, s, B);
    return hipGetLastError();
}

hipError_t launch_gemv_fast(const GemvJob* jobs, int n, hipStream_t s)
{
    if (n <= 0 || n > MAX_JOBS) return hipErrorInvalidValue;
    FastBatch B{};
    B.n = n;
    int wgs = 0;
    const int scheme = jobs[0].m->scheme;
    for (int i = 0; i < n; i++) {
        const GemvJob& J = jobs[i];
        const DeviceMatrix& m = *J.m;
        if (m.scheme != scheme) return hipErrorInvalidValue;
        FastProblem& P = B.p[i];
        P.codes = m.codes;
        P.hp = m.hp;
        P.params = m.params;
        P.x = J.x;
        P.x2 = J.x2;
        P.nw = J.nw;
        P.y = J.y;
        P.bias = J.bias;
        P.part = J.plan->part;
        P.counters = J.plan->counters;
        P.rows = (int)m.rows;
        P.rows_pad = (int)m.rows_pad;
        P.nb = (int)m.nb;
        P.kg = J.plan->kg;
        P.sel = J.sel;
        P.sel_k = J.sel_k;
        P.tw = fast_tiles_per_wg(m.rows, J.routed ? (uint64_t)J.top_k * m.nb : m.nb);
        // the merge reads every chunk state of the whole row per workgroup:
        // one tile each spreads that over twice the workgroups (the slice
        // limit only grows, so the plan's K-split still fits)
        if (J.xform == XF_MERGE) P.tw = 1;
        P.xform = J.xform;
        P.eps = J.eps;
        P.routed = J.routed;
        P.rw = J.rw;
        P.scores = J.scores;
        P.n_exp = J.n_exp;
        P.top_k = J.top_k;
        P.norm_topk = J.norm_topk;
        P.ids_out = J.ids_out;
        P.w_out = J.w_out;
        P.st = J.st;
        P.y2 = J.y2;
        P.x_add = J.x_add;
        P.bias2 = J.bias2;
        P.n_xa = J.n_xa;
        P.n_b2 = J.n_b2;
        P.amax = J.amax;
        P.head_dim = J.head_dim;
        P.n_heads = J.n_heads;
        if (J.routed) {  // the chosen experts' rows side by side
            P.enb = (int)m.nb;
            P.nb = J.top_k * (int)m.nb;
        }
        // shapes the kernel assumes: a normed row is one K-slice; a routed
        // problem has one K-slice per slot, each an expert's whole row;
        // routing reads at most ROUTE_MAXN scores into MAX_JOBS slots
        if (J.xform == XF_NORM && (P.kg != 1 || !J.nw)) return hipErrorInvalidValue;
        if (J.xform == XF_SILU && !J.x2) return hipErrorInvalidValue;
        // the deferred split: 2 or 3 slices, no routing; x_add with the norm; bias2 with a bias
        if (J.y2 && !deferred_split_ok(P.kg, J.routed != 0)) return hipErrorInvalidValue;
        if ((J.x_add && J.xform != XF_NORM) || (J.bias2 && !J.bias)) return hipErrorInvalidValue;
        if (J.n_xa < 1 || J.n_xa > 2 || J.n_b2 < 1 || J.n_b2 > 2) return hipErrorInvalidValue;
        if (J.amax && (P.kg != 1 || J.routed)) return hipErrorInvalidValue;
        if (J.xform == XF_MERGE && (!J.x2 || !J.st || (J.head_dim != 64 && J.head_dim != 128) ||
                                    (uint64_t)J.n_heads * J.head_dim != m.cols))
            return hipErrorInvalidValue;
        if (J.routed && (!J.sel || !J.rw || J.xform != XF_SILU || P.kg != 1 || J.top_k < 1 ||
                         (uint64_t)J.top_k * m.nb > fast_max_slice(m.rows, (uint64_t)J.top_k * m.nb)))
            return hipErrorInvalidValue;
        if (J.scores && (J.n_exp < 1 || J.n_exp > ROUTE_MAXN || J.top_k < 1 || J.top_k > MAX_JOBS ||
                         J.sel_k >= J.top_k || !J.ids_out || !J.w_out))
            return hipErrorInvalidValue;
        // a K-slice's blocks must fit the workgroup (FAST_MAXBK / tw)
        if (!J.routed && ((uint64_t)P.nb + P.kg - 1) / P.kg > (uint64_t)(FAST_MAXBK / P.tw))
            return hipErrorInvalidValue;
        const int tiles = (int)(m.rows_pad / TILE_ROWS);
        P.nwg = (tiles + P.tw - 1) / P.tw * P.kg;
        if (P.nwg >= 65536) return hipErrorInvalidValue;
        P.nbk = (P.nb + P.kg - 1) / P.kg;
        P.ltw = P.tw == 4 ? 2 : P.tw == 2 ? 1 : 0;
        P.kg_inv = P.kg > 1 ? (uint32_t)((0x100000000ull + P.kg - 1) / P.kg) : 0u;
        wgs = std::max(wgs, P.nwg);
    }
    if (wgs == 0) return hipSuccess;
    const int kind = jobs[0].routed ? FK_ROUTED : jobs[0].scores ? FK_ROUTE : FK_PLAIN;
    const int xf = jobs[0].xform;
    for (int i = 1; i < n; i++)
        if ((jobs[i].routed ? FK_ROUTED : jobs[i].scores ? FK_ROUTE : FK_PLAIN) != kind || jobs[i].xform != xf)
            return hipErrorInvalidValue;
    // every problem's K-slice within 32 blocks: two x pairs per wave suffice
    bool short_slices = true;
    for (int i = 0; i < n; i++)
        if (B.p[i].nbk > 32) short_slices = false;
    (void)hipGetLastError();  // report only this launch
    const dim3 grid(wgs, n), block(FAST_WG);
    // the vector-ALU variant: plain problems whose linears ask for it, with
    // no deferred slices, bias vectors or argmax keys
    bool valu = kind == FK_PLAIN && xf == XF_NONE;
    for (int i = 0; i < n && valu; i++)
        valu = jobs[i].plan->valu && !jobs[i].y2 && !jobs[i].bias2 && !jobs[i].amax;
    if (valu) {
        if (scheme == 4)
            hipLaunchKernelGGL(HIP_KERNEL_NAME(k_gemv_valu<4>), grid, block, 0, s, B);
        else
            hipLaunchKernelGGL(HIP_KERNEL_NAME(k_gemv_valu<3>), grid, block, 0, s, B);
        return hipGetLastError();
    }
#define WPCG_FAST(S, K, X) hipLaunchKernelGGL(HIP_KERNEL_NAME(k_gemv_fast<S, K, X>), grid, block, 0, s, B)
#define WPCG_FAST2(S, K, X) hipLaunchKernelGGL(HIP_KERNEL_NAME(k_gemv_fast<S, K, X, 2>), grid, block, 0, s, B)
#define WPCG_FAST_S(S)                                                               \
    do {                                                                             \
        if (kind == FK_PLAIN && xf == XF_NONE) WPCG_FAST(S, FK_PLAIN, XF_NONE);      \
        else if (kind == FK_PLAIN && xf == XF_NORM && short_slices) WPCG_FAST2(S, FK_PLAIN, XF_NORM); \
        else if (kind == FK_PLAIN && xf == XF_NORM) WPCG_FAST(S, FK_PLAIN, XF_NORM); \
        else if (kind == FK_PLAIN && xf == XF_SILU) WPCG_FAST(S, FK_PLAIN, XF_SILU); \
        else if (kind == FK_PLAIN && xf == XF_MERGE) WPCG_FAST(S, FK_PLAIN, XF_MERGE); \
        else if (kind == FK_ROUTE && xf == XF_NONE) WPCG_FAST(S, FK_ROUTE, XF_NONE); \
        else if (kind == FK_ROUTE && xf == XF_NORM) WPCG_FAST(S, FK_ROUTE, XF_NORM); \
        else if (kind == FK_ROUTED && xf == XF_SILU) WPCG_FAST(S, FK_ROUTED, XF_SILU); \
        else return hipErrorInvalidValue;                                            \
    } while (0)
    if (scheme == 4)
        WPCG_FAST_S(4);
    else
        WPCG_FAST_S(3);
#undef WPCG_FAST_S
#undef WPCG_FAST2
#undef WPCG_FAST
    return hipGetLastError();
}

hipError_t launch_route_rows(const float* scores, int n, int rows, int top_k, int norm_topk, int32_t* ids, float* w,
                             hipStream_t s)
{
    if (n < 1 || n > ROUTE_MAXN || top_k < 1 || top_k > MAX_JOBS || rows < 1) return hipErrorInvalidValue;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_route_rows, dim3(rows), dim3(512), 0, s, scores, n, top_k, norm_topk, ids, w);
    return hipGetLastError();
}

hipError_t launch_embed(const DeviceMatrix& m, uint32_t row, float* out, hipStream_t s)
{
    dim3 grid((unsigned)((m.cols + 255) / 256));
    (void)hipGetLastError();  // report only this launch
    if (m.scheme == 4)
        hipLaunchKernelGGL(k_embed<4>, grid, dim3(256), 0, s, m.codes, m.hp, m.params, out,
                           (size_t)row, (int)m.nb);
    else
        hipLaunchKernelGGL(k_embed<3>, grid, dim3(256), 0, s, m.codes, m.hp, m.params, out,
                           (size_t)row, (int)m.nb);
    return hipGetLastError();
}

hipError_t launch_embed_tok(const DeviceMatrix& m, const uint32_t* tokens, const DecodeState* st,
                            float* out, hipStream_t s, const float* cos_t, const float* sin_t, int half,
                            float* rope)
{
    if (rope && (!cos_t || !sin_t || half < 1 || 2 * half > 256)) return hipErrorInvalidValue;
    dim3 grid((unsigned)((m.cols + 255) / 256));
    (void)hipGetLastError();  // report only this launch
    if (m.scheme == 4)
        hipLaunchKernelGGL(k_embed_tok<4>, grid, dim3(256), 0, s, m.codes, m.hp, m.params, out, tokens,
                           st, (int)m.nb, (uint32_t)m.rows, cos_t, sin_t, half, rope);
    else
        hipLaunchKernelGGL(k_embed_tok<3>, grid, dim3(256), 0, s, m.codes, m.hp, m.params, out, tokens,
                           st, (int)m.nb, (uint32_t)m.rows, cos_t, sin_t, half, rope);
    return hipGetLastError();
}

hipError_t launch_embed_rows(const DeviceMatrix& m, const uint32_t* tokens, int n, float* out, hipStream_t s)
{
    dim3 grid((unsigned)((m.cols + 255) / 256), (unsigned)n);
    (void)hipGetLastError();
    if (m.scheme == 4)
        hipLaunchKernelGGL(k_embed_rows<4>, grid, dim3(256), 0, s, m.codes, m.hp, m.params, out, tokens, (int)m.nb,
                           (uint32_t)m.rows);
    else
        hipLaunchKernelGGL(k_embed_rows<3>, grid, dim3(256), 0, s, m.codes, m.hp, m.params, out, tokens, (int)m.nb,
                           (uint32_t)m.rows);
    return hipGetLastError();
}

hipError_t launch_dequant(const DeviceMatrix& m, int rounding, float* w, hipStream_t s)
{
    const size_t n = (size_t)m.rows * m.cols;
    dim3 grid((unsigned)((n + 255) / 256));
    (void)hipGetLastError();  // report only this launch
    if (m.scheme == 4)
        hipLaunchKernelGGL(k_dequant<4>, grid, dim3(256), 0, s, m.codes, m.hp, m.params, w, n,
                           (int)m.nb, rounding);
    else
        hipLaunchKernelGGL(k_dequant<3>, grid, dim3(256), 0, s, m.codes, m.hp, m.params, w, n,
                           (int)m.nb, rounding);
    return hipGetLastError();
}

}  // namespace wpcg
