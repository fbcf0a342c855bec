// Batched dequant-GEMM Y = X W^T for M >= 2 activations (multi-sequence
// decode, chunked prefill) on the bf16 matrix cores of gfx950.
//
// The weights are used as they sit in HBM (tile-major planes, see
// wpcg_internal.hpp) and are never dequantized: the integer codes (0..15 or
// 0..63) are exact in bf16, so v_mfma_f32_16x16x32_bf16 gives, per 16-row
// tile and 128-value block b, the dots D = sum code * x over the block with
// exact products and fp32 accumulation. Each block then adds
//     scale * D + zp * S_b,   S_b = sum of the block's x (per column)
// in fp32, which is the block's w = zp + code * scale without ever rounding
// w. The only rounding of inputs is x to bf16 (none when X is given in
// bf16). (The matrix cores are fed 128 + code, one byte permute per two
// codes; see codes_bf16.)
//
// k-order. A lane of group g (lanes 16g..16g+15) of a tile's 16-byte code
// word holds the codes of k = 8q + g + 4h (q < 8, h < 2; low nibbles) and
// k + 64 (high nibbles), so for kstep i (0..3) lane group g feeds the
// matrix core the eight values of
//     k(i, g, s) = 8s + g + 4(i & 1) + 64(i >> 1),   s = 0..7
// and X is packed once per call into that order (k_gemm_pack): fragment
// (block b, column tile n, kstep i) is 64 lanes x 8 bf16, lane g*16 + c
// holding column n*16 + c.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "wpcg_internal.hpp"
#include "xdigits.h"
#include "xpack.h"

namespace wpcg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint32_t bits)
{
    _Float16 h;
    uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
constexpr int CPOL_NT = 2;   // streamed once
constexpr int CPOL_SC1 = 16; // coherent across the device's L2s (agent scope)

// ---- X -> bf16 fragments in k(i, g, s) order, plus per-block column sums
// of the rounded values. One workgroup per (block, column tile): wave i is
// kstep i, lane g*16 + c column c. SPLIT (fp32 X): column tiles
// [0, NT/2) hold hi = bf16(x) and tiles [NT/2, NT) lo = bf16(x - hi) of the
// same columns, so hi + lo carries x to a relative 2^-18.
//
// The XT column tiles of a block form groups of NT (the tiles one k_gemm
// workgroup reads); with SPLIT each group holds NT/2 hi tiles then the NT/2
// lo tiles of the same columns.
template <bool BF16_IN, bool SPLIT>
__global__ __launch_bounds__(256) void k_gemm_pack(const void* __restrict__ X, int M, int K, int XT, int NT,
                                                   u32x4* __restrict__ xf, float* __restrict__ xsum)
{
    __shared__ float red[4][16];
    const int b = blockIdx.x / XT, n = blockIdx.x % XT;
    const int i = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const int cg = n / NT, w = n % NT;  // group, tile within it
    const int nh = SPLIT ? NT / 2 : NT;
    const bool lo_part = SPLIT && w >= nh;
    const int m = (cg * nh + (lo_part ? w - nh : w)) * 16 + c;
    float v[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const size_t k = (size_t)b * 128 + gk(i, g, s);
        if (m >= M)
            v[s] = 0.0f;
        else if constexpr (BF16_IN)
            v[s] = __uint_as_float((uint32_t)static_cast<const uint16_t*>(X)[(size_t)m * K + k] << 16);
        else
            v[s] = static_cast<const float*>(X)[(size_t)m * K + k];
        if (lo_part) v[s] = v[s] - bf16_round(v[s]);  // exact in fp32
    }
    u32x4 o;
    o.x = pk_bf16(v[0], v[1]);
    o.y = pk_bf16(v[2], v[3]);
    o.z = pk_bf16(v[4], v[5]);
    o.w = pk_bf16(v[6], v[7]);
    xf[((size_t)(b * XT + n) * 4 + i) * 64 + lane] = o;
    float sum = ((bf16_lo(o.x) + bf16_hi(o.x)) + (bf16_lo(o.y) + bf16_hi(o.y))) +
                ((bf16_lo(o.z) + bf16_hi(o.z)) + (bf16_lo(o.w) + bf16_hi(o.w)));
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    if (g == 0) red[i][c] = sum;
    __syncthreads();
    if (threadIdx.x < 16)
        xsum[(size_t)b * XT * 16 + n * 16 + threadIdx.x] =
            (red[0][threadIdx.x] + red[1][threadIdx.x]) + (red[2][threadIdx.x] + red[3][threadIdx.x]);
}

// Another matrix of a launch that shares X (and K) with the first: its
// workgroups start at wg0 (a multiple of 8, so each matrix's row groups keep
// their XCDs).
struct GemmMat {
    const uint8_t* codes;
    const uint8_t* hp;
    const uint32_t* params;
    float* y;
    const float* bias;
    int rows, rows_pad, rgs, rgs8, wg0;
    int rope;            // GEMM_ROPE_*: the prefill's q, k or v epilogue
    float* cache;        // k, v: the layer's cache [head][max_pos][128]
    const float* nw;     // q, k: the head norm's weights [128]
};
constexpr int GEMM_MAX_MATS = 3;
static_assert(GEMM_MAX_MATS == sizeof(GemmRope::mode) / sizeof(int), "GemmRope holds every matrix of a launch");
struct GemmArgs {
    const uint8_t* codes;
    const uint8_t* hp;
    const uint32_t* params;
    const u32x4* xf;     // packed X, [nb][NT][4][64] fragments
    const float* xsum;   // [nb][NT*16]
    float* y;            // [M][rows]
    const float* bias;   // [rows] or null
    const float* res;    // [M][rows] added to Y (may be y itself) or null
    float* part;         // [kg][NT*16][rows_pad] (kg > 1), summed by k_gemm_reduce
    int rows, rows_pad, nb, M, kg;
    // column groups: the packed X holds xt tiles per block (groups of NT);
    // with rgs8 > 0 workgroup cg * rgs8 + rg takes row group rg (< rgs) of
    // column group cg, kg = 1 (the groups of one row group share an XCD's L2)
    int xt, rgs, rgs8;
    int nmore;  // further matrices over the same X (rgs8 > 0 only)
    GemmMat more[GEMM_MAX_MATS - 1];
    // the prefill's q/k/v epilogue (GemmRope): this matrix's mode, cache and
    // norm weights, and the rotation tables of every matrix
    int rope;
    float* cache;
    const float* nw;
    const float* cos_t;  // [max_pos][64]
    const float* sin_t;
    int pos0, max_pos;
    float eps;
};

// The value written for output (m, row): the sum, the bias, the residual.
__device__ __forceinline__ float out_val(float v, const float* bias, const float* res, int rows, int m, int row)
{
    if (bias) v += bias[row];
    if (res) v += res[(size_t)m * rows + row];
    return v;
}

// Eight bf16 of one fragment lane from two consecutive-k pieces: the low
// (odd = 0) or high (odd = 1) halves of dwords a (slot 2q) and b (slot 2q+1).
__device__ __forceinline__ uint32_t pick_halves(uint32_t a, uint32_t b, int odd)
{
    return odd ? (a >> 16) | (b & 0xFFFF0000u) : (a & 0xFFFFu) | (b << 16);
}

constexpr int GM_WG = GEMM_WG_THREADS;   // 8 waves, two per SIMD
constexpr int GM_RT = GEMM_TILES_PER_WAVE;  // row tiles per wave: a row group is GM_WG / 64 * GM_RT = 8 tiles
constexpr int GM_R = 4;                  // blocks of X per LDS round (one barrier per round)
constexpr int GM_LA = GM_R;              // blocks of codes in flight per wave (one ring slot per block of a round)

// Eight codes (two dwords of one byte each, every code < 128) -> the eight
// bf16 values 128 + code, exact: their bit patterns are 0x4300 | code, so
// one byte permute makes two of them. The matrix cores then return
// D' = sum (128 + code) x = D + 128 S, and a block adds
// scale * D' + (zp - 128 scale) * S, which is scale * D + zp * S.
__device__ __forceinline__ bf16x8 codes_bf16(uint32_t a, uint32_t b)
{
    u32x4 r;
    r.x = __builtin_amdgcn_perm(0x43434343u, a, 0x04010400u);
    r.y = __builtin_amdgcn_perm(0x43434343u, a, 0x04030402u);
    r.z = __builtin_amdgcn_perm(0x43434343u, b, 0x04010400u);
    r.w = __builtin_amdgcn_perm(0x43434343u, b, 0x04030402u);
    bf16x8 o;
    __builtin_memcpy(&o, &r, 16);
    return o;
}
// zero point of the offset codes: zp - 128 * scale
__device__ __forceinline__ float zp_off(uint32_t p) { return __builtin_fmaf(-128.0f, h2f(p >> 16), h2f(p & 0xFFFFu)); }

// The prefill's q/k/v epilogue (kg = 1, a row group of 8 waves x 16 rows =
// one 128-wide head, 32 columns = tokens mcol0 ..): q and k get the head
// RMSNorm (FAST: the squares of each lane's four rows by fused multiply-adds,
// the lane groups by exchanges, the eight waves through LDS in a fixed
// order; then (x * scale) * w) and the rotation at each token's position
// (rows d < 64 and d + 64 are a pair: y c - y' s and y' c + y s, as
// fa_norm_rope). The normed rows are staged in LDS as [token][d] and leave
// as whole 16-byte pieces of a token's row (thread t: token t / 16, rows
// 4 (t % 16) .. +3 and the same + 64): q into Y, k and v (v as computed)
// into the cache rows of their position. The bias is added first.
template <typename Acc>
__device__ __forceinline__ void rope_epilogue(const GemmArgs& P, const Acc& acc, int rg, int wave, int g, int j,
                                              int mcol0, float* ex)
{
    constexpr int TOK = 32, EXS = 132;  // ex: [TOK][EXS], rows 16-byte aligned
    float* rsum = ex + TOK * EXS;       // [8][TOK] sums of squares
    const int mode = P.rope;
    float v[2][4];
#pragma unroll
    for (int n = 0; n < 2; n++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int d = wave * 16 + 4 * g + q;
            v[n][q] = acc[0][n][q] + (P.bias ? P.bias[rg * 128 + d] : 0.0f);
        }
    __syncthreads();  // every wave is done with the X buffers
    float sc[2] = {1.0f, 1.0f};
    if (mode != GEMM_ROPE_V) {
#pragma unroll
        for (int n = 0; n < 2; n++) {
            float ss = fmaf(v[n][3], v[n][3], fmaf(v[n][2], v[n][2], fmaf(v[n][1], v[n][1], v[n][0] * v[n][0])));
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            if (g == 0) rsum[wave * TOK + n * 16 + j] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int n = 0; n < 2; n++) {
            const float* r = rsum + n * 16 + j;
            const float tot = ((r[0] + r[TOK]) + (r[2 * TOK] + r[3 * TOK])) +
                              ((r[4 * TOK] + r[5 * TOK]) + (r[6 * TOK] + r[7 * TOK]));
            sc[n] = __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(__fdiv_rn(tot, 128.0f), P.eps)));
        }
    }
#pragma unroll
    for (int n = 0; n < 2; n++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int d = wave * 16 + 4 * g + q;
            ex[(n * 16 + j) * EXS + d] = mode != GEMM_ROPE_V ? (v[n][q] * sc[n]) * P.nw[d] : v[n][q];
        }
    __syncthreads();
    const int tok = threadIdx.x >> 4, d1 = 4 * (threadIdx.x & 15), m = mcol0 + tok;
    if (m >= P.M) return;
    const int pos = P.pos0 + m;
    const float4 y1 = *reinterpret_cast<const float4*>(&ex[tok * EXS + d1]);
    const float4 y2 = *reinterpret_cast<const float4*>(&ex[tok * EXS + d1 + 64]);
    float4 o1 = y1, o2 = y2;
    if (mode != GEMM_ROPE_V) {
        const float4 c = *reinterpret_cast<const float4*>(P.cos_t + (size_t)pos * 64 + d1);
        const float4 sn = *reinterpret_cast<const float4*>(P.sin_t + (size_t)pos * 64 + d1);
        o1 = make_float4(fmaf(y1.x, c.x, -(y2.x * sn.x)), fmaf(y1.y, c.y, -(y2.y * sn.y)),
                         fmaf(y1.z, c.z, -(y2.z * sn.z)), fmaf(y1.w, c.w, -(y2.w * sn.w)));
        o2 = make_float4(fmaf(y2.x, c.x, y1.x * sn.x), fmaf(y2.y, c.y, y1.y * sn.y), fmaf(y2.z, c.z, y1.z * sn.z),
                         fmaf(y2.w, c.w, y1.w * sn.w));
    }
    float* dst = mode == GEMM_ROPE_Q ? P.y + (size_t)m * P.rows + rg * 128
                                     : P.cache + ((size_t)rg * P.max_pos + pos) * 128;
    *reinterpret_cast<float4*>(dst + d1) = o1;
    *reinterpret_cast<float4*>(dst + d1 + 64) = o2;
}

// A workgroup of 8 waves (two per SIMD, so one wave's waits are filled by the
// other's work) computes one row group (8 row tiles) for all NT*16 columns
// over one K-slice. Wave w takes GM_RT tiles from rg*8 + w*GM_RT and every
// column tile, so each tile's codes are unpacked once per block. The codes
// come straight from HBM into registers, GM_LA blocks ahead.
//
// X goes through LDS in rounds of GM_R blocks, double buffered, with one
// barrier per round: round r+1's fragments are fetched into registers at
// the start of round r-1, stored into the free buffer at the start of round
// r (after the barrier that ended round r-1, which every read of that
// buffer preceded) and published by the barrier that ends round r. Each wave
// reads a column tile's fragments from LDS one tile ahead of its matrix
// work, so LDS reads overlap the dots; the barrier that ends a round sits
// before the round's last tile, whose fragments are already in registers,
// and is followed by the read of the next round's first tile.
//
// Every buffer load has an exact range: loads past the slice return zeros,
// and a zero block adds exactly 0.
//
// SPLIT: column tiles [0, NT/2) are the hi parts and [NT/2, NT) the lo parts
// of the same NT/2 column tiles (k_gemm_pack<*, true>); after the loop the
// wave adds each lo tile's sums to its hi tile's and writes the hi tiles.
template <int SCHEME, int NT, bool SPLIT>
__global__ __launch_bounds__(GM_WG) void k_gemm(const GemmArgs P0)
{
    static_assert(!SPLIT || NT % 2 == 0, "split needs hi and lo tiles");
    constexpr int RT = GM_RT;
    static_assert(GM_WG / 64 * RT == 8, "a row group is 8 tiles");
    constexpr int FW = NT * 256;                              // 16-byte X words per block
    constexpr int XV = (GM_R * FW + GM_WG - 1) / GM_WG;       // X words per thread per round
    constexpr int SN = GM_R * NT * 16;                        // X sums per round
    constexpr int SV = (SN + GM_WG - 1) / GM_WG;
    __shared__ __align__(16) u32x4 xb[2][GM_R * FW];
    __shared__ float xsb[2][SN];

    // this workgroup's matrix (uniform)
    GemmArgs P = P0;
    int bid = (int)blockIdx.x;
    for (int e = P0.nmore - 1; e >= 0; e--)
        if (bid >= P0.more[e].wg0) {
            const GemmMat& mm = P0.more[e];
            P.codes = mm.codes;
            P.hp = mm.hp;
            P.params = mm.params;
            P.y = mm.y;
            P.bias = mm.bias;
            P.rows = mm.rows;
            P.rows_pad = mm.rows_pad;
            P.rgs = mm.rgs;
            P.rgs8 = mm.rgs8;
            P.rope = mm.rope;
            P.cache = mm.cache;
            P.nw = mm.nw;
            bid -= mm.wg0;
            break;
        }
    const int kg = P.kg, nb = P.nb, XT = P.xt;
    int kgi, rg, cg;
    if (P.rgs8) {  // workgroup (kgi * ncg + cg) * rgs8 + rg
        const int ncg = P.xt / NT;
        rg = bid % P.rgs8;
        cg = (bid / P.rgs8) % ncg;
        kgi = bid / P.rgs8 / ncg;
        if (rg >= P.rgs) return;  // padding of the row groups, uniform
    } else {
        kgi = bid % kg;
        rg = bid / kg;
        cg = 0;
    }
    const int mcol0 = cg * (SPLIT ? NT / 2 : NT) * 16;  // the group's first output column
    const int nbk = (nb + kg - 1) / kg;
    const int b0 = min(kgi * nbk, nb);
    const int nbl = max(0, min(nb, b0 + nbk) - b0);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int g = lane >> 4, j = lane & 15;
    const int ntiles = P.rows_pad / TILE_ROWS;
    const int T0 = rg * 8 + wave * RT;

    __amdgpu_buffer_rsrc_t crs[RT], hrs[RT], prs[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int T = T0 + rt;
        const bool ok = T < ntiles;
        const size_t rec = (size_t)min(T, ntiles - 1) * nb + b0;
        crs[rt] = buf_rsrc(P.codes + rec * CODE_REC, ok ? nbl * (int)CODE_REC : 0);
        hrs[rt] = buf_rsrc((SCHEME == 3 ? P.hp : P.codes) + rec * HP_REC,
                           ok && SCHEME == 3 ? nbl * (int)HP_REC : 0);
        prs[rt] = buf_rsrc(P.params + rec * TILE_ROWS, ok ? nbl * TILE_ROWS * 4 : 0);
    }
    const auto xrs = buf_rsrc(P.xf + ((size_t)b0 * XT + cg * NT) * 256, (nbl * XT - cg * NT) * 4096);
    const auto srs = buf_rsrc(P.xsum + (size_t)b0 * XT * 16 + cg * NT * 16, (nbl * XT - cg * NT) * 64);

    u32x4 cr[GM_LA][RT], pr[GM_LA][RT];
    u32x2 hr[GM_LA][RT];
    auto load_codes = [&](int u, int b) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            cr[u][rt] = __builtin_amdgcn_raw_buffer_load_b128(crs[rt], b * (int)CODE_REC + lane * 16, 0, CPOL_NT);
            if constexpr (SCHEME == 3)
                hr[u][rt] = __builtin_amdgcn_raw_buffer_load_b64(hrs[rt], b * (int)HP_REC + lane * 8, 0, CPOL_NT);
            pr[u][rt] = __builtin_amdgcn_raw_buffer_load_b128(prs[rt], b * 64 + g * 16, 0, CPOL_NT);
        }
    };
    // X of round r: thread t holds the round's 16-byte words t + v*GM_WG
    // (block r*GM_R + word / FW, word % FW of it) and sums t + v*GM_WG
    // (block r*GM_R + i / (NT*16), column i % (NT*16)).
    u32x4 xr[XV];
    float sr[SV];
    auto load_round = [&](int r) {
#pragma unroll
        for (int v = 0; v < XV; v++) {
            const int i = min((int)threadIdx.x + v * GM_WG, GM_R * FW - 1);
            xr[v] = __builtin_amdgcn_raw_buffer_load_b128(xrs, ((r * GM_R + i / FW) * XT * 256 + i % FW) * 16, 0, 0);
        }
#pragma unroll
        for (int v = 0; v < SV; v++) {
            const int i = min((int)threadIdx.x + v * GM_WG, SN - 1);
            sr[v] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                srs, ((r * GM_R + i / (NT * 16)) * XT * 16 + i % (NT * 16)) * 4, 0, 0));
        }
    };
    // Every thread stores every word it loaded: a thread past the end holds
    // a copy of the last word (its load index was clamped) and writes it to
    // the same place. A store under a condition would leave that load
    // pending on one path into the round loop, and the wait counts merged at
    // the loop edge would then drain every load in flight each round.
    auto store_round = [&](int buf) {
#pragma unroll
        for (int v = 0; v < XV; v++) xb[buf][min((int)threadIdx.x + v * GM_WG, GM_R * FW - 1)] = xr[v];
#pragma unroll
        for (int v = 0; v < SV; v++) xsb[buf][min((int)threadIdx.x + v * GM_WG, SN - 1)] = sr[v];
    };
    // the fragments of kstep i of every column tile of block u of a round buffer
    auto read_kstep = [&](bf16x8 (&B)[NT], int buf, int u, int i) {
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const u32x4 w = xb[buf][u * FW + (n * 4 + i) * 64 + lane];
            __builtin_memcpy(&B[n], &w, 16);
        }
    };
    // The zero-point term of a round, sum_b zp(row, b) * S(b, col) over its
    // GM_R = 4 blocks, is one fp32 matrix-core product per column tile:
    // lane (g, j) supplies zp_off of row j of block g (A, 16 x 4) and the
    // block-g sum of column n*16 + j (B, 4 x 16), and the product adds into
    // the accumulators in their own layout. Zero-point words of round r:
    // one per lane and row tile.
    static_assert(GM_R == 4, "a round is the k = 4 of v_mfma_f32_16x16x4_f32");
    auto load_zp = [&](uint32_t (&z)[RT], int r) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
            z[rt] = __builtin_amdgcn_raw_buffer_load_b32(prs[rt], ((r * GM_R + g) * TILE_ROWS + j) * 4, 0, CPOL_NT);
    };

    // prologue: round 0 and the first GM_LA blocks of codes, then round 1,
    // in the order the loop keeps (so the wait counts at its head match)
    uint32_t zc[RT], zn[RT];
    load_round(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < GM_LA; u++) {
        load_codes(u, u);
        __builtin_amdgcn_sched_barrier(0);
    }
    load_zp(zc, 0);
    store_round(0);
    load_round(1);
    __syncthreads();

    f32x4 acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int n = 0; n < NT; n++) acc[rt][n] = f32x4{0.f, 0.f, 0.f, 0.f};

    bf16x8 Bc[NT];
    read_kstep(Bc, 0, 0, 0);

    // Whole rounds of unconditional steps (guarded steps would merge the
    // wait-counter state at the loop edge and drain every load in flight).
    const int nrounds = (nbl + GM_R - 1) / GM_R;
    for (int r = 0; r < nrounds; r++) {
        const int buf = r & 1;
        // this round's block sums for the zero-point product, read before the
        // barrier after which the buffer may be refilled
        float Sz[NT];
#pragma unroll
        for (int n = 0; n < NT; n++) Sz[n] = xsb[buf][g * NT * 16 + n * 16 + j];
        store_round(buf ^ 1);  // round r+1 into the buffer round r-1 left
        load_round(r + 2);
        load_zp(zn, r + 1);
#pragma unroll
        for (int u = 0; u < GM_R; u++) {
            const int b = r * GM_R + u;
            bf16x8 A[RT][4];
            float sc[RT][4];
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const u32x4 U = cr[u][rt];
                const uint32_t MK = 0x0F0F0F0Fu;
                u32x4 lo = {U.x & MK, U.y & MK, U.z & MK, U.w & MK};
                u32x4 hi = {(U.x >> 4) & MK, (U.y >> 4) & MK, (U.z >> 4) & MK, (U.w >> 4) & MK};
                if constexpr (SCHEME == 3) {
                    const uint32_t T6 = 0x30303030u, hx = hr[u][rt].x, hy = hr[u][rt].y;
                    lo.x |= (hx << 4) & T6; lo.y |= (hx << 2) & T6;
                    lo.z |= (hy << 4) & T6; lo.w |= (hy << 2) & T6;
                    hi.x |= hx & T6;        hi.y |= (hx >> 2) & T6;
                    hi.z |= hy & T6;        hi.w |= (hy >> 2) & T6;
                }
                A[rt][0] = codes_bf16(lo.x, lo.y);
                A[rt][1] = codes_bf16(lo.z, lo.w);
                A[rt][2] = codes_bf16(hi.x, hi.y);
                A[rt][3] = codes_bf16(hi.z, hi.w);
                const u32x4 p = pr[u][rt];
                sc[rt][0] = h2f(p.x >> 16);
                sc[rt][1] = h2f(p.y >> 16);
                sc[rt][2] = h2f(p.z >> 16);
                sc[rt][3] = h2f(p.w >> 16);
            }
            load_codes(u, b + GM_LA);
            // kstep-major: the NT column tiles' products of one kstep are
            // independent, so the matrix cores take them back to back while
            // the next kstep's fragments come from LDS (a column tile's four
            // ksteps in a row would each wait for the one before: M = 64
            // rounds 3.3 -> 2.9 us)
            f32x4 D[RT][NT];
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int n = 0; n < NT; n++) D[rt][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // the next kstep's fragments: this round's buffer, or (before
                // the round's last kstep, after the barrier) the next round's
                bf16x8 Bn[NT];
                if (i + 1 < 4) {
                    read_kstep(Bn, buf, u, i + 1);
                } else if (u + 1 < GM_R) {
                    read_kstep(Bn, buf, u + 1, 0);
                } else {
                    __syncthreads();
                    read_kstep(Bn, buf ^ 1, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);  // the reads go out before this kstep's products
#pragma unroll
                for (int n = 0; n < NT; n++)
#pragma unroll
                    for (int rt = 0; rt < RT; rt++)
                        D[rt][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[rt][i], Bc[n], D[rt][n], 0, 0, 0);
#pragma unroll
                for (int n = 0; n < NT; n++) Bc[n] = Bn[n];
                // keep the kstep's products together (the scheduler would
                // otherwise regroup them into per-tile chains)
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int n = 0; n < NT; n++)
#pragma unroll
                    for (int q = 0; q < 4; q++) acc[rt][n][q] = __builtin_fmaf(sc[rt][q], D[rt][n][q], acc[rt][n][q]);
        }
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const float za = zp_off(zc[rt]);
#pragma unroll
            for (int n = 0; n < NT; n++) acc[rt][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(za, Sz[n], acc[rt][n], 0, 0, 0);
            zc[rt] = zn[rt];
        }
    }

    if constexpr (SPLIT) {  // lo tiles [NT/2, NT) join their hi tiles
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int n = 0; n < NT / 2; n++) acc[rt][n] = acc[rt][n] + acc[rt][n + NT / 2];
    }
    // the column tiles this wave writes: [0, NW) (SPLIT: the hi tiles)
    constexpr int NW = SPLIT ? NT / 2 : NT;

    // lane (g, j) holds rows 4g..4g+3 of each tile for column n*16 + j;
    // the split-K partials have Mp columns (every column group's with rgs8)
    const int Mp = P.rgs8 ? P.xt / NT * NW * 16 : NT * 16;
    if constexpr (SPLIT && RT == 1 && NW == 2) {
        if (P.rope) {  // uniform: the row group is one 128-wide head
            rope_epilogue(P, acc, rg, wave, g, j, mcol0, reinterpret_cast<float*>(&xb[0][0]));
            return;
        }
    }
    if (kg == 1) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int n = 0; n < NW; n++) {
                const int m = mcol0 + n * 16 + j, row = (T0 + rt) * TILE_ROWS + 4 * g;
                if (m >= P.M) continue;
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (row + q < P.rows)
                        P.y[(size_t)m * P.rows + row + q] = out_val(acc[rt][n][q], P.bias, P.res, P.rows, m, row + q);
            }
        return;
    }
    // Split K: the slice's partials go to part[kgi]; k_gemm_reduce, the
    // next launch on the stream, adds the slices in slice order
    // (deterministic) with every CU taking part. (A handoff inside this
    // kernel, the last workgroup of a row group adding all slices after
    // device-scope publishes and a counter, left that sum to one CU per row
    // group: 4.1 us of a 22 us M = 64 gate/up launch at 2 slices, 6.7 of 25
    // us for down_proj at 8.)
    const auto prt = buf_rsrc(P.part, kg * Mp * P.rows_pad * 4);
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int n = 0; n < NW; n++) {
            const int m = mcol0 + n * 16 + j, row = (T0 + rt) * TILE_ROWS + 4 * g;
            if (T0 + rt < ntiles) {
                u32x4 v;
                __builtin_memcpy(&v, &acc[rt][n], 16);
                __builtin_amdgcn_raw_buffer_store_b128(v, prt, ((kgi * Mp + m) * P.rows_pad + row) * 4, 0, 0);
            }
        }
}

// The split-K sum of k_gemm: Y[m][row] = sum over the kg slices of
// part[k][m][row] in slice order, then the bias and the residual. One thread
// per four rows of one column; reads and writes run along the rows.
__global__ __launch_bounds__(256) void k_gemm_reduce(const float* __restrict__ part, int kg, int Mp, int rows_pad,
                                                     int rows, int M, const float* bias, const float* res,
                                                     float* y)
{
    const int per = rows_pad / 4;
    const int idx = (int)(blockIdx.x * 256 + threadIdx.x);
    const int m = idx / per, row = (idx - m * per) * 4;
    if (m >= M) return;
    const f32x4* p = reinterpret_cast<const f32x4*>(part + (size_t)m * rows_pad + row);
    const size_t stride = (size_t)Mp * rows_pad / 4;  // f32x4 per slice
    f32x4 s = p[0];
    for (int k = 1; k < kg; k++) s = s + p[k * stride];
#pragma unroll
    for (int q = 0; q < 4; q++)
        if (row + q < rows) y[(size_t)m * rows + row + q] = out_val(s[q], bias, res, rows, m, row + q);
}

// ---- M <= 16: one kernel. The workgroup packs its whole K-slice of X
// (row-major fp32 or bf16, straight from the caller's buffer) into bf16
// fragments in LDS; its X loads are issued first, then its first blocks of
// codes, so the pack waits for X alone. Two waves own each row tile, one
// per half of the slice, so two waves share every SIMD; each runs its
// blocks in pairs (two independent matrix-core chains) without barriers,
// and the halves are added in a fixed order at the end.
constexpr int GS_WG = 512;
constexpr int GS_TILES = GS_WG / 128;  // row tiles per workgroup
constexpr int GS_LA = 10;              // blocks of codes in flight per wave (even)

struct GemmSmallArgs {
    const uint8_t* codes;
    const uint8_t* hp;
    const uint32_t* params;
    const void* x;       // [M][K] row-major
    float* y;
    const float* bias;
    const float* res;    // [M][rows] added to Y (may be y itself) or null
    float* part;         // [kg][16][rows_pad] (kg > 1)
    uint32_t* counters;
    int rows, rows_pad, nb, M, kg;
};


// The fp32 value held in a dword minus its bf16 rounding (exact), i.e. the
// lo part of a SPLIT column.
__device__ __forceinline__ float lo_of(uint32_t bits)
{
    const float v = __uint_as_float(bits);
    return v - bf16_round(v);
}

// SPLIT (fp32 X, M <= 8): fragment columns [0, M) carry hi = bf16(x) and
// [M, 2M) lo = bf16(x - hi) of the same rows; after the dots lane j adds
// lane j + M (hi + lo) and writes column j.
template <int SCHEME, bool BF16_IN, bool SPLIT>
__global__ __launch_bounds__(GS_WG) void k_gemm_small(const GemmSmallArgs P)
{
    static_assert(!(SPLIT && BF16_IN), "bf16 X has no lo part");
    __shared__ __align__(16) u32x4 xb[GEMM_SMALL_MAXBK][4][64];
    __shared__ float psum[GEMM_SMALL_MAXBK][2][16];
    __shared__ __align__(16) f32x4 red[GS_TILES][64];
    __shared__ int s_last;

    const int kg = P.kg, nb = P.nb, K = nb * 128, M = P.M;
    const int kgi = blockIdx.x % kg, rg = blockIdx.x / kg;
    const int Mx = SPLIT ? 2 * M : M;  // fragment columns in use
    const int nbk = (nb + kg - 1) / kg;
    const int b0 = min(kgi * nbk, nb);
    const int nbl = max(0, min(nb, b0 + nbk) - b0);  // <= GEMM_SMALL_MAXBK (the planner's rule)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int g = lane >> 4, j = lane & 15;
    const int ntiles = P.rows_pad / TILE_ROWS;
    const int T = rg * GS_TILES + (wave % GS_TILES);  // this wave's row tile
    const bool tile_ok = T < ntiles;
    const int part_k = wave / GS_TILES;                // half of the slice
    const int hb = (nbl + 1) / 2;
    const int kb0 = part_k ? hb : 0;                   // first block (within the slice)
    const int kn = part_k ? nbl - hb : hb;             // blocks of this half

    // ---- X loads first. Task (blk, c, h), c < M: the 64 values k in
    // [64h, 64h+64) of row c of block blk, as eight 16-byte pieces of
    // consecutive k; a thread takes tasks t and t + 512 (ntask <= 960).
    constexpr int es = BF16_IN ? 2 : 4;
    constexpr int PIECES = BF16_IN ? 8 : 16;  // 16-byte loads per task
    const auto xrs = buf_rsrc(static_cast<const uint8_t*>(P.x) + (size_t)b0 * 128 * es,
                              (int)(((size_t)(M - 1) * K + (size_t)nbl * 128) * es));
    const int ntask = nbl * 2 * Mx;
    u32x4 xv[2][PIECES];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int t = threadIdx.x + r * GS_WG;
        const int blk = t / (2 * Mx), c = (t >> 1) % Mx, h = t & 1;
        const int xr = SPLIT && c >= M ? c - M : c;  // the X row of fragment column c
        const int base = t < ntask ? (xr * K + blk * 128 + 64 * h) * es : 0x7FFFFFF0;  // past the range: zeros
#pragma unroll
        for (int p = 0; p < PIECES; p++) xv[r][p] = __builtin_amdgcn_raw_buffer_load_b128(xrs, base + p * 16, 0, 0);
    }

    // ---- then the first GS_LA blocks of this wave's codes
    const size_t rec = (size_t)min(T, ntiles - 1) * nb + b0 + kb0;
    const auto crs = buf_rsrc(P.codes + rec * CODE_REC, tile_ok ? kn * (int)CODE_REC : 0);
    const auto hrs = buf_rsrc((SCHEME == 3 ? P.hp : P.codes) + rec * HP_REC, tile_ok && SCHEME == 3 ? kn * (int)HP_REC : 0);
    const auto prs = buf_rsrc(P.params + rec * TILE_ROWS, tile_ok ? kn * TILE_ROWS * 4 : 0);
    u32x4 cr[GS_LA], pr[GS_LA];
    u32x2 hr[GS_LA];
    auto load_codes = [&](int u, int b) {
        cr[u] = __builtin_amdgcn_raw_buffer_load_b128(crs, b * (int)CODE_REC + lane * 16, 0, CPOL_NT);
        if constexpr (SCHEME == 3) hr[u] = __builtin_amdgcn_raw_buffer_load_b64(hrs, b * (int)HP_REC + lane * 8, 0, CPOL_NT);
        pr[u] = __builtin_amdgcn_raw_buffer_load_b128(prs, b * 64 + g * 16, 0, CPOL_NT);
    };
#pragma unroll
    for (int u = 0; u < GS_LA; u++) load_codes(u, u);
    __builtin_amdgcn_sched_barrier(0);

    // ---- pack: fragment (i = 2h + ii, lane group gg) slot s <- piece s,
    // element gg + 4 ii. Columns c >= Mx are zeros.
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int t = threadIdx.x + r * GS_WG;
        if (t < ntask) {
            const int blk = t / (2 * Mx), c = (t >> 1) % Mx, h = t & 1;
            uint32_t pc[8][4];
#pragma unroll
            for (int p = 0; p < 8; p++) {
                if constexpr (BF16_IN) {
                    pc[p][0] = xv[r][p].x; pc[p][1] = xv[r][p].y; pc[p][2] = xv[r][p].z; pc[p][3] = xv[r][p].w;
                } else if (SPLIT && c >= M) {
                    const u32x4 a = xv[r][2 * p], b = xv[r][2 * p + 1];
                    pc[p][0] = pk_bf16(lo_of(a.x), lo_of(a.y));
                    pc[p][1] = pk_bf16(lo_of(a.z), lo_of(a.w));
                    pc[p][2] = pk_bf16(lo_of(b.x), lo_of(b.y));
                    pc[p][3] = pk_bf16(lo_of(b.z), lo_of(b.w));
                } else {
                    const u32x4 a = xv[r][2 * p], b = xv[r][2 * p + 1];
                    pc[p][0] = pk_bf16(__uint_as_float(a.x), __uint_as_float(a.y));
                    pc[p][1] = pk_bf16(__uint_as_float(a.z), __uint_as_float(a.w));
                    pc[p][2] = pk_bf16(__uint_as_float(b.x), __uint_as_float(b.y));
                    pc[p][3] = pk_bf16(__uint_as_float(b.z), __uint_as_float(b.w));
                }
            }
            float sum = 0.0f;
#pragma unroll
            for (int p = 0; p < 8; p++)
#pragma unroll
                for (int d = 0; d < 4; d++) sum += bf16_lo(pc[p][d]) + bf16_hi(pc[p][d]);
            psum[blk][h][c] = sum;
#pragma unroll
            for (int ii = 0; ii < 2; ii++)
#pragma unroll
                for (int gg = 0; gg < 4; gg++) {
                    const int d = (gg >> 1) + 2 * ii, odd = gg & 1;
                    u32x4 o;
                    o.x = pick_halves(pc[0][d], pc[1][d], odd);
                    o.y = pick_halves(pc[2][d], pc[3][d], odd);
                    o.z = pick_halves(pc[4][d], pc[5][d], odd);
                    o.w = pick_halves(pc[6][d], pc[7][d], odd);
                    xb[blk][2 * h + ii][gg * 16 + c] = o;
                }
        }
    }
    // zero columns Mx..15 of every fragment and their sums
    for (int t = threadIdx.x; t < nbl * 2 * (16 - Mx); t += GS_WG) {
        const int blk = t / (2 * (16 - Mx)), c = Mx + (t >> 1) % (16 - Mx), h = t & 1;
        psum[blk][h][c] = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 2; ii++)
#pragma unroll
            for (int gg = 0; gg < 4; gg++) xb[blk][2 * h + ii][gg * 16 + c] = u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();

    // One block: the matrix-core chain (four ksteps) and the fp32 epilogue.
    auto dots = [&](int u, int b) -> f32x4 {
        bf16x8 B[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u32x4 w = xb[kb0 + b][i][lane];
            __builtin_memcpy(&B[i], &w, 16);
        }
        const u32x4 U = cr[u];
        const uint32_t MK = 0x0F0F0F0Fu;
        u32x4 lo = {U.x & MK, U.y & MK, U.z & MK, U.w & MK};
        u32x4 hi = {(U.x >> 4) & MK, (U.y >> 4) & MK, (U.z >> 4) & MK, (U.w >> 4) & MK};
        if constexpr (SCHEME == 3) {
            const uint32_t T6 = 0x30303030u, hx = hr[u].x, hy = hr[u].y;
            lo.x |= (hx << 4) & T6; lo.y |= (hx << 2) & T6;
            lo.z |= (hy << 4) & T6; lo.w |= (hy << 2) & T6;
            hi.x |= hx & T6;        hi.y |= (hx >> 2) & T6;
            hi.z |= hy & T6;        hi.w |= (hy >> 2) & T6;
        }
        f32x4 D = {0.f, 0.f, 0.f, 0.f};
        D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(codes_bf16(lo.x, lo.y), B[0], D, 0, 0, 0);
        D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(codes_bf16(lo.z, lo.w), B[1], D, 0, 0, 0);
        D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(codes_bf16(hi.x, hi.y), B[2], D, 0, 0, 0);
        D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(codes_bf16(hi.z, hi.w), B[3], D, 0, 0, 0);
        return D;
    };
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    auto epilogue = [&](int u, int b, const f32x4& D) {
        const float S = psum[kb0 + b][0][j] + psum[kb0 + b][1][j];
        const u32x4 p = pr[u];
        acc[0] = __builtin_fmaf(zp_off(p.x), S, __builtin_fmaf(h2f(p.x >> 16), D[0], acc[0]));
        acc[1] = __builtin_fmaf(zp_off(p.y), S, __builtin_fmaf(h2f(p.y >> 16), D[1], acc[1]));
        acc[2] = __builtin_fmaf(zp_off(p.z), S, __builtin_fmaf(h2f(p.z >> 16), D[2], acc[2]));
        acc[3] = __builtin_fmaf(zp_off(p.w), S, __builtin_fmaf(h2f(p.w >> 16), D[3], acc[3]));
    };
    // Whole rounds of GS_LA unconditional steps, two blocks per step, each
    // refilling its ring slots GS_LA blocks ahead (past the half: zeros,
    // never used). Guarded steps inside the loop would merge the
    // wait-counter state at the loop edge and make the compiler drain every
    // load in flight once per round; the remainder runs after the loop.
    const int full = kn / GS_LA * GS_LA;
    for (int bl = 0; bl < full; bl += GS_LA) {
#pragma unroll
        for (int u = 0; u < GS_LA; u += 2) {
            const f32x4 D0 = dots(u, bl + u), D1 = dots(u + 1, bl + u + 1);
            epilogue(u, bl + u, D0);
            epilogue(u + 1, bl + u + 1, D1);
            load_codes(u, bl + u + GS_LA);
            load_codes(u + 1, bl + u + 1 + GS_LA);
            __builtin_amdgcn_sched_barrier(0);  // keep the refills here
        }
    }
#pragma unroll
    for (int u = 0; u < GS_LA; u += 2) {
        if (full + u + 1 < kn) {
            const f32x4 D0 = dots(u, full + u), D1 = dots(u + 1, full + u + 1);
            epilogue(u, full + u, D0);
            epilogue(u + 1, full + u + 1, D1);
        } else if (full + u < kn) {
            epilogue(u, full + u, dots(u, full + u));
        }
    }

    // the second half's sums join the first's (fixed order); from here on
    // only the first four waves write, but all take part in every barrier
    if (part_k) red[wave - GS_TILES][lane] = acc;
    __syncthreads();
    if (!part_k) acc = acc + red[wave][lane];
    if constexpr (SPLIT) {  // lane j += lane j + M (lanes j >= M are not written)
#pragma unroll
        for (int q = 0; q < 4; q++) acc[q] += __shfl(acc[q], lane + M);
    }
    const bool writer = !part_k && tile_ok;

    // lane (g, j) holds rows 4g..4g+3 of the tile for column j
    const int row = T * TILE_ROWS + 4 * g;
    if (kg == 1) {
        if (writer && j < M)
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (row + q < P.rows) P.y[(size_t)j * P.rows + row + q] = out_val(acc[q], P.bias, P.res, P.rows, j, row + q);
        return;
    }
    // Split K: publish the slice's partials with coherent stores, then the
    // last workgroup of the row group adds the kg slices in slice order
    // (deterministic) and resets the counter. The stores are complete at
    // the device's coherence point once vmcnt drains, before the barrier
    // that precedes the counter increment; the last workgroup reads with
    // coherent loads after it has seen the count.
    const auto prt = buf_rsrc(P.part, kg * 16 * P.rows_pad * 4);
    if (writer) {
        u32x4 v;
        __builtin_memcpy(&v, &acc, 16);
        __builtin_amdgcn_raw_buffer_store_b128(v, prt, ((kgi * 16 + j) * P.rows_pad + row) * 4, 0, CPOL_SC1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(P.counters + rg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (uint32_t)(kg - 1);
    }
    __syncthreads();
    if (!s_last) return;
    if (writer && j < M) {
        // the slices in slice order, GS_KC loads in flight before the adds
        constexpr int GS_KC = 16;
        f32x4 sum = {0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < kg; k0 += GS_KC) {
            u32x4 v[GS_KC];
#pragma unroll
            for (int kk = 0; kk < GS_KC; kk++)
                v[kk] = __builtin_amdgcn_raw_buffer_load_b128(
                    prt, k0 + kk < kg ? (((k0 + kk) * 16 + j) * P.rows_pad + row) * 4 : 0x7FFFFFF0, 0, CPOL_SC1);
#pragma unroll
            for (int kk = 0; kk < GS_KC; kk++)
                if (k0 + kk < kg) {
                    f32x4 f;
                    __builtin_memcpy(&f, &v[kk], 16);
                    sum = k0 + kk == 0 ? f : sum + f;
                }
        }
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (row + q < P.rows) P.y[(size_t)j * P.rows + row + q] = out_val(sum[q], P.bias, P.res, P.rows, j, row + q);
    }
    if (threadIdx.x == 0) __hip_atomic_store(P.counters + rg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- expert-grouped GEMM (prefill) on the int8 matrix cores, with the
// FAST GEMV's representation of x: each 128-value block of an X row is
// x ~= s_b * Q / 2^21, s_b = max|x_b| / 127,
// Q = rint(x * 127 * 2^21 / max|x_b|) = d0*2^21 + d1*2^14 + d2*2^7 + d3
// with int8 digits (d0 = Q >> 21, d1..d3 7-bit fields). The digits of four
// pairs are the first operand of v_mfma_i32_16x16x64_i8 (row 4p + d: digit d
// of pair p) and a 16-row tile's codes, exact in int8, the second: lane
// (g, j) then receives the four digit dots of pair g with weight row j, and
// a block adds
//     scale_j * s_b * 2^-7 ((D0 2^7 + D1) + (D2 2^7 + D3) 2^-14) + zp_j * sum(x_b)
// to the pair's fp32 accumulator for row j (the scale's 2^-7 is folded
// into s_b). The codes need no conversion
// (the bf16 form of this kernel spent 16 byte permutes per tile and block
// turning them into bf16, and 54 vector instructions per 4 matrix-core
// ones in all). A work item is one expert's run of at most 16 pairs (four
// groups of four), so an expert's weights are streamed once for most
// experts of a 256-token prompt (with 8 pairs per item, an expert routed
// ~16 pairs read its matrices twice: ~270 MB per launch where the experts
// hold ~110 MB).
//
// The digits are made once per X row by k_pf_digits, as records of 512 B
// per (row, block) in the order the LDS operand wants them: piece (h, q, d)
// of 16 B holds digit d of the values k = 64 h + q + 4 m of the block, m in
// the byte order of lane group q's 16-byte code word. (Digitising inside
// this kernel, per item and pair, cost ~13 us of every workgroup's start:
// a gate/up pair's token row was digitised once per item that held it.)
//
// Work is split evenly over a fixed grid (one workgroup per CU), not one
// workgroup per item: a unit is (item, matrix, row tile), units are
// numbered item-major, and workgroup b takes units [b U / G, (b + 1) U / G)
// of the U = items x matrices x tiles. A 256-token prompt routes ~165 items
// over 128 experts: with one workgroup per item (its X digits, 128 KiB of
// LDS, allow one per CU) 91 CUs sat idle and every CU that worked ran a
// whole item. A workgroup's range covers one item or the end of one and the
// start of the next (segments): per item it copies the item's digit records
// into LDS once, and its waves stream the segment's units (tile s0 + w,
// s0 + w + GG_NW, ... for wave w) through the full K, GG_LA units of codes in
// flight, in whole unguarded rounds (units past the wave's last read zeros
// and are dropped), writing each finished tile's rows x pairs. Two matrices
// of one shape over the same X (gate and up) share a launch and each
// item's digits.
// Waves: 8 for gate and up, with the step stream software-pipelined (two
// product sets: 184 VGPRs); 16 for a down projection (128 row tiles, 8 per
// wave), not pipelined (128 VGPRs). Per 256-token Qwen3-30B-A3B-shaped
// layer: gate + up 69 us, down 40 us, against 2 x 45.8 and 37.5 with one
// workgroup per item and the digits made inside. Measured and dropped: a
// per-item count of pair groups (1..4, the work split by weight): 83 and
// 51 us, each variant of the step stream carrying the fixed per-step work
// (code unpack, loads) for fewer products.
constexpr int GG_CT = 2;   // tiles per chunk: the units of one step
constexpr int GG_PG = (GEMM_GROUP_COLS + 3) / 4;  // groups of four pairs
struct GemmGroupArgs {
    const uint8_t* codes[2];
    const uint8_t* hp[2];
    const uint32_t* params[2];
    float* y[2];         // [pairs][rows] per matrix
    const uint8_t* dg;   // X digits, [xrows][nb] records of 512 B (launch_pf_digits)
    const float2* dxs;   // [xrows][nb] {s_b 2^-7, sum}
    const int* rowidx;   // X row of pair p (null: row p)
    const int* items;    // [3 * n]: expert, first pair, count
    const int* nitems;
    size_t ecodes, ehp, eparams;
    int rows, rows_pad, nb, xrows, nmat;
};

// X rows to digit records (the grouped GEMM's X, xdigits.h): workgroup
// (row, group of eight blocks), 32 lanes per block with four consecutive
// values each. SILU: X = silu(x) * xu (the FAST steps' arithmetic). The
// digits are staged in LDS and leave as whole 16-byte pieces.
template <bool SILU>
__global__ __launch_bounds__(256) void k_pf_digits(const float* __restrict__ X, const float* __restrict__ XU, int K,
                                                   uint8_t* __restrict__ dg, float2* __restrict__ dxs)
{
    __shared__ __align__(16) uint8_t stage[8][512];
    const int row = blockIdx.x, nb = K / 128, bl = threadIdx.x >> 5, b = blockIdx.y * 8 + bl;
    const int lane = threadIdx.x & 63, k0 = 4 * (lane & 31);
    const bool ok = b < nb;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (ok) {
        const float4 x = *reinterpret_cast<const float4*>(X + (size_t)row * K + b * 128 + k0);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
        if constexpr (SILU) {
            const float4 u = *reinterpret_cast<const float4*>(XU + (size_t)row * K + b * 128 + k0);
            const float uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] = __fdividef(v[q], 1.0f + __expf(-v[q])) * uu[q];
        }
    }
    const float2 sx = digit_block(v, stage[bl]);
    if (ok && (lane & 31) == 0) dxs[(size_t)row * nb + b] = sx;
    __syncthreads();
    // thread t: piece t % 32 of block t / 32 of the group
    if (ok)
        *reinterpret_cast<u32x4*>(dg + ((size_t)row * nb + b) * 512 + (threadIdx.x & 31) * 16) =
            *reinterpret_cast<const u32x4*>(&stage[bl][(threadIdx.x & 31) * 16]);
}

template <int SCHEME, int GG_NW>
__global__ __launch_bounds__(GG_NW * 64) void k_gemm_grouped(const GemmGroupArgs P)
{
    constexpr int GG_WG = GG_NW * 64;
    constexpr bool PIPE = GG_NW == 8;  // two product sets fit in the registers of 8 waves
    constexpr int GG_LA = PIPE ? 8 : 6;  // units (tile, block) of codes in flight per wave
    __shared__ __align__(16) int8_t xd[GEMM_GROUP_MAXBK][GG_PG][2048];       // digits
    __shared__ float2 xs[GEMM_GROUP_MAXBK][GG_PG * 4];                       // {s_b, sum(x_b)}
    const int nb = P.nb;
    const int ntiles = P.rows_pad / TILE_ROWS, nmat = P.nmat;
    const int64_t total = (int64_t)(*P.nitems) * nmat * ntiles;
    // share v of the units, v = (b % 8) * G / 8 + b / 8 for workgroup b:
    // neighbouring shares (an expert's two items, which read the same
    // weights) run on one XCD and meet in its L2
    const int G = (int)gridDim.x, b = (int)blockIdx.x;
    const int v = G % 8 ? b : (b % 8) * (G / 8) + b / 8;
    const int ub0 = (int)(total * v / G), ub1 = (int)(total * (v + 1) / G);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nrec = ntiles * nb;
    const auto drs = buf_rsrc(P.dg, P.xrows * nb * 512);

    // the segments: matrix mt of item it, row tiles [s0, s1) (a
    // workgroup-uniform loop); the X digits are read when the item changes
    int cur = -1;
    for (int sg = ub0 / ntiles; ub0 < ub1 && sg * ntiles < ub1; sg++) {
        // the lane index passes through an empty asm so that nothing derived
        // from it (LDS and buffer offsets) is hoisted out of this loop and
        // held in registers across the step stream (182 VGPRs against 128)
        int lane = (int)threadIdx.x & 63;
        asm volatile("" : "+v"(lane));
        const int g = lane >> 4, j = lane & 15;
        const int s0 = max(ub0 - sg * ntiles, 0), s1 = min(ub1 - sg * ntiles, ntiles);
        const int it = sg / nmat, mt = sg - it * nmat;
        const int e = P.items[3 * it], p0 = P.items[3 * it + 1], M = P.items[3 * it + 2];
        const bool fresh = it != cur;
        if (fresh && cur >= 0) __syncthreads();  // the previous item's digits are no longer read

        // This wave's tiles are s0 + wave, s0 + wave + GG_NW, ...; it takes
        // them GG_CT at a time (a chunk), block by block: step s is block
        // s % nb of chunk s / nb, and its units are the chunk's tiles at that
        // block, so one read of the block's digits serves GG_CT tiles.
        const int my_tiles = s1 - s0 > wave ? (s1 - s0 - wave + GG_NW - 1) / GG_NW : 0;
        const int nsteps = (my_tiles + GG_CT - 1) / GG_CT * nb;
        const auto crs = buf_rsrc(P.codes[mt] + (size_t)e * P.ecodes, nrec * (int)CODE_REC);
        const auto hrs = buf_rsrc(SCHEME == 3 ? P.hp[mt] + (size_t)e * P.ehp : P.codes[mt],
                                  SCHEME == 3 ? nrec * (int)HP_REC : 0);
        const auto prs = buf_rsrc(P.params[mt] + (size_t)e * P.eparams, nrec * TILE_ROWS * 4);
        float* const y = P.y[mt];
        u32x4 cr[GG_LA];
        u32x2 hr[GG_LA];
        uint32_t pr[GG_LA];
        // units are requested in order: the next step's chunk and block are
        // (lc, lb), unit tt of it tile s0 + wave + GG_NW (GG_CT lc + tt); a
        // tile past the wave's last (or a step past the end) reads record
        // nrec, past the range (zeros, never used)
        int lc = 0, lb = 0;
        auto load_step = [&](int slot0) {
#pragma unroll
            for (int tt = 0; tt < GG_CT; tt++) {
                const int tl = GG_CT * lc + tt;
                const int rec = tl < my_tiles ? (s0 + wave + GG_NW * tl) * nb + lb : nrec;
                const int slot = slot0 + tt;
                cr[slot] = __builtin_amdgcn_raw_buffer_load_b128(crs, rec * (int)CODE_REC + lane * 16, 0, CPOL_NT);
                if constexpr (SCHEME == 3)
                    hr[slot] = __builtin_amdgcn_raw_buffer_load_b64(hrs, rec * (int)HP_REC + lane * 8, 0, CPOL_NT);
                pr[slot] = __builtin_amdgcn_raw_buffer_load_b32(prs, (rec * TILE_ROWS + j) * 4, 0, CPOL_NT);
            }
            if (++lb == nb) {
                lb = 0;
                lc++;
            }
        };

        if (!fresh) {  // the digits in LDS are this item's
#pragma unroll
            for (int u = 0; u < GG_LA; u += GG_CT) load_step(u);
        } else {
            // ---- the item's X digits into LDS: record (pair c, block blk) is
            // 32 pieces of 16 B, piece (h, q, d) to xd[blk][c / 4] at
            // h KiB + q * 256 + (4 (c % 4) + d) * 16; slot u of a thread
            // holds pair c = u * GG_WG / 512 + threadIdx.x / 512 (uniform
            // per wave: its X row is read from lane c of one vector load of
            // the item's rows), block (threadIdx.x / 32) % 16, piece
            // threadIdx.x % 32. Pairs past M keep whatever the LDS holds:
            // their products are never stored.
            constexpr int PS = GEMM_GROUP_COLS * GEMM_GROUP_MAXBK * 32 / GG_WG;  // slots per thread
            constexpr int CPS = GG_WG / 512;                                     // pairs per slot
            const int blk = (threadIdx.x >> 5) & 15, pc = threadIdx.x & 31;
            const int c0 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 9);
            // lane l < 16 of every wave: the X row of pair l
            const int vrow = (lane & 15) < M ? (P.rowidx ? P.rowidx[p0 + (lane & 15)] : p0 + (lane & 15)) : 0;
#pragma unroll
            for (int u = 0; u < GG_LA; u += GG_CT) load_step(u);
            u32x4 pv[PS];
#pragma unroll
            for (int u = 0; u < PS; u++) {
                const int c = u * CPS + c0;
                const int r = __builtin_amdgcn_readlane(vrow, c & 15);
                const bool ok = c < M && blk < nb;
                pv[u] = __builtin_amdgcn_raw_buffer_load_b128(drs, ok ? ((r * nb + blk) * 512 + pc * 16) : 0x7FFFFFF0, 0,
                                                              0);
            }
            // {s_b, sum} of (pair t / 16, block t % 16), threads t < 256
            const int sc_ = (threadIdx.x >> 4) & 15, sb_ = threadIdx.x & 15;
            const bool sok = threadIdx.x < 256 && sc_ < M && sb_ < nb;
            const int srow = __builtin_amdgcn_ds_bpermute(4 * sc_, vrow);
            const float2 sv = sok ? P.dxs[(size_t)srow * nb + sb_] : make_float2(0.0f, 0.0f);
            // every slot is written (zeros past M and nb: harmless), so no
            // load is left pending on any path into the step loop
#pragma unroll
            for (int u = 0; u < PS; u++) {
                const int c = u * CPS + c0;
                *reinterpret_cast<u32x4*>(&xd[blk][c >> 2][(pc >> 4) * 1024 + ((pc >> 2) & 3) * 256 +
                                                           (4 * (c & 3) + (pc & 3)) * 16]) = pv[u];
            }
            if (threadIdx.x < 256) xs[sb_][sc_] = sv;
            __syncthreads();
            cur = it;
        }

        // ---- the step stream, whole rounds of GG_LA / GG_CT steps: per step
        // the block's digits (every pair group, both halves) and {s_b, sum}
        // once, then the chunk's GG_CT tiles, GG_PG independent matrix-core
        // chains each, then their epilogues. With 8 waves (PIPE) it is
        // software-pipelined by one step: step s + 1's products are issued
        // before step s's epilogue, interleaved with its vector
        // instructions (D and {s_b, sum} in two sets, by step parity).
        float acc[GG_CT][GG_PG], zacc[GG_CT][GG_PG];
#pragma unroll
        for (int tt = 0; tt < GG_CT; tt++)
#pragma unroll
            for (int q = 0; q < GG_PG; q++) acc[tt][q] = zacc[tt][q] = 0.0f;
        int ub = 0, uc = 0;  // block and chunk of the next step to finish
        int mb = 0;          // block of the next step to multiply
        v4i D[2][GG_CT][GG_PG];
        float2 sx[2][GG_PG];
        auto products = [&](int slot0, int par) {
            v4i A0[GG_PG], A1[GG_PG];
#pragma unroll
            for (int pg = 0; pg < GG_PG; pg++) {
                const int8_t* a = &xd[mb][pg][g * 256 + j * 16];
                A0[pg] = *reinterpret_cast<const v4i*>(a);
                A1[pg] = *reinterpret_cast<const v4i*>(a + 1024);
                sx[par][pg] = xs[mb][pg * 4 + g];
            }
            if (++mb == nb) mb = 0;
#pragma unroll
            for (int tt = 0; tt < GG_CT; tt++) {
                const int slot = slot0 + tt;
                const u32x4 W = cr[slot];
                const uint32_t MK = 0x0F0F0F0Fu;
                v4i lo = {(int)(W.x & MK), (int)(W.y & MK), (int)(W.z & MK), (int)(W.w & MK)};
                v4i hi4 = {(int)((W.x >> 4) & MK), (int)((W.y >> 4) & MK), (int)((W.z >> 4) & MK),
                           (int)((W.w >> 4) & MK)};
                if constexpr (SCHEME == 3) {
                    // top two bits: group g holds AVX lanes g (h.x) and g+4 (h.y)
                    const uint32_t T6 = 0x30303030u, hx = hr[slot].x, hy = hr[slot].y;
                    lo.x |= (int)((hx << 4) & T6); lo.y |= (int)((hx << 2) & T6);
                    lo.z |= (int)((hy << 4) & T6); lo.w |= (int)((hy << 2) & T6);
                    hi4.x |= (int)(hx & T6);       hi4.y |= (int)((hx >> 2) & T6);
                    hi4.z |= (int)(hy & T6);       hi4.w |= (int)((hy >> 2) & T6);
                }
#pragma unroll
                for (int pg = 0; pg < GG_PG; pg++) {
                    D[par][tt][pg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0[pg], lo, v4i{0, 0, 0, 0}, 0, 0, 0);
                    D[par][tt][pg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1[pg], hi4, D[par][tt][pg], 0, 0, 0);
                }
            }
        };
        auto epilogue = [&](int slot0, int par) {
#pragma unroll
            for (int tt = 0; tt < GG_CT; tt++) {
                const uint32_t pp = pr[slot0 + tt];
                const float sc = h2f(pp >> 16), zp = h2f(pp & 0xFFFFu);
#pragma unroll
                for (int pg = 0; pg < GG_PG; pg++) {
                    // D0 2^7 + D1 and D2 2^7 + D3 are exact in int32 (|D| < 2^21),
                    // so the digit sum is two conversions and one fma
                    const v4i& d = D[par][tt][pg];
                    const float dh = (float)(d.x * 128 + d.y), dl = (float)(d.z * 128 + d.w);
                    const float cd = fmaf(dl, 0x1p-14f, dh);
                    acc[tt][pg] = __builtin_fmaf(cd * sx[par][pg].x, sc, acc[tt][pg]);
                    zacc[tt][pg] = __builtin_fmaf(zp, sx[par][pg].y, zacc[tt][pg]);
                }
            }
            // the next step's products, one matrix-core instruction between
            // every six vector ones (the code unpack and this epilogue)
            if constexpr (PIPE) {
#pragma unroll
                for (int i = 0; i < 2 * GG_CT * GG_PG; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
                }
            }
            if (++ub == nb) {  // the chunk is complete: lane (g, j) has pair pg*4 + g, row j of each tile
#pragma unroll
                for (int tt = 0; tt < GG_CT; tt++) {
                    const int tl = GG_CT * uc + tt;
                    const int row = (s0 + wave + GG_NW * tl) * TILE_ROWS + j;
                    if (tl < my_tiles && row < P.rows) {
#pragma unroll
                        for (int pg = 0; pg < GG_PG; pg++)
                            if (pg * 4 + g < M) y[(size_t)(p0 + pg * 4 + g) * P.rows + row] = acc[tt][pg] + zacc[tt][pg];
                    }
#pragma unroll
                    for (int pg = 0; pg < GG_PG; pg++) acc[tt][pg] = zacc[tt][pg] = 0.0f;
                }
                ub = 0;
                uc++;
            }
        };
        constexpr int SPR = GG_LA / GG_CT;  // steps per round (even when pipelined: step k's set is k & 1)
        static_assert(!PIPE || SPR % 2 == 0, "step parity must be static");
        const int nst = (nsteps + SPR - 1) / SPR * SPR;  // whole rounds
        if constexpr (PIPE) {
            if (nst > 0) products(0, 0);
            for (int st = 0; st < nst; st += SPR) {
#pragma unroll
                for (int k = 0; k < SPR; k++) {
                    // (past the last step: products of zeros, never used)
                    products(((k + 1) % SPR) * GG_CT, (k + 1) & 1);
                    epilogue(k * GG_CT, k & 1);
                    load_step(k * GG_CT);
                }
            }
        } else {
            for (int st = 0; st < nst; st += SPR) {
#pragma unroll
                for (int k = 0; k < SPR; k++) {
                    products(k * GG_CT, 0);
                    epilogue(k * GG_CT, 0);
                    load_step(k * GG_CT);
                }
            }
        }
    }
}

template <int SCHEME, bool SPLIT>
hipError_t launch_nt(int nt, dim3 grid, hipStream_t s, const GemmArgs& a)
{
    if constexpr (SPLIT) {
        if (nt == 2) hipLaunchKernelGGL((k_gemm<SCHEME, 2, true>), grid, dim3(GM_WG), 0, s, a);
        else hipLaunchKernelGGL((k_gemm<SCHEME, 4, true>), grid, dim3(GM_WG), 0, s, a);
    } else {
        switch (nt) {
        case 2: hipLaunchKernelGGL((k_gemm<SCHEME, 2, false>), grid, dim3(GM_WG), 0, s, a); break;
        case 3: hipLaunchKernelGGL((k_gemm<SCHEME, 3, false>), grid, dim3(GM_WG), 0, s, a); break;
        default: hipLaunchKernelGGL((k_gemm<SCHEME, 4, false>), grid, dim3(GM_WG), 0, s, a); break;
        }
    }
    return hipGetLastError();
}

template <int SCHEME>
void launch_small(int x_mode, dim3 grid, hipStream_t s, const GemmSmallArgs& a)
{
    if (x_mode == GX_BF16) hipLaunchKernelGGL((k_gemm_small<SCHEME, true, false>), grid, dim3(GS_WG), 0, s, a);
    else if (x_mode == GX_SPLIT) hipLaunchKernelGGL((k_gemm_small<SCHEME, false, true>), grid, dim3(GS_WG), 0, s, a);
    else hipLaunchKernelGGL((k_gemm_small<SCHEME, false, false>), grid, dim3(GS_WG), 0, s, a);
}

}  // namespace

int gemm_row_groups(uint64_t rows)
{
    const uint64_t tiles = pad_rows(rows) / TILE_ROWS;
    const uint64_t per = (uint64_t)GM_WG / 64 * GM_RT;
    return (int)((tiles + per - 1) / per);
}

int gemm_small_row_groups(uint64_t rows)
{
    const uint64_t tiles = pad_rows(rows) / TILE_ROWS;
    return (int)((tiles + GS_TILES - 1) / GS_TILES);
}

int gemm_kslices(uint64_t rows, uint64_t nb, int req)
{
    if (nb == 0) return 1;
    if (req > 0) return fast_normalize_kslices(nb, (int)std::min<uint64_t>((uint64_t)req, nb));
    // Enough workgroups for two per CU, but K-slices of at least 15 blocks:
    // each slice's partial Y (64 x rows floats) costs a write and a read
    // (measured on 3840 x 15360: 8 slices 38 us, 10 slices 50 us at M = 64).
    const uint64_t rgs = (uint64_t)gemm_row_groups(rows);
    uint64_t kg = (512 + rgs - 1) / rgs;
    kg = std::min<uint64_t>(kg, std::max<uint64_t>(1, nb / 15));
    return fast_normalize_kslices(nb, (int)std::max<uint64_t>(kg, 1));
}

int gemm_small_kslices(uint64_t rows, uint64_t nb, int req)
{
    if (nb == 0) return 1;
    const int kmin = (int)((nb + GEMM_SMALL_MAXBK - 1) / GEMM_SMALL_MAXBK);
    int kg = req;
    if (kg <= 0) {  // about one workgroup per CU, slices of at least 4 blocks
        const uint64_t rgs = (uint64_t)gemm_small_row_groups(rows);
        kg = (int)std::min<uint64_t>((240 + rgs - 1) / rgs, std::max<uint64_t>(1, nb / 4));
    }
    kg = (int)std::min<uint64_t>((uint64_t)std::max(kg, kmin), nb);
    // normalising can only lower the count, so recheck the slice length
    int k = fast_normalize_kslices(nb, kg);
    while ((nb + k - 1) / k > (uint64_t)GEMM_SMALL_MAXBK) k = fast_normalize_kslices(nb, ++kg);
    return k;
}

hipError_t launch_gemm(const DeviceMatrix& m, const GemmWork& w, const void* x, int x_mode, int M,
                       const float* bias, const float* res, float* y, hipStream_t s)
{
    const bool split = x_mode == GX_SPLIT;
    if (M < 1 || M > (split ? GEMM_MAX_M_SPLIT : GEMM_MAX_M) || m.nb == 0) return hipErrorInvalidValue;
    const int cols = split ? 2 * M : M;  // fragment columns
    const int NT = (cols + 15) / 16;
    const int nb = (int)m.nb;
    (void)hipGetLastError();  // report only these launches
    if (cols <= 16) {
        if ((nb + w.kg_small - 1) / w.kg_small > GEMM_SMALL_MAXBK)
            return hipErrorInvalidValue;  // the planner never makes such a split
        GemmSmallArgs a{};
        a.codes = m.codes;
        a.hp = m.hp;
        a.params = m.params;
        a.x = x;
        a.y = y;
        a.bias = bias;
        a.res = res;
        a.part = w.part;
        a.counters = w.counters;
        a.rows = (int)m.rows;
        a.rows_pad = (int)m.rows_pad;
        a.nb = nb;
        a.M = M;
        a.kg = w.kg_small;
        dim3 grid((unsigned)(gemm_small_row_groups(m.rows) * w.kg_small));
        if (m.scheme == 4) launch_small<4>(x_mode, grid, s, a);
        else launch_small<3>(x_mode, grid, s, a);
        return hipGetLastError();
    }
    // SPLIT: hi tiles then as many lo tiles (NT even)
    const int ntiles = split ? 2 * ((M + 15) / 16) : NT;
    dim3 pgrid((unsigned)(nb * ntiles));
    if (x_mode == GX_BF16)
        hipLaunchKernelGGL((k_gemm_pack<true, false>), pgrid, dim3(256), 0, s, x, M, (int)m.cols, ntiles, ntiles,
                           reinterpret_cast<u32x4*>(w.xf), w.xsum);
    else if (split)
        hipLaunchKernelGGL((k_gemm_pack<false, true>), pgrid, dim3(256), 0, s, x, M, (int)m.cols, ntiles, ntiles,
                           reinterpret_cast<u32x4*>(w.xf), w.xsum);
    else
        hipLaunchKernelGGL((k_gemm_pack<false, false>), pgrid, dim3(256), 0, s, x, M, (int)m.cols, ntiles, ntiles,
                           reinterpret_cast<u32x4*>(w.xf), w.xsum);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    GemmArgs a{};
    a.codes = m.codes;
    a.hp = m.hp;
    a.params = m.params;
    a.xf = reinterpret_cast<const u32x4*>(w.xf);
    a.xsum = w.xsum;
    a.y = y;
    a.bias = bias;
    a.res = res;
    a.part = w.part;
    a.rows = (int)m.rows;
    a.rows_pad = (int)m.rows_pad;
    a.nb = nb;
    a.M = M;
    a.kg = w.kg;
    a.xt = ntiles;
    dim3 grid((unsigned)(gemm_row_groups(m.rows) * w.kg));
    if (split) e = m.scheme == 4 ? launch_nt<4, true>(ntiles, grid, s, a) : launch_nt<3, true>(ntiles, grid, s, a);
    else e = m.scheme == 4 ? launch_nt<4, false>(ntiles, grid, s, a) : launch_nt<3, false>(ntiles, grid, s, a);
    if (e != hipSuccess || w.kg == 1) return e;
    const int outs = M * (int)(m.rows_pad / 4);
    hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, s, w.part, w.kg,
                       ntiles * 16, (int)m.rows_pad, (int)m.rows, M, bias, res, y);
    return hipGetLastError();
}

hipError_t launch_gemm_pack_rows(const float* x, int M, int K, void* xf, float* xsum, hipStream_t s)
{
    if (M < 1 || K % 128) return hipErrorInvalidValue;
    const int xt = gemm_rows_tiles(M);
    (void)hipGetLastError();
    hipLaunchKernelGGL((k_gemm_pack<false, true>), dim3((unsigned)(K / 128 * xt)), dim3(256), 0, s, x, M, K, xt, 4,
                       reinterpret_cast<u32x4*>(xf), xsum);
    return hipGetLastError();
}

hipError_t launch_gemm_packed_rows(const DeviceMatrix& m, const void* xf, const float* xsum, int M, const float* bias,
                                   const float* res, float* y, hipStream_t s, int kg, float* part, bool reduce)
{
    if (M < 1 || m.nb == 0 || kg < 1 || kg > (int)m.nb || (kg > 1 && !part)) return hipErrorInvalidValue;
    (void)hipGetLastError();
    GemmArgs a{};
    a.codes = m.codes;
    a.hp = m.hp;
    a.params = m.params;
    a.xf = static_cast<const u32x4*>(xf);
    a.xsum = xsum;
    a.y = y;
    a.bias = bias;
    a.res = res;
    a.rows = (int)m.rows;
    a.rows_pad = (int)m.rows_pad;
    a.nb = (int)m.nb;
    a.M = M;
    a.kg = kg;
    a.part = part;
    a.xt = gemm_rows_tiles(M);
    a.rgs = gemm_row_groups(m.rows);
    a.rgs8 = (a.rgs + 7) / 8 * 8;
    dim3 grid((unsigned)(a.rgs8 * (a.xt / 4) * kg));
    hipError_t e = m.scheme == 4 ? launch_nt<4, true>(4, grid, s, a) : launch_nt<3, true>(4, grid, s, a);
    if (e != hipSuccess || kg == 1 || !reduce) return e;
    const int Mp = a.xt / 4 * 32, outs = M * (int)(m.rows_pad / 4);
    hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, s, part, kg, Mp,
                       (int)m.rows_pad, (int)m.rows, M, bias, res, y);
    return hipGetLastError();
}

hipError_t launch_gemm_packed_rows_multi(const DeviceMatrix* const* ms, const float* const* biases, float* const* ys,
                                         int count, const void* xf, const float* xsum, int M, hipStream_t s,
                                         const GemmRope* rope)
{
    if (M < 1 || count < 1 || count > GEMM_MAX_MATS) return hipErrorInvalidValue;
    for (int e = 0; e < count; e++)
        if (ms[e]->nb == 0 || ms[e]->nb != ms[0]->nb || ms[e]->scheme != ms[0]->scheme) return hipErrorInvalidValue;
    if (rope) {  // whole 128-row heads; q and k have norm weights, k and v a cache
        if (!rope->cos_t || !rope->sin_t || rope->pos0 < 0 || rope->pos0 + M > rope->max_pos)
            return hipErrorInvalidValue;
        for (int e = 0; e < count; e++) {
            const int md = rope->mode[e];
            if (md < 0 || md > GEMM_ROPE_V || (md && ms[e]->rows % 128) || (md && md != GEMM_ROPE_V && !rope->nw[e]) ||
                ((md == GEMM_ROPE_K || md == GEMM_ROPE_V) && !rope->cache[e]))
                return hipErrorInvalidValue;
        }
    }
    (void)hipGetLastError();
    const DeviceMatrix& m = *ms[0];
    GemmArgs a{};
    a.codes = m.codes;
    a.hp = m.hp;
    a.params = m.params;
    a.xf = static_cast<const u32x4*>(xf);
    a.xsum = xsum;
    a.y = ys[0];
    a.bias = biases[0];
    if (rope) {
        a.rope = rope->mode[0];
        a.cache = rope->cache[0];
        a.nw = rope->nw[0];
        a.cos_t = rope->cos_t;
        a.sin_t = rope->sin_t;
        a.pos0 = rope->pos0;
        a.max_pos = rope->max_pos;
        a.eps = rope->eps;
    }
    a.rows = (int)m.rows;
    a.rows_pad = (int)m.rows_pad;
    a.nb = (int)m.nb;
    a.M = M;
    a.kg = 1;
    a.xt = gemm_rows_tiles(M);
    a.rgs = gemm_row_groups(m.rows);
    a.rgs8 = (a.rgs + 7) / 8 * 8;
    int wgs = a.rgs8 * (a.xt / 4);
    a.nmore = count - 1;
    for (int e = 1; e < count; e++) {
        GemmMat& mm = a.more[e - 1];
        mm.codes = ms[e]->codes;
        mm.hp = ms[e]->hp;
        mm.params = ms[e]->params;
        mm.y = ys[e];
        mm.bias = biases[e];
        mm.rows = (int)ms[e]->rows;
        mm.rows_pad = (int)ms[e]->rows_pad;
        mm.rgs = gemm_row_groups(ms[e]->rows);
        mm.rgs8 = (mm.rgs + 7) / 8 * 8;
        mm.wg0 = wgs;
        if (rope) {
            mm.rope = rope->mode[e];
            mm.cache = rope->cache[e];
            mm.nw = rope->nw[e];
        }
        wgs += mm.rgs8 * (a.xt / 4);
    }
    const dim3 grid((unsigned)wgs);
    return m.scheme == 4 ? launch_nt<4, true>(4, grid, s, a) : launch_nt<3, true>(4, grid, s, a);
}

hipError_t launch_pf_digits(const float* x, const float* xu, int rows, int K, void* dg, float* dxs, hipStream_t s)
{
    if (rows < 1 || K < 128 || K % 128) return hipErrorInvalidValue;
    (void)hipGetLastError();
    const dim3 grid((unsigned)rows, (unsigned)((K / 128 + 7) / 8));
    if (xu)
        hipLaunchKernelGGL(k_pf_digits<true>, grid, dim3(256), 0, s, x, xu, K, static_cast<uint8_t*>(dg),
                           reinterpret_cast<float2*>(dxs));
    else
        hipLaunchKernelGGL(k_pf_digits<false>, grid, dim3(256), 0, s, x, xu, K, static_cast<uint8_t*>(dg),
                           reinterpret_cast<float2*>(dxs));
    return hipGetLastError();
}

hipError_t launch_gemm_grouped(const DeviceMatrix& m, const DeviceMatrix* m2, const void* dg, const float* dxs,
                               int xrows, const int* rowidx, const int* items, const int* nitems, int wgs, float* y,
                               float* y2, hipStream_t s)
{
    if (m.nb == 0 || m.nb > (uint64_t)GEMM_GROUP_MAXBK || m.rows_pad > (uint64_t)GEMM_GROUP_MAXROWS || xrows < 1 ||
        (uint64_t)xrows * m.nb * 512 > 0x7FFFFFF0ull || wgs < 1 || !y || (m2 != nullptr) != (y2 != nullptr))
        return hipErrorInvalidValue;
    if (m2 && (m2->scheme != m.scheme || m2->rows != m.rows || m2->rows_pad != m.rows_pad || m2->nb != m.nb))
        return hipErrorInvalidValue;
    (void)hipGetLastError();
    GemmGroupArgs a{};
    const DeviceMatrix* ms[2] = {&m, m2 ? m2 : &m};
    for (int i = 0; i < 2; i++) {
        a.codes[i] = ms[i]->codes;
        a.hp[i] = ms[i]->hp;
        a.params[i] = ms[i]->params;
    }
    a.y[0] = y;
    a.y[1] = m2 ? y2 : y;
    a.dg = static_cast<const uint8_t*>(dg);
    a.dxs = reinterpret_cast<const float2*>(dxs);
    a.rowidx = rowidx;
    a.items = items;
    a.nitems = nitems;
    const size_t tiles = m.rows_pad / TILE_ROWS;
    a.ecodes = tiles * m.nb * CODE_REC;
    a.ehp = m.scheme == 3 ? tiles * m.nb * HP_REC : 0;
    a.eparams = tiles * m.nb * TILE_ROWS;
    a.rows = (int)m.rows;
    a.rows_pad = (int)m.rows_pad;
    a.nb = (int)m.nb;
    a.xrows = xrows;
    a.nmat = m2 ? 2 : 1;
    const dim3 grid((unsigned)wgs);
    // 16 waves for one matrix of 128+ row tiles (a down projection), else 8
    if (!m2 && tiles >= 128) {
        if (m.scheme == 4) hipLaunchKernelGGL((k_gemm_grouped<4, 16>), grid, dim3(1024), 0, s, a);
        else hipLaunchKernelGGL((k_gemm_grouped<3, 16>), grid, dim3(1024), 0, s, a);
    } else {
        if (m.scheme == 4) hipLaunchKernelGGL((k_gemm_grouped<4, 8>), grid, dim3(512), 0, s, a);
        else hipLaunchKernelGGL((k_gemm_grouped<3, 8>), grid, dim3(512), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace wpcg
