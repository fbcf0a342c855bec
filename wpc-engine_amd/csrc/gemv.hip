// Dequant-GEMV kernels for gfx950 (CDNA4, wave64) over WPC blocks of 128
// weights (v4: 4-bit codes, v3: 6-bit codes in two planes). Device layout:
// see wpcg_internal.hpp (paired-lane code bytes, 16-row tile-major params).
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
// and Q = d0*2^21 + d1*2^14 + d2*2^7 + d3 with int8 digits d0 in [-127,127],
// d1..d3 in [-64,64]. v_mfma_i32_16x16x64_i8 then gives the exact integer
// dots D_j = sum(code * d_j) for the four digit columns of a 16-row tile,
// and each block adds
//   scale * s_b * (D0 + D1*2^-7 + D2*2^-14 + D3*2^-21) + zp * sum(x_b)
// to fp32 accumulators (the zp term rides on the idle fifth column). The
// only approximation is x's representation: the fp32 product x*127*2^21/m
// (relative 6e-8, as fp32 itself) plus 0.5*s_b*2^-21 = 1.9e-9 * max|x_b|,
// which keeps the small values of a block that holds an outlier accurate.
#include <hip/hip_runtime.h>

#include "wpcg_internal.hpp"

namespace wpcg {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int dcode_off(int L, int g) { return (L & 3) * 16 + (L >> 2) * 8 + g; }
__device__ __forceinline__ int dhp_off(int L, int m) { return (L & 3) * 8 + (L >> 2) * 4 + m; }
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

// ============================================================ EXACT mode
constexpr int XS_LANE = 20;  // floats per AVX lane in LDS (bank spread)
constexpr int XS_BLK = 8 * XS_LANE;
constexpr int EX_SEG = 32;   // blocks of x per LDS pass (20 KiB)
constexpr int EX_WG = 128;   // 16 rows x 8 lanes

// x staged as xs[s*XS_BLK + L*XS_LANE + G] = x[(b0+s)*128 + G*8 + L]: the 16
// activations AVX lane L uses, in the order it uses them.
__device__ __forceinline__ void stage_x(float* xs, const float* __restrict__ x, int b0, int nbs)
{
    for (int i = threadIdx.x; i < nbs * 128; i += EX_WG) {
        int s = i >> 7, r = i & 127;
        xs[s * XS_BLK + (r & 7) * XS_LANE + (r >> 3)] = x[(size_t)b0 * 128 + i];
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

// AVX2 lane L of matvec_v4_fused over one block: for g in 0..8, the low
// nibble of ref byte g*8+L (activation G = g), then its high nibble (G = 8+g).
__device__ __forceinline__ float v4_exact_block(uint2 c, uint32_t p, const float* xl, float acc)
{
    const float zp = h2f(p & 0xFFFFu), sc = h2f(p >> 16);
    float xv[16];
    load16(xl, xv);
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

// AVX2 lane L of matvec_v3_fused over one block: codes k = G*8+L for G in
// 0..16, natural order. Low 4 bits: low-plane byte G (G < 8, low nibble) or
// G-8 (high nibble); top 2 bits: high-plane byte G&3, bits 2*(G>>2).
__device__ __forceinline__ float v3_exact_block(uint2 c, uint32_t h, uint32_t p, const float* xl,
                                                float acc)
{
    const float zp = h2f(p & 0xFFFFu), sc = h2f(p >> 16);
    float xv[16];
    load16(xl, xv);
#pragma unroll
    for (int G = 0; G < 16; G++) {
        const int gb = G & 7;
        const uint32_t w = gb < 4 ? c.x : c.y;
        const uint32_t byte = (w >> (8 * (gb & 3))) & 0xFFu;
        const uint32_t nib = G < 8 ? (byte & 15u) : (byte >> 4);
        const uint32_t top = (h >> (8 * (G & 3) + 2 * (G >> 2))) & 3u;
        const float code = (float)(nib | (top << 4));
        acc = __builtin_fmaf(__builtin_fmaf(code, sc, zp), xv[G], acc);
    }
    return acc;
}

template <int SCHEME>
__global__ __launch_bounds__(EX_WG) void k_gemv_exact(const uint8_t* __restrict__ codes,
                                                      const uint8_t* __restrict__ hp,
                                                      const uint32_t* __restrict__ params,
                                                      const float* __restrict__ x,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, int rows, int nb)
{
    __shared__ __align__(16) float xs[EX_SEG * XS_BLK];
    const int L = threadIdx.x & 7;
    const int row = blockIdx.x * (EX_WG / 8) + (threadIdx.x >> 3);
    const bool active = row < rows;
    const size_t rb = (size_t)row * (size_t)nb;  // rows are padded: in range
    const uint32_t* pp = params + (size_t)blockIdx.x * nb * TILE_ROWS + (row & (TILE_ROWS - 1));
    float acc = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += EX_SEG) {
        const int nbs = min(EX_SEG, nb - b0);
        __syncthreads();
        stage_x(xs, x, b0, nbs);
        __syncthreads();
        const uint8_t* cp = codes + (rb + b0) * 64 + dcode_off(L, 0);
        const float* xl = xs + L * XS_LANE;
        if constexpr (SCHEME == 4) {
#pragma unroll 4
            for (int s = 0; s < nbs; s++) {
                const uint2 c = *reinterpret_cast<const uint2*>(cp + (size_t)s * 64);
                acc = v4_exact_block(c, pp[(size_t)(b0 + s) * TILE_ROWS], xl + s * XS_BLK, acc);
            }
        } else {
            const uint8_t* hq = hp + (rb + b0) * 32 + dhp_off(L, 0);
#pragma unroll 4
            for (int s = 0; s < nbs; s++) {
                const uint2 c = *reinterpret_cast<const uint2*>(cp + (size_t)s * 64);
                const uint32_t h = *reinterpret_cast<const uint32_t*>(hq + (size_t)s * 32);
                acc = v3_exact_block(c, h, pp[(size_t)(b0 + s) * TILE_ROWS], xl + s * XS_BLK, acc);
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

// ============================================================ FAST mode
struct FastProblem {
    const uint8_t* codes;
    const uint8_t* hp;
    const uint32_t* params;
    const float* x;
    float* y;
    const float* bias;
    float* part;
    uint32_t* counters;
    int rows, rows_pad, nb, kg, wg_begin, pad_;
};
struct FastBatch {
    FastProblem p[MAX_JOBS];
    int n;
};

constexpr int FAST_WG = 256;  // 4 waves: FAST_TILES tiles x KS K-interleaved waves
constexpr int MAXBK = FAST_MAXBK;  // blocks per K-slice (LDS digits: 16 KiB)
constexpr int NDIG = 4;       // int8 digits per x value
constexpr int HALF = 4 * NDIG * 16;  // fragment bytes per MFMA half: 4 groups x digits x 16
constexpr int FRAG = 2 * HALF;       // per block

// Byte position of digit 0 of x index k (0..127) in a block's fragment area.
// MFMA half h = k>>6 covers 64 k; lane group g = k&3; byte (k>>3)&7 + 8*((k>>2)&1).
// This is the inverse of the A-operand packing below, in which lane group g
// holds AVX lanes g and g+4 of a block (16 packed bytes). Digit j of the same
// value sits 16*j bytes further.
__device__ __forceinline__ int frag_pos(int k)
{
    return (k >> 6) * HALF + (k & 3) * (NDIG * 16) + ((k >> 3) & 7) + 8 * ((k >> 2) & 1);
}

// Q = d0*2^21 + d1*2^14 + d2*2^7 + d3 with |Q| <= 127*2^21 (+ rounding):
// d0 = floor((Q + 2^20) / 2^21) in [-127, 127], the rest in [-64, 64].
__device__ __forceinline__ void put_digits(int8_t* blk, int k, float v, float inv)
{
    const int Q = (int)rintf(v * inv);
    const int d0 = (Q + (1 << 20)) >> 21;
    const int r1 = Q - (d0 << 21);
    const int d1 = (r1 + (1 << 13)) >> 14;
    const int r2 = r1 - (d1 << 14);
    const int d2 = (r2 + 64) >> 7;
    const int d3 = r2 - (d2 << 7);
    int8_t* p = blk + frag_pos(k);
    p[0] = (int8_t)d0;
    p[16] = (int8_t)d1;
    p[32] = (int8_t)d2;
    p[48] = (int8_t)d3;
}

// One row of the block epilogue, branch-free: the digit dot d (lanes of
// columns 0..3) scaled by scale*s_b, and the zero-point term zp*sum(x_b)
// (kept by every lane, used from column 4).
__device__ __forceinline__ void fast_step(float& acc, float& zacc, int d, uint32_t p, float sb, float Sb)
{
    acc = __builtin_fmaf((float)d, h2f(p >> 16) * sb, acc);
    zacc = __builtin_fmaf(h2f(p & 0xFFFFu), Sb, zacc);
}

template <int SCHEME>
__global__ __launch_bounds__(FAST_WG) void k_gemv_fast(const FastBatch B)
{
    constexpr int KS = 4 / FAST_TILES;
    __shared__ __align__(16) int8_t xq[MAXBK * FRAG];
    __shared__ float xsc[MAXBK], xsum[MAXBK];
    __shared__ float red[4][TILE_ROWS];
    __shared__ __align__(16) uint32_t spar[FAST_TILES * MAXBK * TILE_ROWS];
    __shared__ int s_last;
    static_assert(FAST_TILES * MAXBK * 4 == FAST_WG, "one parameter chunk per thread");

    const int wgid = blockIdx.x;
    int pi = 0;
#pragma unroll
    for (int i = 1; i < MAX_JOBS; i++)
        if (i < B.n && wgid >= B.p[i].wg_begin) pi = i;
    const FastProblem& P = B.p[pi];
    const int nb = P.nb, kg = P.kg;
    const int local = wgid - P.wg_begin;
    const int kgi = local % kg, tg = local / kg;
    const int nbk = (nb + kg - 1) / kg;
    const int b0 = kgi * nbk;
    const int nbl = max(0, min(nb, b0 + nbk) - b0);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int ti = wave / KS, kw = wave % KS;  // this wave's tile and K interleave
    const int T = tg * FAST_TILES + ti;
    const int ntiles = P.rows_pad / TILE_ROWS;
    const int r = lane & 15, g = lane >> 4, j = lane & 15;
    // An empty slice (possible only for a caller-side split; the host never
    // makes one) still issues the clamped prologue loads: keep them in range.
    const int bb = min(b0, nb - 1);
    const int last = max(nbl - 1, 0);

    // Prologue. Vector-memory loads complete in issue order, so they go out
    // as: x (for the digit prep; L2-resident), block parameters (to LDS),
    // then this wave's first PF blocks of weights (HBM). The prep waits only
    // for the first two while the weights are still in flight. All loads are
    // unconditional with clamped indices (a clamped duplicate is not used),
    // which keeps the compiler's wait counts exact.
    constexpr int XB = MAXBK / 4;  // prep blocks per wave
    float xv0[XB], xv1[XB];
#pragma unroll
    for (int k = 0; k < XB; k++) {
        const float* xb = P.x + (size_t)(bb + min(wave + 4 * k, last)) * 128;
        xv0[k] = xb[lane];
        xv1[k] = xb[lane + 64];
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order described above
    // parameters of the workgroup's tiles: chunk (tt, bl, q) of 16 bytes
    // holds rows 4q..4q+3 of tile tt, block bl
    const int pchunk = threadIdx.x;  // FAST_TILES * MAXBK * 4 == FAST_WG
    const int pq = pchunk & 3, pbl = (pchunk >> 2) % MAXBK, ptt = (pchunk >> 2) / MAXBK;
    const uint4 pv = *reinterpret_cast<const uint4*>(
        P.params + ((size_t)min(tg * FAST_TILES + ptt, ntiles - 1) * nb + bb + min(pbl, last)) *
                       TILE_ROWS + 4 * pq);
    __builtin_amdgcn_sched_barrier(0);
    const size_t row = (size_t)min(T, ntiles - 1) * TILE_ROWS + r;
    const uint8_t* cp = P.codes + (row * nb + bb) * 64 + g * 16;
    const uint8_t* hq = P.hp + (row * nb + bb) * 32 + g * 8;
    constexpr int PF = 8;  // blocks of weights in flight per wave
    u32x4 c[PF];
    u32x2 h[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) {
        const int bl = min(kw + KS * i, last);
        c[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(cp + (size_t)bl * 64));
        if constexpr (SCHEME == 3)
            h[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(hq + (size_t)bl * 32));
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- x -> int8 digit fragments for blocks [b0, b0+nbl), one wave per block
#pragma unroll
    for (int k = 0; k < XB; k++) {
        const int bl = wave + 4 * k;
        if (bl >= nbl) break;
        const float v0 = xv0[k], v1 = xv1[k];
        float m = fmaxf(fabsf(v0), fabsf(v1));
        float s = v0 + v1;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            m = fmaxf(m, __shfl_xor(m, o));
            s += __shfl_xor(s, o);
        }
        const float inv = m > 0.0f ? (127.0f * 2097152.0f) / m : 0.0f;
        int8_t* dst = xq + bl * FRAG;
        put_digits(dst, lane, v0, inv);
        put_digits(dst, lane + 64, v1, inv);
        if (lane == 0) {
            xsc[bl] = m / 127.0f;
            xsum[bl] = s;
        }
    }
    if (pbl < nbl) *reinterpret_cast<uint4*>(spar + ((ptt * MAXBK + pbl) * TILE_ROWS + 4 * pq)) = pv;
    __syncthreads();

    // ---- matrix-core phase: wave -> (tile, K-interleave)
    const bool zcol = j == NDIG;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    float z0 = 0.f, z1 = 0.f, z2 = 0.f, z3 = 0.f;
    if (T < ntiles) {
        const int8_t* xf = xq + g * (NDIG * 16) + j * 16;
        const uint32_t* sp = spar + ti * MAXBK * TILE_ROWS + 4 * g;
        const uint32_t M = 0x0F0F0F0Fu;
        const int nw = (nbl - kw + KS - 1) / KS;  // blocks of this wave
        for (int i0 = 0; i0 < nw; i0 += PF) {
            if (i0 > 0) {
#pragma unroll
                for (int i = 0; i < PF; i++) {
                    const int bl = min(kw + KS * (i0 + i), last);
                    c[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(cp + (size_t)bl * 64));
                    if constexpr (SCHEME == 3)
                        h[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(hq + (size_t)bl * 32));
                }
            }
#pragma unroll
            for (int i = 0; i < PF; i++) {
                if (i0 + i >= nw) break;
                const int bl = kw + KS * (i0 + i);
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
                v4i B0 = {0, 0, 0, 0}, B1 = {0, 0, 0, 0};
                if (j < NDIG) {
                    B0 = *reinterpret_cast<const v4i*>(xf + bl * FRAG);
                    B1 = *reinterpret_cast<const v4i*>(xf + bl * FRAG + HALF);
                }
                v4i d = {0, 0, 0, 0};
                d = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, d, 0, 0, 0);
                const uint4 pr = *reinterpret_cast<const uint4*>(sp + bl * TILE_ROWS);
                const float sb = xsc[bl], Sb = xsum[bl];
                fast_step(a0, z0, d.x, pr.x, sb, Sb);
                fast_step(a1, z1, d.y, pr.y, sb, Sb);
                fast_step(a2, z2, d.z, pr.z, sb, Sb);
                fast_step(a3, z3, d.w, pr.w, sb, Sb);
            }
        }
    }
    // digit weights 2^(-7j), then sum columns 0..7 (columns 5..7 hold zeros;
    // rows 4g..4g+3 live in lanes 16g..16g+7)
    const float wj = j < NDIG ? __builtin_ldexpf(1.0f, -7 * j) : 1.0f;
    a0 *= wj; a1 *= wj; a2 *= wj; a3 *= wj;
    if (zcol) { a0 = z0; a1 = z1; a2 = z2; a3 = z3; }
    a0 += __shfl_xor(a0, 1); a1 += __shfl_xor(a1, 1); a2 += __shfl_xor(a2, 1); a3 += __shfl_xor(a3, 1);
    a0 += __shfl_xor(a0, 2); a1 += __shfl_xor(a1, 2); a2 += __shfl_xor(a2, 2); a3 += __shfl_xor(a3, 2);
    a0 += __shfl_xor(a0, 4); a1 += __shfl_xor(a1, 4); a2 += __shfl_xor(a2, 4); a3 += __shfl_xor(a3, 4);
    if (j == 0) {
        red[wave][4 * g + 0] = a0;
        red[wave][4 * g + 1] = a1;
        red[wave][4 * g + 2] = a2;
        red[wave][4 * g + 3] = a3;
    }
    __syncthreads();

    const int t = threadIdx.x;
    const int tt = t >> 4, rr = t & 15;
    const int TT = tg * FAST_TILES + tt;
    const size_t orow = (size_t)TT * TILE_ROWS + rr;
    const bool mine = t < FAST_TILES * TILE_ROWS && TT < ntiles;
    float sum = 0.f;
    if (mine) {
        sum = red[tt * KS][rr];
#pragma unroll
        for (int k = 1; k < KS; k++) sum += red[tt * KS + k][rr];
    }
    if (kg == 1) {
        if (mine && orow < (size_t)P.rows) P.y[orow] = P.bias ? sum + P.bias[orow] : sum;
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
    if (mine && orow < (size_t)P.rows) {
        float acc = __hip_atomic_load(P.part + orow, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int k = 1; k < kg; k++)
            acc += __hip_atomic_load(P.part + (size_t)k * P.rows_pad + orow, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        P.y[orow] = P.bias ? acc + P.bias[orow] : acc;
    }
    if (t == 0) __hip_atomic_store(P.counters + tg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ============================================================ decode helpers
__device__ __forceinline__ uint32_t code_at(const uint8_t* codes, const uint8_t* hp, size_t blk,
                                            int kk, int scheme)
{
    const int L = kk & 7, G = kk >> 3;
    const uint8_t byte = codes[blk * 64 + dcode_off(L, G & 7)];
    uint32_t code = G < 8 ? (byte & 15u) : (byte >> 4);
    if (scheme == 3) {
        const uint8_t hb = hp[blk * 32 + dhp_off(L, G & 3)];
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
    const size_t blk = row * (size_t)nb + (size_t)(k >> 7);
    const uint32_t code = code_at(codes, hp, blk, k & 127, SCHEME);
    const uint32_t p = params[param_idx(row, nb, k >> 7)];
    out[k] = __fadd_rn(h2f(p & 0xFFFFu), __fmul_rn((float)code, h2f(p >> 16)));
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
    const uint32_t code = code_at(codes, hp, blk, (int)(i & 127), SCHEME);
    const uint32_t p = params[param_idx(row, nb, b)];
    const float zp = h2f(p & 0xFFFFu), sc = h2f(p >> 16);
    w[i] = rounding == WPCG_ROUND_FMA ? __builtin_fmaf((float)code, sc, zp)
                                      : __fadd_rn(zp, __fmul_rn((float)code, sc));
}

}  // namespace

// ============================================================ launchers
int fast_kslices(uint64_t rows, uint64_t nb)
{
    if (nb == 0) return 1;
    constexpr int KS = 4 / FAST_TILES;
    const uint64_t tiles = pad_rows(rows) / TILE_ROWS;
    const uint64_t tgroups = (tiles + FAST_TILES - 1) / FAST_TILES;
    uint64_t kg = (nb + MAXBK - 1) / MAXBK;
    // more K-slices until the launch has >= 512 workgroups, keeping at least
    // two blocks per wave
    while (tgroups * kg < 512) {
        const uint64_t nbk = (nb + kg) / (kg + 1);
        if (nbk < 2 * KS) break;
        kg++;
    }
    return fast_normalize_kslices(nb, (int)kg);
}

hipError_t launch_gemv_exact(const DeviceMatrix& m, const float* x, const float* bias, float* y,
                             hipStream_t s)
{
    const int rows = (int)m.rows, nb = (int)m.nb;
    dim3 grid((unsigned)(m.rows_pad / (EX_WG / 8)));
    (void)hipGetLastError();  // report only this launch
    if (m.scheme == 4)
        hipLaunchKernelGGL(k_gemv_exact<4>, grid, dim3(EX_WG), 0, s, m.codes, m.hp, m.params, x,
                           bias, y, rows, nb);
    else
        hipLaunchKernelGGL(k_gemv_exact<3>, grid, dim3(EX_WG), 0, s, m.codes, m.hp, m.params, x,
                           bias, y, rows, nb);
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
        const DeviceMatrix& m = *jobs[i].m;
        if (m.scheme != scheme) return hipErrorInvalidValue;
        FastProblem& P = B.p[i];
        P.codes = m.codes;
        P.hp = m.hp;
        P.params = m.params;
        P.x = jobs[i].x;
        P.y = jobs[i].y;
        P.bias = jobs[i].bias;
        P.part = jobs[i].plan->part;
        P.counters = jobs[i].plan->counters;
        P.rows = (int)m.rows;
        P.rows_pad = (int)m.rows_pad;
        P.nb = (int)m.nb;
        P.kg = jobs[i].plan->kg;
        P.wg_begin = wgs;
        const int tgroups = (int)((m.rows_pad / TILE_ROWS + FAST_TILES - 1) / FAST_TILES);
        wgs += tgroups * P.kg;
    }
    if (wgs == 0) return hipSuccess;
    (void)hipGetLastError();  // report only this launch
    if (scheme == 4)
        hipLaunchKernelGGL(k_gemv_fast<4>, dim3(wgs), dim3(FAST_WG), 0, s, B);
    else
        hipLaunchKernelGGL(k_gemv_fast<3>, dim3(wgs), dim3(FAST_WG), 0, s, B);
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
