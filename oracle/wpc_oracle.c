/*
 * wpc_oracle.c -- CPU restatement of the reference (jpytka666-jpg/wpc-engine,
 * pure Rust) for the quantized dequant-GEMV and Qwen3-MoE routing path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker the HIP library is compared
 * against, and the CPU baseline bench.py times. The product never links it.
 *
 * Every function names the reference file:line it restates. Compile with
 * -ffp-contract=off (see wpc_oracle.h): the reference is Rust, which never
 * fuses `a + b * c`, and every single-rounding step it does take is an
 * explicit `_mm256_fmadd_ps`, restated here as fmaf().
 *
 * Pinning (what independent check fails if this restatement is wrong) is
 * listed per function in tests/test_oracle_*.py and in the oracle section
 * of the design notes.
 */
#include "wpc_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef OR_POOL_STALL_US
#include <unistd.h>
#endif

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------------ */
/* binary16                                                                  */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Exact widening, as `half::f16::to_f32` (half 2.7.1, Cargo.lock:341-342).
 * NaNs come out quiet with the payload kept in the high mantissa bits. */
float or_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1F)
        return u2f(sign | 0x7F800000u | (m ? (0x00400000u | (m << 13)) : 0u));
    if (e != 0)
        return u2f(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0)
        return u2f(sign);
    /* subnormal: m * 2^-24, exact in binary32 */
    float v = (float)m * 0x1p-24f;
    return sign ? -v : v;
}

/* Round-to-nearest-even narrowing, as `half::f16::from_f32`. Overflow goes
 * to infinity, NaN stays NaN (quiet bit set). */
uint16_t or_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {
        if (ax == 0x7F800000u) return sign | 0x7C00u;
        return sign | 0x7E00u | (uint16_t)((ax & 0x007FFFFFu) >> 13);
    }
    int e = (int)(ax >> 23) - 127; /* unbiased exponent of |f| */
    if (e >= 16) return sign | 0x7C00u;
    /* significand with the implicit bit, scaled so that the value is
     * sig * 2^(e-23) */
    uint32_t sig = (ax & 0x007FFFFFu) | (e > -127 ? 0x00800000u : 0u);
    if (e == -127) e = -126; /* binary32 subnormal */
    /* target: half ulp exponent is max(e, -14) - 10 */
    int half_e = e < -14 ? -14 : e;
    int shift = (half_e - 10) - (e - 23); /* bits of sig to drop */
    uint32_t q, rem, halfway;
    if (shift >= 32) {
        q = 0; rem = sig; halfway = 0xFFFFFFFFu; /* |f| < 2^-25: rounds to 0 */
        if (shift == 32) { halfway = 0x80000000u; }
    } else {
        q = sig >> shift;
        rem = sig & ((1u << shift) - 1u);
        halfway = 1u << (shift - 1);
    }
    if (rem > halfway || (rem == halfway && (q & 1u))) q += 1u;
    /* q is the significand in units of the half ulp at exponent half_e */
    uint32_t bits;
    if (half_e == -14 && q < 0x400u) {
        bits = q; /* subnormal (or zero) */
    } else {
        /* q in [0x400, 0x800]; 0x800 means a carry into the next binade */
        int be = half_e + 15;
        if (q >= 0x800u) { q >>= 1; be += 1; }
        if (be >= 31) return sign | 0x7C00u;
        bits = ((uint32_t)be << 10) | (q & 0x3FFu);
    }
    return sign | (uint16_t)bits;
}

void or_f16_to_f32_array(const uint16_t* h, float* out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(h[i]);
}

void or_f32_to_f16_array(const float* f, uint16_t* out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = or_f32_to_f16(f[i]);
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* ------------------------------------------------------------------------ */
/* codecs                                                                    */
/* ------------------------------------------------------------------------ */

/* QuantBlockV4::pack_codes (wpc-format/src/lib.rs:348-356) */
void or_v4_pack_codes(const uint8_t codes[128], uint8_t packed[64])
{
    for (int j = 0; j < 64; j++)
        packed[j] = (uint8_t)((codes[j] & 0x0F) | ((codes[j + 64] & 0x0F) << 4));
}

/* QuantBlockV4::unpack_codes (wpc-format/src/lib.rs:360-367) */
void or_v4_unpack_codes(const uint8_t packed[64], uint8_t codes[128])
{
    for (int j = 0; j < 64; j++) {
        codes[j] = packed[j] & 0x0F;
        codes[j + 64] = packed[j] >> 4;
    }
}

/* QuantBlockV3::pack_codes (wpc-format/src/lib.rs:229-241): four 6-bit codes
 * in three bytes, c0 in the low bits of byte 0. */
void or_v3_pack_codes(const uint8_t codes[128], uint8_t packed[96])
{
    for (int g = 0; g < 32; g++) {
        uint32_t word = (uint32_t)(codes[4 * g] & 0x3F)
                      | (uint32_t)(codes[4 * g + 1] & 0x3F) << 6
                      | (uint32_t)(codes[4 * g + 2] & 0x3F) << 12
                      | (uint32_t)(codes[4 * g + 3] & 0x3F) << 18;
        packed[3 * g] = (uint8_t)word;
        packed[3 * g + 1] = (uint8_t)(word >> 8);
        packed[3 * g + 2] = (uint8_t)(word >> 16);
    }
}

/* QuantBlockV3::unpack_codes (wpc-format/src/lib.rs:245-257) */
void or_v3_unpack_codes(const uint8_t packed[96], uint8_t codes[128])
{
    for (int g = 0; g < 32; g++) {
        uint32_t word = (uint32_t)packed[3 * g] | (uint32_t)packed[3 * g + 1] << 8
                      | (uint32_t)packed[3 * g + 2] << 16;
        for (int q = 0; q < 4; q++) codes[4 * g + q] = (uint8_t)((word >> (6 * q)) & 0x3F);
    }
}

void or_v3tp_pack(const uint8_t codes[128], uint8_t lp[64], uint8_t hp[32])
{
    for (int j = 0; j < 64; j++)
        lp[j] = (uint8_t)((codes[j] & 0x0F) | ((codes[j + 64] & 0x0F) << 4));
    for (int j = 0; j < 32; j++) {
        uint8_t v = 0;
        for (int q = 0; q < 4; q++) v |= (uint8_t)(((codes[j + 32 * q] >> 4) & 3) << (2 * q));
        hp[j] = v;
    }
}

void or_v3tp_unpack(const uint8_t lp[64], const uint8_t hp[32], uint8_t codes[128])
{
    for (int k = 0; k < 128; k++) {
        uint8_t nib = k < 64 ? (lp[k] & 0x0F) : (lp[k - 64] >> 4);
        uint8_t top = (hp[k & 31] >> (2 * (k >> 5))) & 3;
        codes[k] = (uint8_t)(nib | (top << 4));
    }
}

/* ------------------------------------------------------------------------ */
/* encoder (wpc-core/src/quant_encoder.rs)                                   */
/* ------------------------------------------------------------------------ */

/* Shared min/max affine fit of affine_quant_block (:7-26) and
 * affine_quant_block_v4 (:66-85). `levels` is 63 or 15. Codes use the fp32
 * min and scale; f32::round is half-away-from-zero (roundf). */
static void affine_fit(const float w[128], float levels, uint8_t codes[128],
                       uint16_t* zp_out, uint16_t* scale_out)
{
    float min_v = 3.40282347e+38f, max_v = -3.40282347e+38f;
    for (int i = 0; i < 128; i++) {
        if (w[i] < min_v) min_v = w[i];
        if (w[i] > max_v) max_v = w[i];
    }
    float scale = max_v > min_v ? (max_v - min_v) / levels : 1.0f;
    for (int i = 0; i < 128; i++) {
        float c = roundf((w[i] - min_v) / scale);
        /* f32::clamp then `as u8`: NaN saturates to 0 */
        if (c != c) c = 0.0f;
        if (c < 0.0f) c = 0.0f;
        if (c > levels) c = levels;
        codes[i] = (uint8_t)c;
    }
    *zp_out = or_f32_to_f16(min_v);
    *scale_out = or_f32_to_f16(scale);
}

void or_affine_quant_block_v2(const float w[128], uint8_t out[132])
{
    uint16_t zp, sc;
    affine_fit(w, 63.0f, out + 4, &zp, &sc);
    wr16(out, zp);
    wr16(out + 2, sc);
}

/* affine_quant_block_v3 (:44-46): the v2 block re-laid out (from_v2). */
void or_affine_quant_block_v3(const float w[128], uint8_t out[100])
{
    uint8_t v2[132];
    or_affine_quant_block_v2(w, v2);
    memcpy(out, v2, 4);
    or_v3_pack_codes(v2 + 4, out + 4);
}

void or_affine_quant_block_v4(const float w[128], uint8_t out[68])
{
    uint8_t codes[128];
    uint16_t zp, sc;
    affine_fit(w, 15.0f, codes, &zp, &sc);
    wr16(out, zp);
    wr16(out + 2, sc);
    or_v4_pack_codes(codes, out + 4);
}

/* encode_tensor_v4 (:88-96) / encode_tensor_v3 (:49-57) */
void or_encode_tensor_v4(const float* data, size_t n, uint8_t* out)
{
    for (size_t b = 0; b < n / 128; b++) or_affine_quant_block_v4(data + 128 * b, out + 68 * b);
}

void or_encode_tensor_v3(const float* data, size_t n, uint8_t* out)
{
    for (size_t b = 0; b < n / 128; b++) or_affine_quant_block_v3(data + 128 * b, out + 100 * b);
}

/* ------------------------------------------------------------------------ */
/* row kernels (wpc-eval/src/fused_kernel.rs)                                */
/* ------------------------------------------------------------------------ */

/* hsum_avx2 (fused_kernel.rs:8-19): ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) */
static inline float hsum8(const float a[8])
{
    float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s1) + (s2 + s3);
}

/* matvec_v4_scalar (fused_kernel.rs:278-294): stored order, two roundings
 * per dequant (`zp + lo * scale`), sequential accumulation. */
float or_matvec_v4_scalar(const uint8_t* blocks, const float* x, size_t n_blocks)
{
    float acc = 0.0f;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* blk = blocks + 68 * b;
        float zp = or_f16_to_f32(rd16(blk)), sc = or_f16_to_f32(rd16(blk + 2));
        const float* xr = x + 128 * b;
        for (int j = 0; j < 64; j++) {
            uint8_t byte = blk[4 + j];
            float lo = (float)(byte & 0x0F), hi = (float)(byte >> 4);
            acc += (zp + lo * sc) * xr[j];
            acc += (zp + hi * sc) * xr[64 + j];
        }
    }
    return acc;
}

/* matvec_v4_fused (fused_kernel.rs:237-271), one AVX2 lane at a time: lane
 * l of group g takes byte g*8+l; low nibble pairs with x[g*8+l], high
 * nibble with x[64+g*8+l]; w = fma(code, scale, zp); acc = fma(w, x, acc),
 * low before high; hsum_avx2 at the end. */
float or_matvec_v4_fused(const uint8_t* blocks, const float* x, size_t n_blocks)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* blk = blocks + 68 * b;
        float zp = or_f16_to_f32(rd16(blk)), sc = or_f16_to_f32(rd16(blk + 2));
        const float* xr = x + 128 * b;
        for (int g = 0; g < 8; g++)
            for (int l = 0; l < 8; l++) {
                uint8_t byte = blk[4 + g * 8 + l];
                float wlo = fmaf((float)(byte & 0x0F), sc, zp);
                acc[l] = fmaf(wlo, xr[g * 8 + l], acc[l]);
                float whi = fmaf((float)(byte >> 4), sc, zp);
                acc[l] = fmaf(whi, xr[64 + g * 8 + l], acc[l]);
            }
    }
    return hsum8(acc);
}

/* matvec_v3_scalar (fused_kernel.rs:196-220): natural order, two roundings */
float or_matvec_v3_scalar(const uint8_t* blocks, const float* x, size_t n_blocks)
{
    float acc = 0.0f;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* blk = blocks + 100 * b;
        float zp = or_f16_to_f32(rd16(blk)), sc = or_f16_to_f32(rd16(blk + 2));
        uint8_t codes[128];
        or_v3_unpack_codes(blk + 4, codes);
        for (int k = 0; k < 128; k++) acc += (zp + (float)codes[k] * sc) * x[128 * b + k];
    }
    return acc;
}

/* matvec_v3_fused (fused_kernel.rs:163-189): codes unpacked to natural order,
 * 16 groups of 8 lanes, acc = fma(fma(c, scale, zp), x, acc). */
float or_matvec_v3_fused(const uint8_t* blocks, const float* x, size_t n_blocks)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* blk = blocks + 100 * b;
        float zp = or_f16_to_f32(rd16(blk)), sc = or_f16_to_f32(rd16(blk + 2));
        uint8_t codes[128];
        or_v3_unpack_codes(blk + 4, codes);
        for (int g = 0; g < 16; g++)
            for (int l = 0; l < 8; l++)
                acc[l] = fmaf(fmaf((float)codes[g * 8 + l], sc, zp), x[128 * b + g * 8 + l], acc[l]);
    }
    return hsum8(acc);
}

/* matvec_v2_scalar (fused_kernel.rs:133-147), used to pin v3 against v2 as the
 * reference's own tests do (fused_kernel.rs:488-498). */
float or_matvec_v2_scalar(const uint8_t* blocks, const float* x, size_t n_blocks)
{
    float acc = 0.0f;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* blk = blocks + 132 * b;
        float zp = or_f16_to_f32(rd16(blk)), sc = or_f16_to_f32(rd16(blk + 2));
        for (int k = 0; k < 128; k++) acc += (zp + (float)blk[4 + k] * sc) * x[128 * b + k];
    }
    return acc;
}

#if defined(__x86_64__)
#include <cpuid.h>
int or_have_avx2_fma(void)
{
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

__attribute__((target("avx2,fma"))) static float hsum_avx2(__m256 v)
{
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    __m128 sh = _mm_movehdup_ps(s);
    __m128 sums = _mm_add_ps(s, sh);
    __m128 sh2 = _mm_movehl_ps(sh, sums);
    return _mm_cvtss_f32(_mm_add_ss(sums, sh2));
}

/* matvec_v4_fused with the reference's own intrinsic sequence
 * (fused_kernel.rs:237-271). */
__attribute__((target("avx2,fma"))) static float v4_fused_avx2(const uint8_t* blocks,
                                                               const float* x, size_t nb)
{
    __m256 acc = _mm256_setzero_ps();
    const __m256i mask = _mm256_set1_epi32(0x0F);
    for (size_t i = 0; i < nb; i++) {
        const uint8_t* blk = blocks + 68 * i;
        __m256 zp = _mm256_set1_ps(or_f16_to_f32(rd16(blk)));
        __m256 sc = _mm256_set1_ps(or_f16_to_f32(rd16(blk + 2)));
        const float* row = x + 128 * i;
        for (int g = 0; g < 8; g++) {
            __m128i raw = _mm_loadl_epi64((const __m128i*)(blk + 4 + 8 * g));
            __m256i wide = _mm256_cvtepu8_epi32(raw);
            __m256 lo = _mm256_cvtepi32_ps(_mm256_and_si256(wide, mask));
            acc = _mm256_fmadd_ps(_mm256_fmadd_ps(lo, sc, zp), _mm256_loadu_ps(row + 8 * g), acc);
            __m256 hi = _mm256_cvtepi32_ps(_mm256_srli_epi32(wide, 4));
            acc = _mm256_fmadd_ps(_mm256_fmadd_ps(hi, sc, zp), _mm256_loadu_ps(row + 64 + 8 * g), acc);
        }
    }
    return hsum_avx2(acc);
}

/* matvec_v3_fused with intrinsics (fused_kernel.rs:163-189) */
__attribute__((target("avx2,fma"))) static float v3_fused_avx2(const uint8_t* blocks,
                                                               const float* x, size_t nb)
{
    __m256 acc = _mm256_setzero_ps();
    for (size_t i = 0; i < nb; i++) {
        const uint8_t* blk = blocks + 100 * i;
        uint8_t codes[128];
        or_v3_unpack_codes(blk + 4, codes);
        __m256 zp = _mm256_set1_ps(or_f16_to_f32(rd16(blk)));
        __m256 sc = _mm256_set1_ps(or_f16_to_f32(rd16(blk + 2)));
        for (int g = 0; g < 16; g++) {
            __m128i raw = _mm_loadl_epi64((const __m128i*)(codes + 8 * g));
            __m256 c = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(raw));
            __m256 w = _mm256_fmadd_ps(c, sc, zp);
            acc = _mm256_fmadd_ps(w, _mm256_loadu_ps(x + 128 * i + 8 * g), acc);
        }
    }
    return hsum_avx2(acc);
}

int or_matvec_v4_fused_avx2(const uint8_t* blocks, const float* x, size_t nb, float* out)
{
    if (!or_have_avx2_fma()) return 0;
    *out = v4_fused_avx2(blocks, x, nb);
    return 1;
}

int or_matvec_v3_fused_avx2(const uint8_t* blocks, const float* x, size_t nb, float* out)
{
    if (!or_have_avx2_fma()) return 0;
    *out = v3_fused_avx2(blocks, x, nb);
    return 1;
}
#else
int or_have_avx2_fma(void) { return 0; }
int or_matvec_v4_fused_avx2(const uint8_t* b, const float* x, size_t n, float* o)
{ (void)b; (void)x; (void)n; (void)o; return 0; }
int or_matvec_v3_fused_avx2(const uint8_t* b, const float* x, size_t n, float* o)
{ (void)b; (void)x; (void)n; (void)o; return 0; }
#endif

/* ------------------------------------------------------------------------ */
/* row-parallel driver (rayon par_iter_mut over output rows in the reference)*/
/* ------------------------------------------------------------------------ */

typedef void (*row_fn)(void* ctx, size_t r0, size_t r1);

typedef struct {
    row_fn fn;
    void* ctx;
    size_t n, chunk;
    atomic_size_t next;
} par_job;

static void* par_worker(void* arg)
{
    par_job* j = (par_job*)arg;
    for (;;) {
        size_t r0 = atomic_fetch_add(&j->next, j->chunk);
        if (r0 >= j->n) break;
        size_t r1 = r0 + j->chunk < j->n ? r0 + j->chunk : j->n;
        j->fn(j->ctx, r0, r1);
    }
    return NULL;
}

/* A persistent worker pool, as rayon's global pool in the reference: worker
 * threads are started on first need; between jobs each spins briefly on the
 * job generation and then sleeps on a condition variable, so a call costs a
 * wake-up (or nothing, when calls follow closely) rather than thread
 * creation, which made a decode step slower on 16 threads than on one. One
 * job runs at a time; the caller takes part and returns when every worker it
 * woke is done. After fork() the child starts with an empty pool. */
#define POOL_MAX 255
#define POOL_SPIN 1024 /* pause iterations before sleeping (tens of us) */
static struct {
    pthread_mutex_t mu;
    pthread_cond_t cv_job, cv_done;
    int nworkers;          /* started, excluding callers */
    atomic_ulong gen;      /* job generation */
    _Atomic(par_job*) job;
    atomic_int want;       /* workers with id < want take part in the job */
    atomic_int pending;    /* of those, not yet done */
} g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER, 0, 0, NULL, 0, 0};
static pthread_mutex_t g_pool_call = PTHREAD_MUTEX_INITIALIZER;
static pthread_once_t g_pool_once = PTHREAD_ONCE_INIT;
/* the job generation when worker i was started: it first runs the next one
 * (the job it was started for, published before it can take the lock) */
static unsigned long g_pool_gen0[POOL_MAX];

static inline void cpu_pause(void)
{
#if defined(__x86_64__)
    _mm_pause();
#endif
}

static void pool_reset_in_child(void)
{
    pthread_mutex_init(&g_pool.mu, NULL);
    pthread_cond_init(&g_pool.cv_job, NULL);
    pthread_cond_init(&g_pool.cv_done, NULL);
    pthread_mutex_init(&g_pool_call, NULL);
    g_pool.nworkers = 0;
    atomic_store(&g_pool.gen, 0);
    atomic_store(&g_pool.job, NULL);
    atomic_store(&g_pool.want, 0);
    atomic_store(&g_pool.pending, 0);
}
static void pool_init_once(void) { pthread_atfork(NULL, NULL, pool_reset_in_child); }

static void* pool_worker(void* arg)
{
    const int id = (int)(intptr_t)arg;  /* 0-based among the workers */
    pthread_mutex_lock(&g_pool.mu);
    unsigned long seen = g_pool_gen0[id];
    pthread_mutex_unlock(&g_pool.mu);
    for (;;) {
        for (int i = 0; i < POOL_SPIN && atomic_load(&g_pool.gen) == seen; i++) cpu_pause();
        /* The generation, `want` and the job are read together under the
         * lock the caller holds while it publishes all three. Read without
         * it, a worker that sits a job out could read the generation, stall,
         * and then read the next call's `want` and job: it would run that
         * job under the old generation and, seeing the new one on its next
         * loop, run it a second time, counting `pending` down twice. A
         * worker counted in a job always sees that job's generation: no new
         * job is published before `pending` reaches zero. */
        pthread_mutex_lock(&g_pool.mu);
        while (atomic_load(&g_pool.gen) == seen) pthread_cond_wait(&g_pool.cv_job, &g_pool.mu);
        seen = atomic_load(&g_pool.gen);
#ifdef OR_POOL_STALL_US /* stress builds only: widen the window between the reads */
        usleep(OR_POOL_STALL_US);
#endif
        const int take = id < atomic_load(&g_pool.want);
        par_job* j = atomic_load(&g_pool.job);
        pthread_mutex_unlock(&g_pool.mu);
        if (!take) continue;
        par_worker(j);
        if (atomic_fetch_sub(&g_pool.pending, 1) == 1) {
            pthread_mutex_lock(&g_pool.mu);
            pthread_cond_signal(&g_pool.cv_done);
            pthread_mutex_unlock(&g_pool.mu);
        }
    }
    return NULL;
}

static void parallel_rows(size_t n, int threads, row_fn fn, void* ctx)
{
    if (threads <= 1 || n < 64) { fn(ctx, 0, n); return; }
    if (threads > POOL_MAX + 1) threads = POOL_MAX + 1;
    pthread_once(&g_pool_once, pool_init_once);
    par_job j;
    j.fn = fn; j.ctx = ctx; j.n = n;
    j.chunk = n / ((size_t)threads * 8);
    if (j.chunk < 16) j.chunk = 16;
    atomic_init(&j.next, 0);
    pthread_mutex_lock(&g_pool_call);
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.nworkers < threads - 1) {
        pthread_t t;
        pthread_attr_t at;
        pthread_attr_init(&at);
        pthread_attr_setdetachstate(&at, PTHREAD_CREATE_DETACHED);
        g_pool_gen0[g_pool.nworkers] = atomic_load(&g_pool.gen);
        const int ok = pthread_create(&t, &at, pool_worker, (void*)(intptr_t)g_pool.nworkers) == 0;
        pthread_attr_destroy(&at);
        if (!ok) break;
        g_pool.nworkers++;
    }
    const int w = g_pool.nworkers < threads - 1 ? g_pool.nworkers : threads - 1;
    atomic_store(&g_pool.job, &j);
    atomic_store(&g_pool.want, w);
    atomic_store(&g_pool.pending, w);
    atomic_fetch_add(&g_pool.gen, 1);
    pthread_cond_broadcast(&g_pool.cv_job);
    pthread_mutex_unlock(&g_pool.mu);
    par_worker(&j);
    for (int i = 0; i < POOL_SPIN && atomic_load(&g_pool.pending) > 0; i++) cpu_pause();
    pthread_mutex_lock(&g_pool.mu);
    while (atomic_load(&g_pool.pending) > 0) pthread_cond_wait(&g_pool.cv_done, &g_pool.mu);
    pthread_mutex_unlock(&g_pool.mu);
    pthread_mutex_unlock(&g_pool_call);
}

typedef struct {
    const uint8_t* blocks;
    size_t nb, bpb;
    const float* x;
    float* y;
    int kernel, scheme;
} lin_ctx;

static void lin_rows(void* p, size_t r0, size_t r1)
{
    lin_ctx* c = (lin_ctx*)p;
    for (size_t r = r0; r < r1; r++) {
        const uint8_t* rb = c->blocks + r * c->nb * c->bpb;
        float v;
        if (c->scheme == 4) {
            if (c->kernel == 0) v = or_matvec_v4_scalar(rb, c->x, c->nb);
            else if (c->kernel == 2 && or_matvec_v4_fused_avx2(rb, c->x, c->nb, &v)) {}
            else v = or_matvec_v4_fused(rb, c->x, c->nb);
        } else {
            if (c->kernel == 0) v = or_matvec_v3_scalar(rb, c->x, c->nb);
            else if (c->kernel == 2 && or_matvec_v3_fused_avx2(rb, c->x, c->nb, &v)) {}
            else v = or_matvec_v3_fused(rb, c->x, c->nb);
        }
        c->y[r] = v;
    }
}

/* WpcLinearV4::matvec (wpc_runtime/src/wpc_weights_v4.rs:165-193): one row
 * kernel per output row, then `y += bias` when a bias is present. */
void or_linear_v4_matvec(const uint8_t* blocks, size_t out_f, size_t in_f, const float* x,
                         const float* bias, float* y, int kernel, int threads)
{
    lin_ctx c = {blocks, in_f / 128, 68, x, y, kernel, 4};
    parallel_rows(out_f, threads, lin_rows, &c);
    if (bias)
        for (size_t r = 0; r < out_f; r++) y[r] += bias[r];
}

/* WpcLinearV3::matvec (wpc_weights_v3.rs:164-193) */
void or_linear_v3_matvec(const uint8_t* blocks, size_t out_f, size_t in_f, const float* x,
                         const float* bias, float* y, int kernel, int threads)
{
    lin_ctx c = {blocks, in_f / 128, 100, x, y, kernel, 3};
    parallel_rows(out_f, threads, lin_rows, &c);
    if (bias)
        for (size_t r = 0; r < out_f; r++) y[r] += bias[r];
}

void or_linear_v4_matmul(const uint8_t* blocks, size_t out_f, size_t in_f, const float* X,
                         size_t M, float* Y, int kernel, int threads)
{
    for (size_t m = 0; m < M; m++)
        or_linear_v4_matvec(blocks, out_f, in_f, X + m * in_f, NULL, Y + m * out_f, kernel, threads);
}

/* row_decode_into_v4 (wpc_weights_v4.rs:103-115) via WpcEmbeddingV4::embed
 * (:241-249): natural order, `zp + code * scale` with two roundings. */
void or_embed_v4(const uint8_t* blocks, size_t hidden, uint32_t token, float* out)
{
    size_t nb = hidden / 128;
    const uint8_t* rb = blocks + (size_t)token * nb * 68;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = rb + 68 * b;
        float zp = or_f16_to_f32(rd16(blk)), sc = or_f16_to_f32(rd16(blk + 2));
        uint8_t codes[128];
        or_v4_unpack_codes(blk + 4, codes);
        for (int k = 0; k < 128; k++) out[128 * b + k] = zp + (float)codes[k] * sc;
    }
}

/* row_decode_into_v3 (wpc_weights_v3.rs:101-114) */
void or_embed_v3(const uint8_t* blocks, size_t hidden, uint32_t token, float* out)
{
    size_t nb = hidden / 128;
    const uint8_t* rb = blocks + (size_t)token * nb * 100;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = rb + 100 * b;
        float zp = or_f16_to_f32(rd16(blk)), sc = or_f16_to_f32(rd16(blk + 2));
        uint8_t codes[128];
        or_v3_unpack_codes(blk + 4, codes);
        for (int k = 0; k < 128; k++) out[128 * b + k] = zp + (float)codes[k] * sc;
    }
}

/* ------------------------------------------------------------------------ */
/* dense ops                                                                 */
/* ------------------------------------------------------------------------ */

/* DenseLinear::matvec (wpc-runtime/src/weights.rs:59-78): sequential row dot,
 * `acc += row[i] * x[i]` rounded twice. */
void or_dense_matvec(const float* W, size_t out_f, size_t in_f, const float* x,
                     const float* bias, float* y)
{
    for (size_t r = 0; r < out_f; r++) {
        const float* row = W + r * in_f;
        float acc = 0.0f;
        for (size_t i = 0; i < in_f; i++) acc += row[i] * x[i];
        y[r] = acc;
    }
    if (bias)
        for (size_t r = 0; r < out_f; r++) y[r] += bias[r];
}

/* softmax_inplace (wpc-runtime/src/norm.rs:28-43). f32::max drops NaN like
 * fmaxf; f32::exp is libm expf. */
void or_softmax_inplace(float* x, size_t n)
{
    if (n == 0) return;
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = fmaxf(mx, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    if (sum > 0.0f)
        for (size_t i = 0; i < n; i++) x[i] /= sum;
}

/* rms_norm (wpc-runtime/src/norm.rs:4-13) */
void or_rms_norm(const float* x, const float* w, size_t n, float eps, float* out)
{
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s += x[i] * x[i];
    float mean_sq = s / (float)n;
    float scale = 1.0f / sqrtf(mean_sq + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* apply_rope / apply_rope_partial with rotary_pairs = d/2
 * (wpc-runtime/src/rope.rs:10-40): angles in f64, cos/sin cast to f32. */
void or_apply_rope(float* x, size_t d, size_t pos, double theta)
{
    size_t half = d / 2;
    for (size_t i = 0; i < half; i++) {
        double inv_freq = pow(theta, -(2.0 * (double)i) / (double)d);
        double angle = (double)pos * inv_freq;
        float s = (float)sin(angle), c = (float)cos(angle);
        float x1 = x[i], x2 = x[i + half];
        x[i] = x1 * c - x2 * s;
        x[i + half] = x2 * c + x1 * s;
    }
}

/* argmax (wpc-runtime/src/sampling.rs:3-14): first index of the maximum */
uint32_t or_argmax(const float* logits, size_t n)
{
    size_t best = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (logits[i] > bv) { bv = logits[i]; best = i; }
    return (uint32_t)best;
}

/* SiLU(g) * u as at qwen3_moe_model.rs:518-522 and model.rs:527-531 */
float or_silu_mul(float g, float u)
{
    float silu = g / (1.0f + expf(-g));
    return silu * u;
}

void or_silu_mul_array(const float* g, const float* u, float* out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = or_silu_mul(g[i], u[i]);
}
/* Qwen3MoeModel::route (qwen3_moe_model.rs:376-402): k strict-`>` scans, so
 * ties go to the lowest index; then divide by the (sequential) sum of the k
 * weights when norm_topk and that sum is positive. */
size_t or_route(const float* scores, size_t n, size_t top_k, int norm_topk, int32_t* ids,
                float* weights)
{
    unsigned char* taken = (unsigned char*)calloc(n ? n : 1, 1);
    size_t got = 0;
    for (size_t k = 0; k < top_k; k++) {
        size_t best = (size_t)-1;
        float bv = -INFINITY;
        for (size_t i = 0; i < n; i++)
            if (!taken[i] && scores[i] > bv) { bv = scores[i]; best = i; }
        if (best == (size_t)-1) break;
        taken[best] = 1;
        ids[got] = (int32_t)best;
        weights[got] = bv;
        got++;
    }
    free(taken);
    if (norm_topk) {
        float sum = 0.0f;
        for (size_t k = 0; k < got; k++) sum += weights[k];
        if (sum > 0.0f)
            for (size_t k = 0; k < got; k++) weights[k] /= sum;
    }
    return got;
}

/* Sparse MLP half of Qwen3MoeModel::forward_token (qwen3_moe_model.rs:500-530) */
void or_moe_ffn_v4(const float* router_w, size_t n_exp, size_t hidden, size_t inter,
                   size_t top_k, int norm_topk, const or_expert_v4* experts, const float* x,
                   float* mlp_out, int32_t* chosen_ids, float* chosen_w, int kernel, int threads)
{
    float* scores = (float*)malloc(n_exp * sizeof(float));
    float* gate = (float*)malloc(inter * sizeof(float));
    float* up = (float*)malloc(inter * sizeof(float));
    float* eo = (float*)malloc(hidden * sizeof(float));
    or_dense_matvec(router_w, n_exp, hidden, x, NULL, scores);
    or_softmax_inplace(scores, n_exp);
    size_t got = or_route(scores, n_exp, top_k, norm_topk, chosen_ids, chosen_w);
    for (size_t i = 0; i < hidden; i++) mlp_out[i] = 0.0f;
    for (size_t k = 0; k < got; k++) {
        const or_expert_v4* e = &experts[chosen_ids[k]];
        float w = chosen_w[k];
        or_linear_v4_matvec(e->gate, inter, hidden, x, NULL, gate, kernel, threads);
        or_linear_v4_matvec(e->up, inter, hidden, x, NULL, up, kernel, threads);
        for (size_t i = 0; i < inter; i++) gate[i] = or_silu_mul(gate[i], up[i]);
        or_linear_v4_matvec(e->down, hidden, inter, gate, NULL, eo, kernel, threads);
        for (size_t i = 0; i < hidden; i++) mlp_out[i] += w * eo[i];
    }
    for (size_t k = got; k < top_k; k++) { chosen_ids[k] = -1; chosen_w[k] = 0.0f; }
    free(scores); free(gate); free(up); free(eo);
}

/* ------------------------------------------------------------------------ */
/* decode step                                                               */
/* ------------------------------------------------------------------------ */

struct or_kv_cache {
    size_t n_layers, n_kv, head_dim, max_pos, len;
    float* k; /* [layer][kv_head][max_pos][head_dim] */
    float* v;
};

or_kv_cache* or_kv_cache_new(const or_model_cfg* cfg, size_t max_pos)
{
    or_kv_cache* c = (or_kv_cache*)calloc(1, sizeof(*c));
    if (!c) return NULL;
    c->n_layers = cfg->n_layers; c->n_kv = cfg->n_kv_heads; c->head_dim = cfg->head_dim;
    c->max_pos = max_pos; c->len = 0;
    size_t n = cfg->n_layers * cfg->n_kv_heads * max_pos * cfg->head_dim;
    c->k = (float*)malloc((n ? n : 1) * sizeof(float));
    c->v = (float*)malloc((n ? n : 1) * sizeof(float));
    if (!c->k || !c->v) { free(c->k); free(c->v); free(c); return NULL; }
    return c;
}

void or_kv_cache_free(or_kv_cache* c)
{
    if (!c) return;
    free(c->k); free(c->v); free(c);
}

size_t or_kv_cache_len(const or_kv_cache* c) { return c->len; }

/* Model::forward_token (model.rs:419-547) when cfg.n_exp == 0 (dense Qwen3:
 * q_norm/k_norm present, logits through embed.logits, model.rs:545, whatever
 * the checkpoint's tie_word_embeddings: qwen3_model.rs:187-206 builds no
 * lm_head), and Qwen3MoeModel::forward_token (qwen3_moe_model.rs:406-542)
 * otherwise, whose logits always come from lm_head (:337-343, :540).
 * Returns -1 for a MoE model without lm_head. */
int or_forward_token_v4(const or_model_v4* m, uint32_t token, or_kv_cache* cache,
                        float* logits, int kernel, int threads)
{
    const or_model_cfg* cfg = &m->cfg;
    size_t h = cfg->hidden, hd = cfg->head_dim, nh = cfg->n_heads, nkv = cfg->n_kv_heads;
    size_t n_rep = nh / nkv, pos = cache->len;
    if (pos >= cache->max_pos || token >= cfg->vocab) return -1;
    const uint8_t* head = cfg->n_exp ? m->lm_head : m->embed;
    if (!head) return -1;
    float eps = cfg->eps;
    size_t qd = nh * hd, kvd = nkv * hd;
    size_t inter = cfg->n_exp ? cfg->moe_inter : cfg->inter;
    size_t seq_len = pos + 1;

    float* residual = (float*)malloc(h * sizeof(float));
    float* normed = (float*)malloc(h * sizeof(float));
    float* q = (float*)malloc(qd * sizeof(float));
    float* k = (float*)malloc(kvd * sizeof(float));
    float* v = (float*)malloc(kvd * sizeof(float));
    float* tmp = (float*)malloc(hd * sizeof(float));
    float* attn = (float*)malloc(qd * sizeof(float));
    float* proj = (float*)malloc(h * sizeof(float));
    float* scores = (float*)malloc(seq_len * sizeof(float));
    float* gate = (float*)malloc((cfg->inter > inter ? cfg->inter : inter) * sizeof(float) + 4);
    float* up = (float*)malloc((cfg->inter > inter ? cfg->inter : inter) * sizeof(float) + 4);
    float* mlp = (float*)malloc(h * sizeof(float));
    int32_t ids[64];
    float wts[64];

    or_embed_v4(m->embed, h, token, residual);
    for (size_t li = 0; li < cfg->n_layers; li++) {
        const or_layer_v4* L = &m->layers[li];
        or_rms_norm(residual, L->input_ln, h, eps, normed);
        or_linear_v4_matvec(L->q, qd, h, normed, NULL, q, kernel, threads);
        or_linear_v4_matvec(L->k, kvd, h, normed, NULL, k, kernel, threads);
        or_linear_v4_matvec(L->v, kvd, h, normed, NULL, v, kernel, threads);
        for (size_t x = 0; x < nh; x++) {
            or_rms_norm(q + x * hd, L->q_norm, hd, eps, tmp);
            memcpy(q + x * hd, tmp, hd * sizeof(float));
        }
        for (size_t x = 0; x < nkv; x++) {
            or_rms_norm(k + x * hd, L->k_norm, hd, eps, tmp);
            memcpy(k + x * hd, tmp, hd * sizeof(float));
        }
        for (size_t x = 0; x < nh; x++) or_apply_rope(q + x * hd, hd, pos, cfg->rope_theta);
        for (size_t x = 0; x < nkv; x++) or_apply_rope(k + x * hd, hd, pos, cfg->rope_theta);
        for (size_t x = 0; x < nkv; x++) {
            size_t base = ((li * nkv + x) * cache->max_pos + pos) * hd;
            memcpy(cache->k + base, k + x * hd, hd * sizeof(float));
            memcpy(cache->v + base, v + x * hd, hd * sizeof(float));
        }
        float scale = 1.0f / sqrtf((float)hd);
        for (size_t qh = 0; qh < nh; qh++) {
            size_t kvh = qh / n_rep;
            const float* qv = q + qh * hd;
            const float* kc = cache->k + (li * nkv + kvh) * cache->max_pos * hd;
            const float* vc = cache->v + (li * nkv + kvh) * cache->max_pos * hd;
            for (size_t t = 0; t < seq_len; t++) {
                float dot = 0.0f;
                for (size_t d = 0; d < hd; d++) dot += qv[d] * kc[t * hd + d];
                scores[t] = dot * scale;
            }
            or_softmax_inplace(scores, seq_len);
            float* o = attn + qh * hd;
            for (size_t d = 0; d < hd; d++) o[d] = 0.0f;
            for (size_t t = 0; t < seq_len; t++) {
                float w = scores[t];
                for (size_t d = 0; d < hd; d++) o[d] += w * vc[t * hd + d];
            }
        }
        or_linear_v4_matvec(L->o, h, qd, attn, NULL, proj, kernel, threads);
        for (size_t i = 0; i < h; i++) residual[i] += proj[i];

        or_rms_norm(residual, L->post_ln, h, eps, normed);
        if (cfg->n_exp) {
            or_moe_ffn_v4(L->router, cfg->n_exp, h, cfg->moe_inter, cfg->top_k, cfg->norm_topk,
                          L->experts, normed, mlp, ids, wts, kernel, threads);
        } else {
            or_linear_v4_matvec(L->gate, cfg->inter, h, normed, NULL, gate, kernel, threads);
            or_linear_v4_matvec(L->up, cfg->inter, h, normed, NULL, up, kernel, threads);
            for (size_t i = 0; i < cfg->inter; i++) gate[i] = or_silu_mul(gate[i], up[i]);
            or_linear_v4_matvec(L->down, h, cfg->inter, gate, NULL, mlp, kernel, threads);
        }
        for (size_t i = 0; i < h; i++) residual[i] += mlp[i];
    }
    cache->len += 1;
    or_rms_norm(residual, m->final_norm, h, eps, normed);
    or_linear_v4_matvec(head, cfg->vocab, h, normed, NULL, logits, kernel, threads);

    free(residual); free(normed); free(q); free(k); free(v); free(tmp); free(attn);
    free(proj); free(scores); free(gate); free(up); free(mlp);
    return 0;
}
