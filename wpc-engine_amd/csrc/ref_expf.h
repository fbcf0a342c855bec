// expf with the exact results of the reference's f32::exp on its x86-64
// host: glibc's expf (2.35, FMA variant), which is the table method of ARM's
// optimized-routines:
//   k = round(x * 32/ln2), r = x*32/ln2 - k  (r from one fused multiply-add),
//   exp(x) = 2^(k/32) * P(r),  P(r) = 1 + C2 r + C1 r^2 + C0 r^3  (double),
// with the 32 table values 2^(i/32) rounded to double and the cubic's
// coefficients those of the published method. The result is not always
// the correctly rounded float (0.502 ulp), so a correctly rounded exp
// would differ on about 170000 inputs; this one matches on every float
// (tests/test_ref_expf.py compares it with the host's expf).
//
// Compiles as host C/C++ and as HIP device code (REF_EXPF_FN); needs IEEE
// double arithmetic and fma().
#pragma once
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifndef REF_EXPF_FN
#define REF_EXPF_FN static inline
#endif

// 2^(i/32), i = 0..31, rounded to nearest double.
#define REF_EXPF_TABLE \
    {0x1.0000000000000p+0, 0x1.059b0d3158574p+0, 0x1.0b5586cf9890fp+0, 0x1.11301d0125b51p+0, \
     0x1.172b83c7d517bp+0, 0x1.1d4873168b9aap+0, 0x1.2387a6e756238p+0, 0x1.29e9df51fdee1p+0, \
     0x1.306fe0a31b715p+0, 0x1.371a7373aa9cbp+0, 0x1.3dea64c123422p+0, 0x1.44e086061892dp+0, \
     0x1.4bfdad5362a27p+0, 0x1.5342b569d4f82p+0, 0x1.5ab07dd485429p+0, 0x1.6247eb03a5585p+0, \
     0x1.6a09e667f3bcdp+0, 0x1.71f75e8ec5f74p+0, 0x1.7a11473eb0187p+0, 0x1.82589994cce13p+0, \
     0x1.8ace5422aa0dbp+0, 0x1.93737b0cdc5e5p+0, 0x1.9c49182a3f090p+0, 0x1.a5503b23e255dp+0, \
     0x1.ae89f995ad3adp+0, 0x1.b7f76f2fb5e47p+0, 0x1.c199bdd85529cp+0, 0x1.cb720dcef9069p+0, \
     0x1.d5818dcfba487p+0, 0x1.dfc97337b9b5fp+0, 0x1.ea4afa2a490dap+0, 0x1.f50765b6e4540p+0}

// The same with the 32-entry table read from `tab` (e.g. a copy in GPU LDS,
// where a lookup is cheaper than a read of the constant array).
REF_EXPF_FN float ref_expf_tab(float x, const double* tab)
{
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    uint32_t ux;
    memcpy(&ux, &x, 4);
    if (((ux >> 20) & 0x7ff) >= 0x42b) {   // |x| >= 88, inf or nan
        if (ux == 0xff800000u) return 0.0f; // -inf
        if (((ux >> 20) & 0x7ff) >= 0x7f8) return x + x;  // +inf, nan
        if (x > 0x1.62e42ep6f) return (float)INFINITY;     // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;               // underflow
    }
    const double xd = (double)x;
    const double z = inv_ln2_32 * xd;
    double kd = z + shift;
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = fma(inv_ln2_32, xd, -kd);
    uint64_t t;
    memcpy(&t, &tab[ki & 31], 8);
    t += (ki >> 5) << 52;  // 2^(k/32) = 2^(k>>5) * 2^((k&31)/32)
    double s;
    memcpy(&s, &t, 8);
    const double p = fma(fma(c0, r, c1), r * r, fma(c2, r, 1.0));
    return (float)(p * s);
}

REF_EXPF_FN float ref_expf(float x)
{
    const double tab[32] = REF_EXPF_TABLE;
    return ref_expf_tab(x, tab);
}
