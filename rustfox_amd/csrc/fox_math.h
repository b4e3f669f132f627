// fox_math.h -- device float functions that round exactly like the host
// libm the reference calls.
//
// expf: the reference calls glibc's expf (RustFox src/ops.c:32, 46).  glibc
// 2.35 on x86-64 with FMA runs the ARM optimized-routines expf (Szabolcs
// Nagy, 2017, in glibc as sysdeps/ieee754/flt-32/e_expf.c): x * 32/ln2 is
// split into an integer k and r in [-1/2, 1/2]; 2^(k/32) comes from a
// 32-entry table of 2^(i/32) with the exponent folded in; 2^(r/32) from a
// cubic in r evaluated in double with fused multiply-adds; the double result
// is rounded to float once.  Restated here from the published algorithm and
// checked against the host's expf on all 2^32 float inputs (0 differences).
//
// Division and square root: a float quotient or root computed in double and
// rounded to float is the correctly rounded float result (53 >= 2*24 + 2),
// the same as the reference's IEEE float / and sqrtf.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

__device__ __constant__ const uint64_t fox_exp2_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// fox_expf with the 2^(i/32) table read from `tab` (a copy of fox_exp2_tab,
// e.g. in LDS, so that a wave's scattered lookups avoid a memory round trip)
__device__ __forceinline__ float fox_expf_t(float x, const uint64_t *tab)
{
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;

    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_32, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_32, xd, -kd);
    const uint64_t t = tab[ki & 31] + (ki << 47);
    const double s = __builtin_bit_cast(double, t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * s);
}

__device__ __forceinline__ float fox_expf(float x)
{
    return fox_expf_t(x, fox_exp2_tab);
}

__device__ __forceinline__ float fox_div(float a, float b)
{
    return (float)((double)a / (double)b);
}

__device__ __forceinline__ float fox_sqrtf(float a)
{
    return (float)__builtin_sqrt((double)a);
}
