/* f16.c -- IEEE binary16 <-> binary32 on the host (include/fox/fox.h:357-358).
 *
 * fox_f16_to_f32 is exact.  fox_f32_to_f16 follows RustFox's encoder
 * (src/kernels.c:41-74): round to nearest even while the result is normal,
 * round half up (away from zero in magnitude) when it is subnormal, a signed
 * zero below 2^-25, infinity at and above 65520 after rounding, and the
 * quiet NaN 0x7E00 (sign kept, payload dropped) for every NaN.
 */
#include "fox_host_internal.h"

#include <string.h>

static uint32_t bits_of(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float float_of(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float fox_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1F) return float_of(sign | 0x7F800000u | (m << 13));   /* inf, NaN payload */
    if (e != 0) return float_of(sign | ((e + 112u) << 23) | (m << 13));
    /* zero and subnormals: m * 2^-24, exact in binary32 */
    {
        const float mag = (float)m * float_of(0x33800000u);            /* 2^-24 */
        return float_of(sign | bits_of(mag));
    }
}

uint16_t fox_f32_to_f16(float f)
{
    const uint32_t u = bits_of(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t be = (u >> 23) & 0xFFu, frac = u & 0x7FFFFFu;
    const int e = (int)be - 112;                   /* the half's biased exponent */
    if (be == 0xFF) return (uint16_t)(sign | (frac ? 0x7E00u : 0x7C00u));
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e >= 1) {
        /* 13 bits dropped, ties to the even result; a carry out of the
         * fraction moves into the exponent (up to infinity) */
        const uint32_t kept = frac >> 13, rest = frac & 0x1FFFu;
        uint32_t out = ((uint32_t)e << 10) | kept;
        if (rest > 0x1000u || (rest == 0x1000u && (kept & 1u))) out++;
        return (uint16_t)(sign | out);
    }
    if (e < -10) return sign;
    /* subnormal result: the significand with its leading one, shifted right
     * 14 - e places, a half or more rounding up */
    {
        const uint32_t sig = frac | 0x800000u;
        const int sh = 14 - e;
        return (uint16_t)(sign | ((sig >> sh) + ((sig >> (sh - 1)) & 1u)));
    }
}
