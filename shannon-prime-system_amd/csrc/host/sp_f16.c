/* sp_f16.c -- IEEE binary16 <-> binary32 by bit manipulation.
 * Semantics of core/weight_dtype/weight_dtype.c:9-53: subnormal halves are
 * normalised on widening, NaN payloads shifted (not quieted); narrowing rounds
 * to nearest-even, overflows to inf, flushes below the smallest subnormal. */
#include "sp_model_abi.h"
#include <string.h>

float sp_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u, m = h & 1023u, bits;
    if (e == 31u) {
        bits = s | 0x7F800000u | (m << 13);
    } else if (e) {
        bits = s | ((e + 112u) << 23) | (m << 13);
    } else if (!m) {
        bits = s;
    } else {                      /* subnormal: value = m * 2^-24, renormalise */
        int sh = 0;
        while (!(m & 1024u)) { m <<= 1; sh++; }
        bits = s | ((uint32_t)(113 - sh) << 23) | ((m & 1023u) << 13);
    }
    float f; memcpy(&f, &bits, 4); return f;
}

uint16_t sp_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t s = (x >> 16) & 0x8000u, e8 = (x >> 23) & 255u, m = x & 0x7FFFFFu;
    if (e8 == 255u) return (uint16_t)(s | 0x7C00u | (m ? 0x200u : 0u));
    int e = (int)e8 - 112;                     /* rebias 127 -> 15 */
    if (e >= 31) return (uint16_t)(s | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)s;
        uint32_t full = m | 0x800000u;
        int sh = 14 - e;                       /* 14..24 */
        uint32_t q = full >> sh, r = full & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (r > half || (r == half && (q & 1u))) q++;
        return (uint16_t)(s | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (m >> 13), r = m & 0x1FFFu;
    if (r > 0x1000u || (r == 0x1000u && (q & 1u))) q++;   /* carry may ripple into exponent */
    return (uint16_t)(s | q);
}
