// kvd_exact.h -- integer building blocks shared by the exact-mode kernels.
// Same integer arithmetic as the exact islands (core/exact_islands/exact_islands.c:21-124);
// every function here is a deterministic integer map, so device results are
// bit-identical to the CPU arithmetic that defines them.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvd {
typedef __int128 i128;
typedef unsigned __int128 u128;

constexpr int FB = 30;
constexpr int64_t ONE = (int64_t)1 << FB;
constexpr int64_t LOG2E = 1549082005LL;                    // round(log2(e) * 2^30)
__device__ constexpr int64_t EXPC[7] = {1073741824LL, 744261118LL, 257941248LL, 59597083LL,
                                        10327387LL, 1431680LL, 165394LL};   // round((ln2)^k/k! * 2^30)
constexpr int64_t GK = 856722024LL;                        // round(sqrt(2/pi) * 2^30)
constexpr int64_t GA = 48012366LL;                         // round(0.044715 * 2^30)

__device__ __forceinline__ int64_t exp2_frac(int64_t r) {
    int64_t acc = EXPC[6];
    #pragma unroll
    for (int k = 5; k >= 0; k--) acc = ((acc * r) >> FB) + EXPC[k];
    return acc;
}
// e^d for d <= 0, Q30 in and out
__device__ __forceinline__ int64_t exp_fixed(int64_t d) {
    int64_t g = (int64_t)(-(((i128)d * LOG2E) >> FB));
    int64_t n = g >> FB, r = g - (n << FB);
    if (n >= 32) return 0;
    if (r) return exp2_frac(ONE - r) >> (n + 1);
    return ONE >> n;
}
// floor(sqrt(v)): double estimate, then exact integer correction (the result
// is the unique floor, identical to the bit-serial isqrt of the islands)
__device__ __forceinline__ uint64_t isqrt_u64(uint64_t v) {
    uint64_t x = (uint64_t)sqrt((double)v);
    if (x > 0xFFFFFFFFull) x = 0xFFFFFFFFull;
    while (x * x > v) x--;
    while ((x + 1) * (x + 1) <= v && x < 0xFFFFFFFFull) x++;
    return x;
}
// floor(num / den) for 0 <= num < 2^127, 0 < den < 2^63 with a quotient below
// 2^64: double estimate refined twice, then exact +-1 correction.  128-bit
// values go to double through their two 64-bit halves (one rounding each).
__device__ __forceinline__ double u128_to_double(u128 v) {
    return fma((double)(uint64_t)(v >> 64), 18446744073709551616.0, (double)(uint64_t)v);
}
__device__ __forceinline__ double i128_to_double(i128 v) {
    return fma((double)(int64_t)(v >> 64), 18446744073709551616.0, (double)(uint64_t)v);
}
__device__ __forceinline__ uint64_t udiv128_64(u128 num, uint64_t den) {
    if ((uint64_t)(num >> 64) >= den) return (uint64_t)(num / (u128)den);   // quotient >= 2^64: wraps like the cast
    const double dd = (double)den;
    uint64_t q = (uint64_t)fmin(u128_to_double(num) / dd, 1.8446744073709550e19);
    for (int it = 0; it < 2; it++) {
        const i128 r = (i128)num - (i128)((u128)q * den);
        q += (uint64_t)(int64_t)(i128_to_double(r) / dd);   // |step| <= q * 2^-51, wraps like the sum
    }
    i128 r = (i128)num - (i128)((u128)q * den);
    while (r < 0) { q--; r += den; }
    while (r >= (i128)den) { q++; r -= den; }
    return q;
}
// v mod m for v >= 0 (v < 2^100), 0 < m < 2^63: estimate the quotient in
// double, correct exactly
// isqrt(floor((n << 72) / ss)) for n > 0, ss > 0 -- the island's RMS inverse.
// While the quotient is below 2^64 this is the largest x with
// x^2 * ss <= n << 72 (floor(sqrt(floor(v))) = floor(sqrt(v))): a double
// estimate of sqrt((n << 72) / ss), off by at most one, corrected with exact
// 128-bit products.  Larger quotients wrap in the island's 64-bit cast, so
// they take the division and the integer square root of the wrapped value.
__device__ __forceinline__ int64_t rms_inv_q72(int n, int64_t ss) {
    const u128 num = (u128)(uint64_t)n << 72, den = (u128)(uint64_t)ss;
    if ((uint64_t)(num >> 64) >= (uint64_t)ss)
        return (int64_t)isqrt_u64(udiv128_64(num, (uint64_t)ss));
    uint64_t x = (uint64_t)sqrt(ldexp((double)n, 72) / (double)ss);
    if (x > 0xFFFFFFFFull) x = 0xFFFFFFFFull;
    while ((u128)(x * x) * den > num) x--;
    while (x < 0xFFFFFFFFull && (u128)((x + 1) * (x + 1)) * den <= num) x++;
    return (int64_t)x;
}
__device__ __forceinline__ int64_t umod128_64(i128 v, int64_t m) {
    const int64_t q = (int64_t)((double)v / (double)m);
    i128 r = v - (i128)q * m;
    while (r < 0) r += m;
    while (r >= m) r -= m;
    return (int64_t)r;
}
// low 64 bits of xi * inv * wi -- the island converts its 128-bit product with
// (int64_t), i.e. exactly this wrap-around value
__device__ __forceinline__ int64_t mul3_lo64(int64_t a, int64_t b, int64_t c) {
    return (int64_t)((uint64_t)a * (uint64_t)b * (uint64_t)c);
}
// floor(num / den) for 0 <= num < 2^62, 0 < den < 2^62 and a quotient below
// 2^31 (the islands' divisions): the double estimate is within one of it and
// is corrected exactly, in place of a generic 64/128-bit division routine.
__device__ __forceinline__ int64_t udiv_small(int64_t num, int64_t den) {
    int64_t q = (int64_t)((double)num / (double)den);
    int64_t r = num - q * den;
    while (r < 0) { q--; r += den; }
    while (r >= den) { q++; r -= den; }
    return q;
}
__device__ __forceinline__ int64_t tanh_fixed(int64_t t) {
    int s = (t >= 0) ? 1 : -1;
    int64_t a = (t >= 0) ? t : -t;
    int64_t e2 = exp_fixed(-(2 * a));
    int64_t num = (2 * e2) << FB;                  // <= 2^61, quotient <= 2^31
    return (int64_t)s * (ONE - udiv_small(num, ONE + e2));
}
// roundf (half away from zero) in three instructions instead of six: adding
// the float just below 1/2, with v's sign, and truncating gives roundf(v)
// bit for bit for every float (checked over all 2^32 bit patterns by the
// tests: no carry of the sum can round up a value below a half).
__device__ __forceinline__ float round_away(float v) { return truncf(v + copysignf(0x1.fffffep-2f, v)); }
// round half away from zero of a double to int64 (llround)
__device__ __forceinline__ int64_t llround_d(double d) { return (int64_t)round(d); }
// llround(x * 2^SH) of a float: x * 2^SH is exact in float short of overflow,
// roundf is exact, and results below 2^31 convert in 32 bits; anything else
// takes the double route.  The same value either way.
template <int SH> __device__ __forceinline__ int64_t llround_pow2(float x) {
    const float r = round_away(x * (float)(1 << SH));
    if (fabsf(r) < 2147483648.0f) return (int64_t)(int32_t)r;
    return llround_d((double)x * (double)(1 << SH));
}

__device__ __forceinline__ float gelu_exact1(float x) {
    int64_t xq = llround_pow2<16>(x);
    int64_t X = (xq * ONE) >> 16;
    i128 X2 = ((i128)X * X) >> FB;
    int64_t x3 = (int64_t)((X2 * X) >> FB);
    i128 inner = ((i128)GK * (X + (int64_t)(((i128)GA * x3) >> FB))) >> FB;
    int64_t t = tanh_fixed((int64_t)inner);
    int64_t g = (int64_t)(((i128)(X >> 1) * (ONE + t)) >> FB);
    return (float)((double)g / (double)ONE);
}
__device__ __forceinline__ float silu_exact1(float x) {
    int64_t xq = llround_pow2<16>(x);
    int64_t X = (xq * ONE) >> 16;
    int64_t e = exp_fixed(X >= 0 ? -X : X);
    int64_t sg = X >= 0 ? udiv_small(ONE << FB, ONE + e)          // 2^60 / [2^30, 2^31]
                        : udiv_small(e << FB, ONE + e);
    int64_t g = (int64_t)(((i128)X * sg) >> FB);
    return (float)((double)g / (double)ONE);
}

// Round-to-nearest-even of (mag * 2^k) to float, mag > 0.  Exact for every
// input (normal, subnormal, overflow to inf): the one rounding primitive of
// exact mode.  Any correct RNE gives the same bits, so this matches the CPU.
__device__ __forceinline__ float rne_u128_scaled(u128 mag, int k) {
    if (!mag) return 0.0f;
    uint64_t hi = (uint64_t)(mag >> 64), lo = (uint64_t)mag;
    int msb = hi ? 127 - __builtin_clzll(hi) : 63 - __builtin_clzll(lo);
    int e = msb + k;
    int keep = 24;
    if (e < -126) keep = 24 - (-126 - e);
    if (keep <= 0) {
        if (keep == 0) return (mag == ((u128)1 << msb)) ? 0.0f : 0x1.0p-149f;
        return 0.0f;
    }
    int drop = msb + 1 - keep;
    uint32_t q;
    if (drop > 0) {
        u128 qq = mag >> drop;
        u128 rem = mag & (((u128)1 << drop) - 1u), half = (u128)1 << (drop - 1);
        if (rem > half || (rem == half && (qq & 1u))) qq++;
        q = (uint32_t)qq;
    } else {
        q = (uint32_t)(mag << (-drop));
    }
    return ldexpf((float)q, k + drop);
}
__device__ __forceinline__ float rne_i128_scaled(i128 v, int k) {
    return v >= 0 ? rne_u128_scaled((u128)v, k) : -rne_u128_scaled((u128)(-v), k);
}
__device__ __forceinline__ float rne_i64_scaled(int64_t v, int k) {
    return v >= 0 ? rne_u128_scaled((u128)(uint64_t)v, k) : -rne_u128_scaled((u128)(uint64_t)(-v), k);
}
// RNE of num / (den * 2^k), den > 0
__device__ __forceinline__ int bitlen128(u128 v) {
    uint64_t hi = (uint64_t)(v >> 64), lo = (uint64_t)v;
    return hi ? 128 - __builtin_clzll(hi) : (lo ? 64 - __builtin_clzll(lo) : 0);
}
__device__ __forceinline__ float rne_div_to_float(i128 num, int64_t den, int k) {
    if (!num) return 0.0f;
    // Fast path: with both operands below 2^53 the double quotient is the
    // correctly rounded exact one, and scaling by 2^-k is exact; it rounds to
    // the float the exact quotient rounds to unless it lies exactly on a float
    // rounding midpoint (low 29 mantissa bits 1000...0) -- then, and for
    // results outside the normal float range, the exact path below decides.
    if (num > -((i128)1 << 53) && num < ((i128)1 << 53) && den < ((int64_t)1 << 53) && k >= 0 && k < 64) {
        const double q = ldexp((double)(int64_t)num / (double)den, -k);
        const uint64_t b = (uint64_t)__double_as_longlong(q);
        const int ex = (int)((b >> 52) & 0x7FF) - 1023;
        if (ex >= -126 && ex < 128 && (b & 0x1FFFFFFFull) != 0x10000000ull) return (float)q;
    }
    bool neg = num < 0;
    u128 n = neg ? (u128)(-num) : (u128)num, d = (u128)(uint64_t)den;
    int sh = 28 + bitlen128(d) - bitlen128(n);
    if (sh < 0) sh = 0;
    n <<= sh;
    u128 q, r;
    if ((uint64_t)(n >> 64) < (uint64_t)den) {            // quotient fits 64 bits: fast path
        // a quotient below 2^52 (the usual case: n is scaled to ~2^29 d) is the
        // double estimate (within 2) corrected exactly; larger ones refine
        const double qe = u128_to_double(n) / (double)den;
        if (qe < 4503599627370496.0) {
            uint64_t q64 = (uint64_t)qe;
            i128 rr = (i128)n - (i128)((u128)q64 * d);
            while (rr < 0) { q64--; rr += (i128)d; }
            while (rr >= (i128)d) { q64++; rr -= (i128)d; }
            q = q64; r = (u128)rr;
        } else {
            q = udiv128_64(n, (uint64_t)den); r = n - q * d;
        }
    } else { q = n / d; r = n % d; }
    q = (q << 1) | (r ? 1u : 0u);
    float f = rne_u128_scaled(q, -(k + sh + 1));
    return neg ? -f : f;
}
}  // namespace kvd
