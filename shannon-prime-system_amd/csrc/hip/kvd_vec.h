// kvd_vec.h -- per-vector device building blocks shared by the GEMV and the
// batched prefill kernels: block reductions, RMSNorm (float and exact island),
// the GEMV input transform, f16 scale parts, FFN activations.
#pragma once
#include "kvd_internal.h"
#include "kvd_exact.h"

namespace kvd {

// ---------------------------------------------------------------- reductions
template <typename T> __device__ __forceinline__ T wave_sum(T v) {
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ i128 wave_sum128(i128 v) {
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint64_t lo = (uint64_t)v, hi = (uint64_t)((u128)v >> 64);
        uint64_t lo2 = __shfl_xor(lo, o, 64), hi2 = __shfl_xor(hi, o, 64);
        v += (i128)(((u128)hi2 << 64) | lo2);
    }
    return v;
}
// Wave reductions to lane 63 through DPP (no LDS round trips): pair and quad
// swaps, the half-row and row mirrors leave each 16-lane row's total in all of
// its lanes, then row_bcast15 / row_bcast31 fold rows 0+1 and 2+3 and then
// both halves into lane 63.  `ident` is what lanes outside a broadcast's row
// mask add.
template <int CTRL, int RMASK> __device__ __forceinline__ uint32_t dpp32(uint32_t v, uint32_t old) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, RMASK, 0xF, false);
}
template <int CTRL, int RMASK> __device__ __forceinline__ uint64_t dpp64(uint64_t v, uint64_t old) {
    return ((uint64_t)dpp32<CTRL, RMASK>((uint32_t)(v >> 32), (uint32_t)(old >> 32)) << 32) |
           dpp32<CTRL, RMASK>((uint32_t)v, (uint32_t)old);
}
template <typename T, typename Op> __device__ __forceinline__ T wave_to63(T v, T ident, Op op) {
    typedef typename std::conditional<sizeof(T) == 8, uint64_t, uint32_t>::type B;
    auto mv = [&](auto ctrl_tag, T x) -> T {
        constexpr int C = decltype(ctrl_tag)::value >> 4, M = decltype(ctrl_tag)::value & 15;
        if constexpr (sizeof(T) == 8) return __builtin_bit_cast(T, dpp64<C, M>(__builtin_bit_cast(B, x), __builtin_bit_cast(B, ident)));
        else return __builtin_bit_cast(T, dpp32<C, M>(__builtin_bit_cast(B, x), __builtin_bit_cast(B, ident)));
    };
    v = op(v, mv(std::integral_constant<int, (0xB1 << 4) | 0xF>{}, v));     // quad_perm 1,0,3,2
    v = op(v, mv(std::integral_constant<int, (0x4E << 4) | 0xF>{}, v));     // quad_perm 2,3,0,1
    v = op(v, mv(std::integral_constant<int, (0x141 << 4) | 0xF>{}, v));    // row_half_mirror
    v = op(v, mv(std::integral_constant<int, (0x140 << 4) | 0xF>{}, v));    // row_mirror
    v = op(v, mv(std::integral_constant<int, (0x142 << 4) | 0xA>{}, v));    // row_bcast15 -> rows 1, 3
    v = op(v, mv(std::integral_constant<int, (0x143 << 4) | 0xC>{}, v));    // row_bcast31 -> rows 2, 3
    return v;
}

// All-lane results: the lane-63 total read back as a wave-uniform value.
template <typename T> __device__ __forceinline__ T bcast63(T v) {
    if constexpr (sizeof(T) == 8) {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
        return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    } else {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    }
}
template <typename T> __device__ __forceinline__ T wave_allsum(T v) {
    return bcast63(wave_to63(v, (T)0, [](T a, T b) { return a + b; }));
}
__device__ __forceinline__ float wave_allmax(float v) {
    return bcast63(wave_to63(v, -INFINITY, [](float a, float b) { return fmaxf(a, b); }));
}
__device__ __forceinline__ int wave_allmax_i(int v) {
    return bcast63(wave_to63(v, (int)INT32_MIN, [](int a, int b) { return a > b ? a : b; }));
}
// Sum over the 4 lanes of each quad (all four get it): two DPP quad swaps.
template <typename T> __device__ __forceinline__ T quad_sum(T v) {
    typedef typename std::conditional<sizeof(T) == 8, uint64_t, uint32_t>::type B;
    auto sw = [](T x, auto ctrl_tag) -> T {
        constexpr int C = decltype(ctrl_tag)::value;
        if constexpr (sizeof(T) == 8) return __builtin_bit_cast(T, dpp64<C, 0xF>(__builtin_bit_cast(B, x), 0));
        else return __builtin_bit_cast(T, dpp32<C, 0xF>(__builtin_bit_cast(B, x), 0));
    };
    v = v + sw(v, std::integral_constant<int, 0xB1>{});      // quad_perm 1,0,3,2
    return v + sw(v, std::integral_constant<int, 0x4E>{});   // quad_perm 2,3,0,1
}
// Sum over aligned groups of N = 4 or 8 lanes (all lanes of a group get it):
// after the quad sums, the half-row mirror pairs each quad with the other
// quad of its 8 lanes.
template <int N, typename T> __device__ __forceinline__ T group_sum(T v) {
    static_assert(N == 4 || N == 8, "groups of 4 or 8 lanes");
    typedef typename std::conditional<sizeof(T) == 8, uint64_t, uint32_t>::type B;
    v = quad_sum(v);
    if constexpr (N == 8) {
        if constexpr (sizeof(T) == 8) v = v + __builtin_bit_cast(T, dpp64<0x141, 0xF>(__builtin_bit_cast(B, v), 0));
        else v = v + __builtin_bit_cast(T, dpp32<0x141, 0xF>(__builtin_bit_cast(B, v), 0));
    }
    return v;
}

// Block-wide reductions through one LDS slot array per reduction: lane 63 of
// each wave posts its wave total, one barrier, every thread combines the
// totals.  A reduction writes only its own `red` slots, so consecutive
// reductions need no barrier in between; a slot array is used once per launch.
constexpr int RED_WAVES = 16;                 // slots per reduction (waves per workgroup)
constexpr int RED_SLOTS = 4;                  // reductions per input transform
template <typename T> __device__ T block_sum(T v, T *red) {
    v = wave_to63(v, (T)0, [](T a, T b) { return a + b; });
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 63) red[w] = v;
    __syncthreads();
    T t = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) t += red[i];
    return t;
}
__device__ float block_max(float v, float *red) {
    v = wave_to63(v, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 63) red[w] = v;
    __syncthreads();
    float t = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) t = fmaxf(t, red[i]);
    return t;
}
// slot k of a RED_SLOTS x RED_WAVES x 8-byte reduction scratch
__device__ __forceinline__ void *red_slot(void *red, int k) { return (uint8_t *)red + (size_t)k * RED_WAVES * 8; }

// ------------------------------------------------------- RMSNorm (both modes)
// Float mode: core/forward_kernels/forward_kernels.c:17-22 (sum of squares in
// double, 1/sqrtf((float)(ss/n)+eps), out = x*scale*w).  Exact mode: the
// integer island core/exact_islands/exact_islands.c:60-79 (no eps).
struct NormScale { float f; int64_t inv; double invd; int zero; };
constexpr int SH_ZERO_V = -1000000;       // grid exponent of an all-zero vector

// One thread's share of a sum of squares: double in float mode, the exact
// int64 sum of the Q16 values in exact mode.
__device__ __forceinline__ int64_t llround_q16(float x) { return llround_pow2<16>(x); }
struct SumSq {
    double f = 0.0; int64_t i = 0;
    __device__ __forceinline__ void add(float v, int mode) {
        if (mode == FLOAT) { f += (double)v * (double)v; return; }
        // llround(v * 2^16): roundf of the exact float product is that integer;
        // below 2^31 its square is one 32 x 32 -> 64 multiply
        const float r = round_away(v * 65536.0f);
        if (fabsf(r) < 2147483648.0f) { const int32_t q = (int32_t)r; i += (int64_t)q * q; }
        else { const int64_t q = llround_q16(v); i += q * q; }
    }
};
// A producer statistic (VecStat) is kept in STAT_REP replicas so that the
// atomics of many workgroups spread over addresses: a thread accumulates the
// values it writes (StatAcc: llround(v 2^16)^2 -- the consumer's exact sum of
// squares -- and max |v|, NaN adding nothing as in the consumer's fmaxf scan),
// the workgroup combines its threads, and one atomic of each kind goes to
// replica blockIdx.x % STAT_REP.  The consumer sums / maxes the replicas.
struct StatAcc {
    int64_t q2 = 0;
    float mx = 0.0f;
    __device__ __forceinline__ void add(float v) {
        const float r = round_away(v * 65536.0f);
        if (fabsf(r) < 2147483648.0f) { const int32_t q = (int32_t)r; q2 += (int64_t)q * q; }
        else { const int64_t q = llround_q16(v); q2 += q * q; }
        mx = fmaxf(mx, fabsf(v));
    }
};
// Every thread of the workgroup calls this (it has a barrier).
__device__ __forceinline__ void stat_flush_block(VecStat *slot, StatAcc acc) {
    __shared__ int64_t sq[RED_WAVES];
    __shared__ float sm[RED_WAVES];
    const int64_t q2 = wave_to63(acc.q2, (int64_t)0, [](int64_t a, int64_t b) { return a + b; });
    const float mx = wave_to63(acc.mx, 0.0f, [](float a, float b) { return fmaxf(a, b); });
    if ((threadIdx.x & 63) == 63) { sq[threadIdx.x >> 6] = q2; sm[threadIdx.x >> 6] = mx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t t = sq[0];
        float m = sm[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) { t += sq[w]; m = fmaxf(m, sm[w]); }
        VecStat *r = slot + blockIdx.x % STAT_REP;
        if (t) atomicAdd(&r->ss, (unsigned long long)t);
        atomicMax(&r->maxbits, __float_as_uint(m));
    }
}
// A statistic is read in two steps so that its loads can be issued early:
// stat_load gives lane l < STAT_REP replica l's values, stat_reduce the
// totals over the replicas, uniform across the wave.
// (stat_load reads replica lane % STAT_REP on every lane, unconditionally, so
// that nothing waits for the values before stat_reduce masks the copies, and
// only the fields asked for: an unused load would still occupy its register.)
template <bool SS = true, bool MAX = true>
__device__ __forceinline__ void stat_load(const VecStat *slot, int64_t &q, float &m) {
    const int r = threadIdx.x & (STAT_REP - 1);
    q = SS ? (int64_t)ld_agent(&slot[r].ss) : 0;
    m = MAX ? __uint_as_float(ld_agent(&slot[r].maxbits)) : 0.0f;
}
__device__ __forceinline__ void stat_reduce(int64_t q, float m, int64_t &ss, float &mx) {
    if ((threadIdx.x & 63) >= STAT_REP) { q = 0; m = 0.0f; }
    q = wave_to63(q, (int64_t)0, [](int64_t a, int64_t b) { return a + b; });
    m = wave_to63(m, 0.0f, [](float a, float b) { return fmaxf(a, b); });
    const uint64_t qu = (uint64_t)q;
    ss = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(qu >> 32), 63) << 32) |
                   (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)qu, 63));
    mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 63));
}
// The exact-mode RMS scale of a vector whose sum of squares a producer accumulated
// rms_inv_q72 of a workgroup-uniform sum of squares (0 for ss == 0), formed by
// wave 0 alone and handed to the other waves through the LDS slot: the exact
// inverse (double divide and square root, 128-bit corrections: a few hundred
// instructions) would otherwise run once per wave, on SIMDs that several
// waves share.  Every thread of the workgroup calls this (it has a barrier);
// each call site has a slot of its own.
__device__ __forceinline__ int64_t rms_inv_wg(int n, int64_t ss, int64_t *slot) {
    if (threadIdx.x < 64) {
        const int64_t v = ss ? rms_inv_q72(n, ss) : 0;
        if (threadIdx.x == 0) *slot = v;
    }
    __syncthreads();
    return *slot;
}
__device__ __forceinline__ NormScale stat_scale(int64_t ss, int n, int64_t *slot) {
    NormScale s; s.f = 0.0f; s.inv = 0; s.invd = 0.0; s.zero = ss == 0;
    s.inv = rms_inv_wg(n, ss, slot);
    s.invd = (double)s.inv;
    return s;
}
__device__ __forceinline__ int sh_of_max(float m) {
    if (m == 0.0f) return SH_ZERO_V;
    int e; frexpf(m, &e);
    return 22 - e;
}

// slot: an LDS int64 of the call site's own (exact mode's broadcast inverse)
__device__ NormScale norm_finish(const SumSq &p, int n, float eps, int mode, void *red, int64_t *slot) {
    NormScale s; s.f = 0.0f; s.inv = 0; s.invd = 0.0; s.zero = 0;
    if (mode == FLOAT) {
        const double ss = block_sum<double>(p.f, (double *)red);
        s.f = 1.0f / sqrtf((float)(ss / n) + eps);
    } else {
        const int64_t ss = block_sum<int64_t>(p.i, (int64_t *)red);
        s.zero = ss == 0;
        s.inv = rms_inv_wg(n, ss, slot);
        s.invd = (double)s.inv;                       // inv < 2^43: exact
    }
    return s;
}
// Exact mode: the island's (int64)(xi * inv * wi) / 2^52 rounded to float.
// With xi = llround(x 2^16), wi = llround(w 2^16): xi * wi is exact in double
// below 2^53, and the double product with inv is then the double nearest the
// exact integer product -- the island's int64 -> double conversion -- as long
// as that product does not wrap (|product| < 2^62 checked); otherwise the
// 64-bit integer path.
__device__ __forceinline__ float norm_apply(float x, float w, const NormScale &s, int mode) {
    if (mode == FLOAT) return x * s.f * w;
    if (s.zero) return 0.0f;
    const double dx = (double)round_away(x * 65536.0f) * (double)round_away(w * 65536.0f);
    if (fabs(dx) < 9007199254740992.0) {              // 2^53
        const double pr = dx * s.invd;
        if (fabs(pr) < 4611686018427387904.0)          // 2^62
            return (float)(pr * 2.220446049250313e-16);  // 2^-52
    }
    const int64_t xi = llround_q16(x), wi = llround_q16(w);
    return (float)((double)mul3_lo64(xi, s.inv, wi) / 4503599627370496.0);   // 2^52
}
// norm_apply with the weight given as its Q16 integer w16 = round_away(w * 2^16)
// (exact mode; the same value: llround_q16(w) is that integer)
__device__ __forceinline__ float norm_apply_q16(float x, float w16, const NormScale &s) {
    if (s.zero) return 0.0f;
    const double dx = (double)round_away(x * 65536.0f) * (double)w16;
    if (fabs(dx) < 9007199254740992.0) {              // 2^53
        const double pr = dx * s.invd;
        if (fabs(pr) < 4611686018427387904.0)          // 2^62
            return (float)(pr * 2.220446049250313e-16);  // 2^-52
    }
    const int64_t xi = llround_q16(x), wi = llround_d((double)w16);
    return (float)((double)mul3_lo64(xi, s.inv, wi) / 4503599627370496.0);   // 2^52
}
// a weight pro_load loaded: the Q16 half in exact mode, w itself in float mode
__device__ __forceinline__ float norm_apply_loaded(float x, float wl, const NormScale &s, int mode) {
    return mode == EXACT ? norm_apply_q16(x, wl, s) : norm_apply(x, wl, s, mode);
}

// ------------------------------------------------------- input transform
// Latency matters more than work here (every GEMV workgroup runs it before its
// matrix pass), so every pass over the vector issues its loads before using
// any of them, and independent passes are fused: the residual pass also sums
// the squares for the next norm, the last norm pass also takes the maximum.
constexpr int SH_ZERO = SH_ZERO_V;
constexpr int PB = 8;
constexpr int PB4 = 2;          // float4 loads per thread and array on the register path (n <= 4 * PB4 * T)

// The global-memory inputs of the input transform, loaded by pro_load before
// anything else the kernel requests: vector-memory loads complete in order, so
// waiting for a value requested after a weight prefetch waits for the
// prefetch too.  Register path only (n <= 4 * PB4 * T); the loop path for
// longer vectors loads as it goes.
struct ProLoads {
    float4 xv[PB4], dv[PB4], pw[PB4], nw[PB4];
    int64_t sq;                 // this lane's replica of the producer's statistic
    float sm;
};
template <int PRO>
__device__ __forceinline__ bool pro_uses_stat(const ProArgs &p, int mode) {
    return p.stat && (PRO == PRO_PLAIN || (PRO == PRO_RESID && p.post_w && mode == EXACT));
}
template <int PRO>
__device__ __forceinline__ void pro_load(const ProArgs &p, int mode, ProLoads &L) {
    const int n = p.n, T = blockDim.x, tid = threadIdx.x;
    // PRO_PLAIN takes the maximum, PRO_RESID the sum of squares
    if (pro_uses_stat<PRO>(p, mode)) stat_load<PRO != PRO_PLAIN, PRO == PRO_PLAIN>(p.stat, L.sq, L.sm);
    if (PRO == PRO_PLAIN || n > 4 * PB4 * T) return;
    // every load reads a valid address (a lane past the end re-reads element
    // 0, a missing post_w reads x); input_transform masks the values when it
    // uses them -- masking here would wait for the loads at once, and a select
    // between loads would become a load through a selected pointer
    // exact mode: the weights' Q16 halves (round_away(w * 2^16) as floats)
    const int wq = mode == EXACT ? n : 0;
    const float *pwp = p.post_w ? p.post_w + wq : p.x;
    #pragma unroll
    for (int k = 0; k < PB4; k++) {
        const int i = 4 * (k * T + tid);
        const int ic = i < n ? i : 0;                    // n is a multiple of 4
        L.xv[k] = *(const float4 *)(p.x + ic);
        L.nw[k] = *(const float4 *)(p.norm_w + wq + ic);
        if constexpr (PRO == PRO_RESID) {
            L.dv[k] = *(const float4 *)(p.delta + ic);
            L.pw[k] = *(const float4 *)(pwp + ic);
        }
    }
}
__device__ __forceinline__ float f4c(const float4 &v, int c) { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; }
__device__ __forceinline__ void f4s(float4 &v, int c, float x) { if (c == 0) v.x = x; else if (c == 1) v.y = x; else if (c == 2) v.z = x; else v.w = x; }

// The GEMV input transform of one vector by one workgroup: residual add (+
// sandwich norm of the branch), RMSNorm, and the grid exponent
// sh = 22 - frexp_exponent(max |x|) of the result (SH_ZERO for an all-zero
// vector).  The result is left in xf (LDS, n floats), or read from p.x for
// PRO_PLAIN.  x_out (the updated residual) is written when write_x is set.
// red: RED_SLOTS x RED_WAVES x 8 bytes of LDS, used once per launch.
// L: what pro_load<PRO> loaded for the same p and mode.
// [c_lo, c_hi): the columns of xf the caller reads (the exact residual path
// forms only those; every other path writes the whole vector).
// The GEMV's digit planes (six balanced base-16 planes of rne(y 2^sh), 8
// columns per dword, dig[plane * nb + block - b_lo]): the exact residual path
// writes them itself, straight from its registers, when a caller passes one
// (and sets done); the caller forms them otherwise.
struct DigOut { uint4 *dig; int b_lo, nb; bool done; };
// 4 consecutive columns' planes as 16-bit halves (nibble j = column j): byte
// b of the even and of the odd columns gathered by v_perm_b32, then the low
// nibbles of E | O << 4 are plane 2b and the high nibbles plane 2b + 1;
// h[k] = plane k.
__device__ __forceinline__ void digits4(const float y[4], int sh, uint32_t h[6]) {
    uint32_t u[4];
    #pragma unroll
    for (int j = 0; j < 4; j++) u[j] = (uint32_t)((int32_t)rintf(ldexpf(y[j], sh)) + 0x888888);
    const uint32_t e01 = __builtin_amdgcn_perm(u[2], u[0], 0x05010400u), o01 = __builtin_amdgcn_perm(u[3], u[1], 0x05010400u);
    const uint32_t e2 = __builtin_amdgcn_perm(u[2], u[0], 0x0C0C0602u), o2 = __builtin_amdgcn_perm(u[3], u[1], 0x0C0C0602u);
    const uint32_t l01 = ((e01 & 0x0F0F0F0Fu) | ((o01 << 4) & 0xF0F0F0F0u)) ^ 0x88888888u;
    const uint32_t h01 = (((e01 >> 4) & 0x0F0F0F0Fu) | (o01 & 0xF0F0F0F0u)) ^ 0x88888888u;
    const uint32_t l2 = ((e2 & 0x0F0F0F0Fu) | ((o2 << 4) & 0xF0F0F0F0u)) ^ 0x88888888u;
    const uint32_t h2 = (((e2 >> 4) & 0x0F0F0F0Fu) | (o2 & 0xF0F0F0F0u)) ^ 0x88888888u;
    h[0] = l01 & 0xFFFFu; h[1] = h01 & 0xFFFFu; h[2] = l01 >> 16; h[3] = h01 >> 16; h[4] = l2 & 0xFFFFu; h[5] = h2 & 0xFFFFu;
}

template <int PRO>
__device__ int input_transform(const ProArgs &p, int mode, const ProLoads &L, float *xf, void *red, bool write_x,
                               int c_lo = 0, int c_hi = 0x7FFFFFFF, DigOut *dout = nullptr) {
    const int n = p.n, T = blockDim.x, tid = threadIdx.x;
    __shared__ int64_t bcs[2];                       // broadcast RMS inverses: branch norm, pre-norm
    float m = 0.0f;
    if constexpr (PRO == PRO_PLAIN) {
        // the producer's maximum: no pass over the vector here (callers read
        // only the columns they need)
        if (p.stat) { int64_t ss; float mx; stat_reduce(L.sq, L.sm, ss, mx); return sh_of_max(mx); }
        for (int base = 0; base < n; base += PB * T) {
            float a[PB];
            #pragma unroll
            for (int k = 0; k < PB; k++) { const int i = base + k * T + tid; a[k] = p.x[i < n ? i : 0]; }
            #pragma unroll
            for (int k = 0; k < PB; k++) m = fmaxf(m, fabsf(a[k]));     // a re-read x[0] changes no maximum
        }
    } else if (n <= 4 * PB4 * T) {
        // whole vector in registers (loaded by pro_load): only reductions here;
        // lanes past the end hold copies of element 0 and are zeroed
        const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float4 xv[PB4], dv[PB4], pw[PB4], nw[PB4];
        #pragma unroll
        for (int k = 0; k < PB4; k++) {
            const bool ok = 4 * (k * T + tid) < n;
            xv[k] = ok ? L.xv[k] : z;
            nw[k] = ok ? L.nw[k] : z;
            dv[k] = (PRO == PRO_RESID && ok) ? L.dv[k] : z;
            pw[k] = (PRO == PRO_RESID && ok && p.post_w) ? L.pw[k] : z;
        }
        if constexpr (PRO == PRO_RESID) {
            NormScale sd; sd.f = 0.0f; sd.inv = 0; sd.invd = 0.0; sd.zero = 0;
            if (pro_uses_stat<PRO>(p, mode)) {
                int64_t ss; float mx;
                stat_reduce(L.sq, L.sm, ss, mx);             // the producer's exact sum of squares
                sd = stat_scale(ss, n, &bcs[0]);
            } else if (p.post_w) {
                SumSq q;
                #pragma unroll
                for (int k = 0; k < PB4; k++)
                    if (4 * (k * T + tid) < n)
                        #pragma unroll
                        for (int c = 0; c < 4; c++) q.add(f4c(dv[k], c), mode);
                sd = norm_finish(q, n, p.eps, mode, red_slot(red, 0), &bcs[0]);
            }
            const bool wr = write_x && p.x_out;
            if (mode == EXACT) {
                // The residual add and the statistics of the exact norm of the
                // result in one pass: the sum of squares of the Q16 values and
                // the largest exact product |llround(r 2^16) * llround(w 2^16)|.
                // Branch-free for inputs on the norms' double paths (products
                // below 2^53, scaled below 2^62, Q16 values below 2^31); a
                // thread with any other element redoes its elements with the
                // general per-element arithmetic (same results).
                int64_t ss = 0;
                double pm = 0.0;
                const bool pn = p.post_w != nullptr;
                bool bad = false;
                #pragma unroll
                for (int k = 0; k < PB4; k++)
                    #pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const float d = f4c(dv[k], c);
                        float nd = d;
                        if (pn) {
                            const double dx = (double)round_away(d * 65536.0f) * (double)f4c(pw[k], c);
                            const double pr = dx * sd.invd;
                            bad |= !(fabs(dx) < 9007199254740992.0) | !(fabs(pr) < 4611686018427387904.0);
                            nd = sd.zero ? 0.0f : (float)(pr * 2.220446049250313e-16);
                        }
                        const float r = f4c(xv[k], c) + nd;
                        f4s(xv[k], c, r);
                        const float r16 = round_away(r * 65536.0f), w16 = f4c(nw[k], c);
                        bad |= !(fabsf(r16) < 2147483648.0f);
                        const int32_t q = (int32_t)r16;
                        ss += (int64_t)q * q;
                        const double dx2 = fabs((double)r16 * (double)w16);
                        bad |= !(dx2 < 9007199254740992.0);
                        pm = fmax(pm, dx2);
                    }
                if (bad) {
                    // (a rolled loop over reloaded inputs, the results passed
                    // through xf: the fast pass keeps no registers for this)
                    ss = 0; pm = 0.0;
                    #pragma unroll 1
                    for (int j = 0; j < 4 * PB4; j++) {
                        const int i = 4 * ((j >> 2) * T + tid) + (j & 3);
                        if (i >= n) continue;
                        const float d = p.delta[i];
                        const float r = p.x[i] + (pn ? norm_apply(d, p.post_w[i], sd, mode) : d);
                        xf[i] = r;
                        const float r16 = round_away(r * 65536.0f);
                        if (fabsf(r16) < 2147483648.0f) { const int32_t q = (int32_t)r16; ss += (int64_t)q * q; }
                        else { const int64_t q = llround_q16(r); ss += q * q; }
                        const double dx2 = fabs((double)r16 * (double)round_away(p.norm_w[i] * 65536.0f));
                        pm = dx2 < 9007199254740992.0 ? fmax(pm, dx2) : INFINITY;     // NaN too
                    }
                    #pragma unroll
                    for (int k = 0; k < PB4; k++)
                        if (4 * (k * T + tid) < n) xv[k] = *(const float4 *)(xf + 4 * (k * T + tid));
                }
                #pragma unroll
                for (int k = 0; k < PB4; k++) {
                    const int i = 4 * (k * T + tid);
                    if (wr && i < n) *(float4 *)(p.x_out + i) = xv[k];
                }
                // max |y| is the largest product's when every product takes
                // norm_apply's double path (each |y| is then a monotone function
                // of its product); otherwise every y is formed and compared.
                // Only the columns [c_lo, c_hi) of the result are formed.
                int64_t *rs = (int64_t *)red_slot(red, 1);
                double *rm = (double *)red_slot(red, 2);
                ss = wave_to63(ss, (int64_t)0, [](int64_t a, int64_t b) { return a + b; });
                pm = wave_to63(pm, 0.0, [](double a, double b) { return fmax(a, b); });
                if ((tid & 63) == 63) { rs[tid >> 6] = ss; rm[tid >> 6] = pm; }
                __syncthreads();
                ss = rs[0]; pm = rm[0];
                for (int w = 1; w < (T >> 6); w++) { ss += rs[w]; pm = fmax(pm, rm[w]); }
                NormScale s; s.f = 0.0f; s.zero = ss == 0;
                s.inv = rms_inv_wg(n, ss, &bcs[1]);
                s.invd = (double)s.inv;
                const double pmx = pm * s.invd;
                if (s.zero || (pm < 9007199254740992.0 && pmx < 4611686018427387904.0)) {
                    m = s.zero ? 0.0f : (float)(pmx * 2.220446049250313e-16);
                    if (dout) {
                        // the digit planes from the registers: no pass through xf
                        const int sh = sh_of_max(m);
                        if (sh != SH_ZERO) {
                            #pragma unroll
                            for (int k = 0; k < PB4; k++) {
                                const int i = 4 * (k * T + tid);
                                if (i < n && i + 3 >= c_lo && i < c_hi) {
                                    float y[4];
                                    #pragma unroll
                                    for (int c = 0; c < 4; c++)
                                        y[c] = (float)(((double)round_away(f4c(xv[k], c) * 65536.0f) * (double)f4c(nw[k], c) *
                                                        s.invd) * 2.220446049250313e-16);
                                    uint32_t h[6];
                                    digits4(y, sh, h);
                                    // column i: block i / 32, dword (i % 32) / 8, half (i % 8) / 4
                                    const int rel = i - dout->b_lo * 32;
                                    uint16_t *d16 = (uint16_t *)(dout->dig + (rel >> 5)) + ((rel & 31) >> 2);
                                    #pragma unroll
                                    for (int pl = 0; pl < 6; pl++) d16[(size_t)pl * dout->nb * 8] = (uint16_t)h[pl];
                                }
                            }
                        }
                        __syncthreads();                               // orders the plane writes
                        dout->done = true;
                        return sh;
                    }
                    #pragma unroll
                    for (int k = 0; k < PB4; k++) {
                        const int i = 4 * (k * T + tid);
                        if (i < n && i + 3 >= c_lo && i < c_hi) {
                            // (straight-line: for a zero vector, inverse 0, the
                            // values are +-0 and sh is SH_ZERO, so nobody reads them)
                            float4 y;
                            #pragma unroll
                            for (int c = 0; c < 4; c++)
                                f4s(y, c, (float)(((double)round_away(f4c(xv[k], c) * 65536.0f) *
                                                   (double)f4c(nw[k], c) * s.invd) *
                                                  2.220446049250313e-16));
                            *(float4 *)(xf + i) = y;
                        }
                    }
                    __syncthreads();                                   // orders the xf writes
                    return sh_of_max(m);
                }
                #pragma unroll
                for (int k = 0; k < PB4; k++) {
                    const int i = 4 * (k * T + tid);
                    if (i < n) {
                        float4 y;
                        #pragma unroll
                        for (int c = 0; c < 4; c++) {
                            const float v = norm_apply_loaded(f4c(xv[k], c), f4c(nw[k], c), s, mode);
                            f4s(y, c, v);
                            m = fmaxf(m, fabsf(v));
                        }
                        *(float4 *)(xf + i) = y;
                    }
                }
                m = block_max(m, (float *)red_slot(red, 3));
                return sh_of_max(m);
            }
            #pragma unroll
            for (int k = 0; k < PB4; k++) {
                const int i = 4 * (k * T + tid);
                #pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float d = f4c(dv[k], c);
                    f4s(xv[k], c, f4c(xv[k], c) + (p.post_w ? norm_apply(d, f4c(pw[k], c), sd, mode) : d));
                }
                if (wr && i < n) *(float4 *)(p.x_out + i) = xv[k];
            }
        }
        SumSq q;
        #pragma unroll
        for (int k = 0; k < PB4; k++)
            if (4 * (k * T + tid) < n)
                #pragma unroll
                for (int c = 0; c < 4; c++) q.add(f4c(xv[k], c), mode);
        const NormScale s = norm_finish(q, n, p.eps, mode, red_slot(red, 1), &bcs[1]);
        #pragma unroll
        for (int k = 0; k < PB4; k++) {
            const int i = 4 * (k * T + tid);
            if (i < n) {
                float4 y;
                #pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float v = norm_apply_loaded(f4c(xv[k], c), f4c(nw[k], c), s, mode);
                    f4s(y, c, v);
                    m = fmaxf(m, fabsf(v));
                }
                *(float4 *)(xf + i) = y;
            }
        }
    } else {
        NormScale s;
        if constexpr (PRO == PRO_NORM) {
            SumSq q;
            for (int base = 0; base < n; base += PB * T) {
                float a[PB];
                #pragma unroll
                for (int k = 0; k < PB; k++) { const int i = base + k * T + tid; a[k] = i < n ? p.x[i] : 0.0f; }
                #pragma unroll
                for (int k = 0; k < PB; k++) q.add(a[k], mode);
                #pragma unroll
                for (int k = 0; k < PB; k++) { const int i = base + k * T + tid; if (i < n) xf[i] = a[k]; }
            }
            s = norm_finish(q, n, p.eps, mode, red_slot(red, 1), &bcs[1]);
        } else {
            NormScale sd; sd.f = 0.0f; sd.inv = 0; sd.invd = 0.0; sd.zero = 0;
            if (pro_uses_stat<PRO>(p, mode)) {
                int64_t ss; float mx;
                stat_reduce(L.sq, L.sm, ss, mx);
                sd = stat_scale(ss, n, &bcs[0]);
            } else if (p.post_w) {
                SumSq q;
                for (int base = 0; base < n; base += PB * T) {
                    float a[PB];
                    #pragma unroll
                    for (int k = 0; k < PB; k++) { const int i = base + k * T + tid; a[k] = i < n ? p.delta[i] : 0.0f; }
                    #pragma unroll
                    for (int k = 0; k < PB; k++) q.add(a[k], mode);
                }
                sd = norm_finish(q, n, p.eps, mode, red_slot(red, 0), &bcs[0]);
            }
            // residual add (+ sandwich norm of the branch), sum of squares of the result
            SumSq q;
            const bool wr = write_x && p.x_out;
            for (int base = 0; base < n; base += PB * T) {
                float xv[PB], dv[PB], pw[PB];
                #pragma unroll
                for (int k = 0; k < PB; k++) {
                    const int i = base + k * T + tid;
                    xv[k] = i < n ? p.x[i] : 0.0f;
                    dv[k] = i < n ? p.delta[i] : 0.0f;
                    pw[k] = (i < n && p.post_w) ? p.post_w[i] : 0.0f;
                }
                #pragma unroll
                for (int k = 0; k < PB; k++) {
                    const int i = base + k * T + tid;
                    const float r = xv[k] + (p.post_w ? norm_apply(dv[k], pw[k], sd, mode) : dv[k]);
                    if (i < n) { xf[i] = r; if (wr) p.x_out[i] = r; q.add(r, mode); }
                }
            }
            s = norm_finish(q, n, p.eps, mode, red_slot(red, 1), &bcs[1]);
        }
        // xf <- norm(xf) * w; running max
        for (int base = 0; base < n; base += PB * T) {
            float w[PB];
            #pragma unroll
            for (int k = 0; k < PB; k++) { const int i = base + k * T + tid; w[k] = i < n ? p.norm_w[i] : 0.0f; }
            #pragma unroll
            for (int k = 0; k < PB; k++) {
                const int i = base + k * T + tid;
                if (i < n) { const float y = norm_apply(xf[i], w[k], s, mode); xf[i] = y; m = fmaxf(m, fabsf(y)); }
            }
        }
    }
    m = block_max(m, (float *)red_slot(red, 2));         // its barrier also orders the xf writes above
    return sh_of_max(m);
}

// Loads and transforms in one call (kernels with nothing to prefetch).
template <int PRO>
__device__ int input_transform(const ProArgs &p, int mode, float *xf, void *red, bool write_x) {
    ProLoads L;
    pro_load<PRO>(p, mode, L);
    return input_transform<PRO>(p, mode, L, xf, red, write_x);
}

__device__ __forceinline__ void f16_parts(uint32_t h, int32_t &M, int &e) {
    const int E5 = (h >> 10) & 31, mant = h & 1023;
    M = E5 ? 1024 + mant : mant;
    if (h & 0x8000u) M = -M;
    e = E5 ? E5 - 25 : -24;
}
__device__ __forceinline__ float act_apply(float g, float u, int act, int mode) {
    if (act == ACT_GELU) {
        if (mode == EXACT) return gelu_exact1(g) * u;
        const float k = 0.7978845608028654f;                       // sp_session.c:365-368
        return 0.5f * g * (1.0f + tanhf(k * (g + 0.044715f * g * g * g))) * u;
    }
    if (mode == EXACT) return silu_exact1(g) * u;
    return g / (1.0f + expf(-g)) * u;                              // sp_session.c:354
}

}  // namespace kvd
