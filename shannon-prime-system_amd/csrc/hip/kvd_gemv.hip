// kvd_gemv.hip -- OK_Q4B GEMV for batch-1 decode (CDNA4 / gfx950).
//
// Reference semantics: the OK_Q4B branch of matmul_arena
// (core/forward_dispatch/forward_dispatch.c:69-85): y[j] = sum_b f16(bs[j,b]) *
// sum_{i in b} code[j,i] * x[i].  Here the sum is evaluated exactly:
//
//   1. every workgroup runs the input transform (residual add / RMSNorm) and
//      puts x on a per-vector power-of-two grid: xq = rne(x * 2^sh), |xq| < 2^22;
//   2. xq is split into six balanced base-16 digit planes (digits in [-8,7])
//      held in LDS, so the packed int4 weight codes feed v_dot8_i32_i4 directly:
//      sum code*xq = sum_k 16^k * dot8(code, digit_k) -- no nibble unpacking;
//   3. block scale f16 = M * 2^e is applied exactly into an int64 row
//      accumulator relative to the row's smallest block exponent (int128 when a
//      row's exponent spread could overflow), lanes are combined exactly and the
//      row result is rounded to float once (RNE).
// Integer sums are order-free, so the result is bit-identical to the CPU oracle
// whatever the wave/lane decomposition.  It is also within ~1e-7 relative of
// the reference's float accumulation, so float mode uses the same kernel.
//
// Layout: one wave owns GEMV_R rows at a time; lane l walks blocks l, l+64, ...
// loading 16 B of codes per row per block (fully coalesced 1 KiB per wave-load)
// and one 16 B LDS read per digit plane, shared by the wave's rows.
#include "kvd_internal.h"
#include "kvd_exact.h"
#include <cstdio>
#include <cstdlib>

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
// block-wide reductions for 256 threads through a small LDS scratch
template <typename T> __device__ T block_sum(T v, T *red) {   // red: blockDim/64 slots
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    T t = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) t += red[i];
    return t;
}
__device__ float block_max(float v, float *red) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) t = fmaxf(t, red[i]);
    return t;
}

// ------------------------------------------------------- RMSNorm (both modes)
// Float mode: core/forward_kernels/forward_kernels.c:17-22 (sum of squares in
// double, 1/sqrtf((float)(ss/n)+eps), out = x*scale*w).  Exact mode: the
// integer island core/exact_islands/exact_islands.c:60-79 (no eps).
struct NormScale { float f; int64_t inv; int zero; };

__device__ NormScale norm_scale(const float *v, int n, float eps, int mode, void *red) {
    NormScale s; s.f = 0.0f; s.inv = 0; s.zero = 0;
    if (mode == FLOAT) {
        double ss = 0.0;
        for (int i = threadIdx.x; i < n; i += blockDim.x) ss += (double)v[i] * (double)v[i];
        ss = block_sum<double>(ss, (double *)red);
        s.f = 1.0f / sqrtf((float)(ss / n) + eps);
    } else {
        int64_t ss = 0;
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            int64_t xi = llround_d((double)v[i] * 65536.0);
            ss += xi * xi;
        }
        ss = block_sum<int64_t>(ss, (int64_t *)red);
        if (ss == 0) { s.zero = 1; return s; }
        const uint64_t q = udiv128_64((u128)n << 72, (uint64_t)ss);
        s.inv = (int64_t)isqrt_u64(q);
    }
    return s;
}
__device__ __forceinline__ float norm_apply(float x, float w, const NormScale &s, int mode) {
    if (mode == FLOAT) return x * s.f * w;
    if (s.zero) return 0.0f;
    const int64_t xi = llround_d((double)x * 65536.0), wi = llround_d((double)w * 65536.0);
    return (float)((double)mul3_lo64(xi, s.inv, wi) / 4503599627370496.0);   // 2^52
}

// ------------------------------------------------------- prologue
// Builds the GEMV input (float, in xf) and its digit planes (in dig), returns sh
// (or INT_MIN for an all-zero input).
constexpr int SH_ZERO = -1000000;

__device__ int gemv_prologue(const ProArgs &p, int mode, float *xf, uint4 *dig, int nblk, void *red) {
    const int n = p.n;
    // PRO_PLAIN reads its input straight from global memory (two passes: max,
    // then digits); the norm prologues stage the transformed vector in xf.
    const bool plain = p.kind == PRO_PLAIN;
    if (p.kind == PRO_NORM) {
        NormScale s = norm_scale(p.x, n, p.eps, mode, red);
        for (int i = threadIdx.x; i < n; i += blockDim.x) xf[i] = norm_apply(p.x[i], p.norm_w[i], s, mode);
    } else if (p.kind == PRO_RESID) {
        if (p.post_w) {
            NormScale sd = norm_scale(p.delta, n, p.eps, mode, red);
            for (int i = threadIdx.x; i < n; i += blockDim.x)
                xf[i] = p.x[i] + norm_apply(p.delta[i], p.post_w[i], sd, mode);
        } else {
            for (int i = threadIdx.x; i < n; i += blockDim.x) xf[i] = p.x[i] + p.delta[i];
        }
        __syncthreads();
        if (blockIdx.x == 0 && p.x_out)
            for (int i = threadIdx.x; i < n; i += blockDim.x) p.x_out[i] = xf[i];
        NormScale s = norm_scale(xf, n, p.eps, mode, red);
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += blockDim.x) xf[i] = norm_apply(xf[i], p.norm_w[i], s, mode);
    }
    const float *src = plain ? p.x : xf;
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, fabsf(src[i]));
    m = block_max(m, (float *)red);                      // also orders the xf writes above
    if (m == 0.0f) return SH_ZERO;
    int e; frexpf(m, &e);
    const int sh = 22 - e;
    // digits: one thread per 8 consecutive columns (one nibble-dword per plane)
    const int ngroups = nblk * 4;
    for (int g = threadIdx.x; g < ngroups; g += blockDim.x) {
        uint32_t dw[NDIG] = {0, 0, 0, 0, 0, 0};
        #pragma unroll
        for (int j = 0; j < 8; j++) {
            const int c = g * 8 + j;
            int32_t v = c < n ? (int32_t)rint(ldexp((double)src[c], sh)) : 0;
            #pragma unroll
            for (int k = 0; k < NDIG; k++) {
                int32_t d = ((v + 8) & 15) - 8;
                v = (v - d) >> 4;
                dw[k] |= (uint32_t)(d & 15) << (4 * j);
            }
        }
        const int b = g >> 2, q = g & 3;
        #pragma unroll
        for (int k = 0; k < NDIG; k++) ((uint32_t *)&dig[k * nblk + b])[q] = dw[k];
    }
    __syncthreads();
    return sh;
}

// ------------------------------------------------------- main kernel
__device__ __forceinline__ void f16_parts(uint32_t h, int32_t &M, int &e) {
    const int E5 = (h >> 10) & 31, mant = h & 1023;
    M = E5 ? 1024 + mant : mant;
    if (h & 0x8000u) M = -M;
    e = E5 ? E5 - 25 : -24;
}
__device__ __forceinline__ int32_t dot_digits(const uint4 c, const uint4 *D) {
    // sum over the 32 codes of code * xq, xq = sum_k 16^k digit_k
    int32_t a = 0;
    #pragma unroll
    for (int k = NDIG - 1; k >= 0; k--) {
        int32_t t = 0;
        t = __builtin_amdgcn_sdot8((int)c.x, (int)D[k].x, t, false);
        t = __builtin_amdgcn_sdot8((int)c.y, (int)D[k].y, t, false);
        t = __builtin_amdgcn_sdot8((int)c.z, (int)D[k].z, t, false);
        t = __builtin_amdgcn_sdot8((int)c.w, (int)D[k].w, t, false);
        a = a * 16 + t;
    }
    return a;
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

// Sum GEMV_R = 8 per-lane int64 partials over the wave with 10 exchanges
// instead of 48: each step halves the rows a lane carries.  Afterwards lane l
// holds the total of row ((l>>5)&1)*4 + ((l>>4)&1)*2 + ((l>>3)&1) (all lanes
// of an aligned group of 8 agree).
__device__ __forceinline__ int64_t transpose_reduce8(const int64_t v[8], int lane) {
    const bool hi32 = lane & 32, hi16 = lane & 16, hi8 = lane & 8;
    int64_t w[4], x[2];
    #pragma unroll
    for (int r = 0; r < 4; r++) {
        const int64_t send = hi32 ? v[r] : v[r + 4];
        w[r] = (hi32 ? v[r + 4] : v[r]) + __shfl_xor(send, 32, 64);
    }
    #pragma unroll
    for (int r = 0; r < 2; r++) {
        const int64_t send = hi16 ? w[r] : w[r + 2];
        x[r] = (hi16 ? w[r + 2] : w[r]) + __shfl_xor(send, 16, 64);
    }
    const int64_t send = hi8 ? x[0] : x[1];
    int64_t y = (hi8 ? x[1] : x[0]) + __shfl_xor(send, 8, 64);
    y += __shfl_xor(y, 4, 64);
    y += __shfl_xor(y, 2, 64);
    y += __shfl_xor(y, 1, 64);
    return y;
}

template <bool WIDE>
__global__ __launch_bounds__(512) void k_gemv(GemvArgs a) {
    extern __shared__ uint4 smem4[];
    const int cols = a.cols, nblk = (cols + 31) / 32;
    uint4 *dig = smem4;                                   // NDIG * nblk
    float *xf = (float *)(dig + NDIG * nblk);             // pro.n floats (norm prologues only)
    __shared__ double red[GEMV_WAVES];

    const int sh = gemv_prologue(a.pro, a.mode, xf, dig, nblk, red);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rows0 = a.seg[0].w.rows;
    const int paired = a.act != ACT_NONE;
    const int HR = GEMV_R / 2;                            // paired: HR gate rows + HR up rows
    int total_groups;
    if (paired) total_groups = (rows0 + HR - 1) / HR;
    else {
        int tr = 0;
        for (int s = 0; s < a.nseg; s++) tr += a.seg[s].w.rows;
        total_groups = (tr + GEMV_R - 1) / GEMV_R;
    }
    const size_t rb = (size_t)(cols + 1) / 2;

    for (int grp = blockIdx.x * GEMV_WAVES + wave; grp < total_groups; grp += gridDim.x * GEMV_WAVES) {
        // A group never straddles segments (segment row counts are multiples of
        // the group size, checked by the host), so its rows are consecutive and
        // addressed from one wave-uniform base per half.
        int seg0, row0, nvalid;
        if (paired) {
            seg0 = 0; row0 = grp * HR;
            nvalid = rows0 - row0 < HR ? rows0 - row0 : HR;
        } else {
            int g = grp * GEMV_R, s = 0;
            while (s < a.nseg - 1 && g >= a.seg[s].w.rows) { g -= a.seg[s].w.rows; s++; }
            seg0 = s; row0 = g;
            nvalid = a.seg[s].w.rows - g < GEMV_R ? a.seg[s].w.rows - g : GEMV_R;
        }
        seg0 = __builtin_amdgcn_readfirstlane(seg0);
        row0 = __builtin_amdgcn_readfirstlane(row0);
        nvalid = __builtin_amdgcn_readfirstlane(nvalid);
        const DevW &wa = a.seg[seg0].w;
        const DevW &wb = a.seg[paired ? 1 : seg0].w;
        const uint8_t *cba = wa.codes + (size_t)row0 * rb, *cbb = wb.codes + (size_t)row0 * rb;
        const uint16_t *sba = wa.bs + (size_t)row0 * nblk, *sbb = wb.bs + (size_t)row0 * nblk;
        const int per = paired ? HR : GEMV_R;             // rows taken from each base
        int eb[GEMV_R];
        #pragma unroll
        for (int r = 0; r < GEMV_R; r++) {
            const int rr = r % per;
            const DevW &w = (paired && r >= HR) ? wb : wa;
            eb[r] = WIDE ? -24 : (rr < nvalid ? (int)w.ebase[row0 + rr] : 0);
        }
        typedef typename std::conditional<WIDE, i128, int64_t>::type acc_t;
        acc_t acc[GEMV_R];
        #pragma unroll
        for (int r = 0; r < GEMV_R; r++) acc[r] = 0;

        if (sh != SH_ZERO) {
            for (int b = lane; b < nblk; b += 64) {
                uint4 c[GEMV_R];
                uint32_t h[GEMV_R];
                #pragma unroll
                for (int r = 0; r < GEMV_R; r++) {
                    const int rr = r % per;
                    const bool second = paired && r >= HR;
                    if (rr < nvalid) {
                        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
                        const uint8_t *cp = (second ? cbb : cba) + (size_t)rr * rb + (size_t)b * 16;
                        const u32x4 t = __builtin_nontemporal_load((const u32x4 *)cp);
                        c[r] = make_uint4(t.x, t.y, t.z, t.w);
                        h[r] = (second ? sbb : sba)[(size_t)rr * nblk + b];
                    } else { c[r] = make_uint4(0, 0, 0, 0); h[r] = 0; }
                }
                uint4 D[NDIG];
                #pragma unroll
                for (int k = 0; k < NDIG; k++) D[k] = dig[k * nblk + b];
                #pragma unroll
                for (int r = 0; r < GEMV_R; r++) {
                    const int32_t d = dot_digits(c[r], D);
                    int32_t M; int e; f16_parts(h[r], M, e);
                    const int64_t p = (int64_t)d * (int64_t)M;
                    if constexpr (WIDE) acc[r] += (i128)((u128)(i128)p << (e + 24));
                    else {
                        const int s = e - eb[r];
                        acc[r] += (int64_t)((uint64_t)p << (s > 0 ? s : 0));
                    }
                }
            }
        }
        float y[GEMV_R];
        int myrow = 0;
        if constexpr (WIDE) {
            #pragma unroll
            for (int r = 0; r < GEMV_R; r++) {
                const i128 t = wave_sum128(acc[r]);
                y[r] = sh == SH_ZERO ? 0.0f : rne_i128_scaled(t, -24 - sh);
            }
        } else {
            const int64_t t = transpose_reduce8(acc, lane);
            myrow = ((lane >> 5) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 3) & 1);
            int ebm = eb[0];
            #pragma unroll
            for (int r = 1; r < GEMV_R; r++) if (myrow == r) ebm = eb[r];
            y[0] = sh == SH_ZERO ? 0.0f : rne_i64_scaled(t, ebm - sh);
        }
        if constexpr (WIDE) {
            if (lane == 0) {
                if (paired) {
                    for (int r = 0; r < nvalid; r++) {
                        const int j = row0 + r;
                        a.seg[0].out[j] = y[r]; a.seg[1].out[j] = y[r + HR];
                        a.act_out[j] = act_apply(y[r], y[r + HR], a.act, a.mode);
                    }
                } else {
                    for (int r = 0; r < nvalid; r++) a.seg[seg0].out[row0 + r] = y[r];
                }
            }
        } else {
            // lane (myrow*8) owns row myrow's total; paired rows fetch their up partner
            const float partner = __shfl_xor(y[0], 32, 64);          // row myrow^4
            if ((lane & 7) == 0) {
                if (paired) {
                    if (myrow < HR && myrow < nvalid) {
                        const int j = row0 + myrow;
                        a.seg[0].out[j] = y[0]; a.seg[1].out[j] = partner;
                        a.act_out[j] = act_apply(y[0], partner, a.act, a.mode);
                    }
                } else if (myrow < nvalid) {
                    a.seg[seg0].out[row0 + myrow] = y[0];
                }
            }
        }
    }
}

static int g_num_cu = 0;
int gemv_grid(int nrows_total, int cols, int paired) {
    if (!g_num_cu) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_num_cu = n;
        else
            g_num_cu = 256;
    }
    const int groups = paired ? (nrows_total + GEMV_R / 2 - 1) / (GEMV_R / 2) : (nrows_total + GEMV_R - 1) / GEMV_R;
    const int blocks = (groups + GEMV_WAVES - 1) / GEMV_WAVES;
    const int cap = 2 * g_num_cu;                      // every workgroup pays the input prologue once
    (void)cols;
    return blocks < cap ? blocks : cap;
}

void launch_gemv(const GemvArgs &a, int nrows_total, hipStream_t s) {
    const int nblk = (a.cols + 31) / 32;
    // a wave's row group must not straddle segments
    for (int i = 0; i + 1 < a.nseg; i++)
        if (a.seg[i].w.rows % GEMV_R) { fprintf(stderr, "kvd: GEMV segment rows %d not a multiple of %d\n", a.seg[i].w.rows, GEMV_R); abort(); }
    const size_t lds = (size_t)NDIG * nblk * sizeof(uint4) +
                       (a.pro.kind == PRO_PLAIN ? 0 : (size_t)a.pro.n * sizeof(float));
    const int grid = gemv_grid(nrows_total, a.cols, a.act != ACT_NONE);
    bool wide = false;
    for (int i = 0; i < a.nseg; i++) wide |= a.seg[i].w.wide != 0;
    if (wide) hipLaunchKernelGGL(k_gemv<true>, dim3(grid), dim3(GEMV_WAVES * 64), lds, s, a);
    else      hipLaunchKernelGGL(k_gemv<false>, dim3(grid), dim3(GEMV_WAVES * 64), lds, s, a);
}

}  // namespace kvd
