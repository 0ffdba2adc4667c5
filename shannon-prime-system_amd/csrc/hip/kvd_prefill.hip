// kvd_prefill.hip -- batched prefill: per-token input staging and the OK_Q4B
// GEMM on the int8 matrix cores (v_mfma_i32_16x16x32_i8, CDNA3/CDNA4).
//
// The arithmetic is the decode GEMV's, so every token's outputs are
// bit-identical to a decode step's (exact integer sum, one RNE):
//   xq = rne(x * 2^sh) per token, |xq| <= 2^22, split into three balanced
//   base-256 digits beta_p in [-128, 127] (xq = sum_p 256^p beta_p);
//   per 32-column block b and plane p one MFMA gives the exact int32
//   sum_i code[j,i] * beta_p[t,i] for a 16-row x 16-token tile;
//   d = sum_p 256^p * plane_p (|d| < 2^30), and d * M_jb << (e_jb - ebase_j)
//   accumulates in int64 exactly as in the GEMV.
// A workgroup (4 waves) owns 64 rows x 32 tokens; a wave owns 16 rows and two
// 16-token MFMA tiles that share its A operand (the unpacked weight codes).
#include "kvd_internal.h"
#include "kvd_exact.h"
#include "kvd_vec.h"
#include <cstdio>
#include <cstdlib>

namespace kvd {

typedef int v4i __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------- staging
// Planes layout: planes[p][b][t][32] int8 for p < 3, b < nblk, t < TP.  The 32
// bytes of a (block, token) follow the A operand's unpack order: within each
// group of 8 columns 8g..8g+7 the order is 8g + {0, 2, 4, 6, 1, 3, 5, 7}
// (low nibbles, then high nibbles, of the packed codes).
template <int PRO>
__global__ __launch_bounds__(512) void k_stage(StageArgs a) {
    extern __shared__ float xf[];                      // pro.n floats (norm prologues)
    __shared__ double red[8];
    const int t = blockIdx.x, n = a.pro.n, nblk = n / 32, tid = threadIdx.x;
    int8_t *planes = a.planes;
    if (t >= a.T) {                                     // padding tokens: zero planes
        for (int g = tid; g < nblk * 4; g += blockDim.x)
            #pragma unroll
            for (int p = 0; p < 3; p++)
                *(uint2 *)(planes + (((size_t)p * nblk + (g >> 2)) * a.TP + t) * 32 + 8 * (g & 3)) = make_uint2(0, 0);
        if (tid == 0) a.sh[t] = SH_ZERO;
        return;
    }
    ProArgs p = a.pro;
    p.x += (size_t)t * n;
    if (p.delta) p.delta += (size_t)t * n;
    if (p.x_out) p.x_out += (size_t)t * n;
    const int sh = input_transform<PRO>(p, a.mode, xf, red, true);
    if (tid == 0) a.sh[t] = sh;
    const float *src = PRO == PRO_PLAIN ? p.x : xf;
    for (int g = tid; g < nblk * 4; g += blockDim.x) {
        uint32_t lo[3] = {0, 0, 0}, hi[3] = {0, 0, 0};
        if (sh != SH_ZERO) {
            const float4 v0 = *(const float4 *)(src + g * 8), v1 = *(const float4 *)(src + g * 8 + 4);
            const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            #pragma unroll
            for (int j = 0; j < 8; j++) {
                int32_t q = (int32_t)rintf(ldexpf(v[j], sh));
                const int slot = (j & 1) ? 4 + (j >> 1) : (j >> 1);      // unpack order
                #pragma unroll
                for (int pl = 0; pl < 3; pl++) {
                    const int32_t d = ((q + 128) & 255) - 128;
                    q = (q - d) >> 8;
                    const uint32_t byte = (uint32_t)(d & 255) << (8 * (slot & 3));
                    if (slot < 4) lo[pl] |= byte; else hi[pl] |= byte;
                }
            }
        }
        #pragma unroll
        for (int pl = 0; pl < 3; pl++)
            *(uint2 *)(planes + (((size_t)pl * nblk + (g >> 2)) * a.TP + t) * 32 + 8 * (g & 3)) = make_uint2(lo[pl], hi[pl]);
    }
}

// ------------------------------------------------------------- GEMM
// 8 signed nibbles (low nibble = even column) -> 8 int8 in unpack order
__device__ __forceinline__ long unpack_codes(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const uint32_t slo = lo | ((lo & 0x08080808u) * 0x1Eu);    // sign-extend each byte from 4 bits
    const uint32_t shi = hi | ((hi & 0x08080808u) * 0x1Eu);
    return (long)(((uint64_t)shi << 32) | slo);
}

template <bool PAIRED>
__global__ __launch_bounds__(256) void k_gemm_q4b(GemmArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c16 = lane & 15, g = lane >> 4;
    // row tile -> segment (segment row counts are multiples of 64)
    int tile_row = blockIdx.x * 64, s = 0;
    if (!PAIRED) while (s < a.nseg - 1 && tile_row >= a.seg[s].w.rows) { tile_row -= a.seg[s].w.rows; s++; }
    const DevW &wa = a.seg[s].w;
    const DevW &wb = a.seg[PAIRED ? 1 : s].w;
    const int nblk = wa.nblk;
    const size_t rb = (size_t)wa.cols / 2;
    const int rbase = tile_row + wave * 16;              // this wave's 16 rows
    const int t0 = blockIdx.y * 32;
    const uint8_t *ca = wa.codes + (size_t)(rbase + c16) * rb + 4 * g;
    const uint8_t *cb = wb.codes + (size_t)(rbase + c16) * rb + 4 * g;
    const int8_t *pl = a.planes;
    const size_t pstride = (size_t)nblk * a.TP * 32;   // bytes per plane
    int eb_a[4], eb_b[4];
    #pragma unroll
    for (int i = 0; i < 4; i++) {
        eb_a[i] = wa.ebase[rbase + 4 * g + i];
        eb_b[i] = PAIRED ? wb.ebase[rbase + 4 * g + i] : 0;
    }
    int64_t acc_a[2][4], acc_b[2][4];
    #pragma unroll
    for (int j = 0; j < 2; j++)
        #pragma unroll
        for (int i = 0; i < 4; i++) { acc_a[j][i] = 0; acc_b[j][i] = 0; }

    for (int b0 = 0; b0 < nblk; b0 += 8) {
        // f16 scales of this lane's 4 output rows for 8 blocks (16 B per row)
        uint4 sa[4], sb[4];
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            sa[i] = *(const uint4 *)(wa.bs + (size_t)(rbase + 4 * g + i) * nblk + b0);
            if (PAIRED) sb[i] = *(const uint4 *)(wb.bs + (size_t)(rbase + 4 * g + i) * nblk + b0);
        }
        #pragma unroll 2
        for (int bb = 0; bb < 8; bb++) {
            const int b = b0 + bb;
            const long A = unpack_codes(*(const uint32_t *)(ca + (size_t)b * 16));
            long A2 = 0;
            if (PAIRED) A2 = unpack_codes(*(const uint32_t *)(cb + (size_t)b * 16));
            long B[2][3];
            #pragma unroll
            for (int j = 0; j < 2; j++)
                #pragma unroll
                for (int p = 0; p < 3; p++)
                    B[j][p] = *(const long *)(pl + p * pstride + ((size_t)b * a.TP + t0 + 16 * j + c16) * 32 + 8 * g);
            #pragma unroll
            for (int j = 0; j < 2; j++) {
                const v4i z = {0, 0, 0, 0};
                const v4i p0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B[j][0], z, 0, 0, 0);
                const v4i p1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B[j][1], z, 0, 0, 0);
                const v4i p2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B[j][2], z, 0, 0, 0);
                #pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int32_t d = p0[i] + (p1[i] << 8) + (p2[i] << 16);
                    const uint32_t hw = (((const uint32_t *)&sa[i])[bb >> 1] >> (16 * (bb & 1))) & 0xFFFFu;
                    int32_t M; int e; f16_parts(hw, M, e);
                    const int sft = e - eb_a[i];
                    acc_a[j][i] += (int64_t)((uint64_t)((int64_t)d * M) << (sft > 0 ? sft : 0));
                }
                if (PAIRED) {
                    const v4i q0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A2, B[j][0], z, 0, 0, 0);
                    const v4i q1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A2, B[j][1], z, 0, 0, 0);
                    const v4i q2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A2, B[j][2], z, 0, 0, 0);
                    #pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int32_t d = q0[i] + (q1[i] << 8) + (q2[i] << 16);
                        const uint32_t hw = (((const uint32_t *)&sb[i])[bb >> 1] >> (16 * (bb & 1))) & 0xFFFFu;
                        int32_t M; int e; f16_parts(hw, M, e);
                        const int sft = e - eb_b[i];
                        acc_b[j][i] += (int64_t)((uint64_t)((int64_t)d * M) << (sft > 0 ? sft : 0));
                    }
                }
            }
        }
    }
    // outputs: lane holds rows rbase + 4g + i, tokens t0 + 16j + c16
    #pragma unroll
    for (int j = 0; j < 2; j++) {
        const int t = t0 + 16 * j + c16;
        if (t >= a.T) continue;
        const int sh = a.sh[t];
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = rbase + 4 * g + i;
            const float ya = sh == SH_ZERO ? 0.0f : rne_i64_scaled(acc_a[j][i], eb_a[i] - sh);
            if (PAIRED) {
                const float yb = sh == SH_ZERO ? 0.0f : rne_i64_scaled(acc_b[j][i], eb_b[i] - sh);
                const size_t o = (size_t)t * wa.rows + row;
                a.seg[0].out[o] = ya; a.seg[1].out[o] = yb;
                a.act_out[o] = act_apply(ya, yb, a.act, a.mode);
            } else {
                a.seg[s].out[(size_t)t * wa.rows + row] = ya;
            }
        }
    }
}

// ------------------------------------------------------------- launchers
void launch_stage(const StageArgs &a, hipStream_t s) {
    const size_t lds = a.pro.kind == PRO_PLAIN ? 0 : (size_t)a.pro.n * sizeof(float);
    if (a.pro.n % 32 || a.TP % 32 || a.T > a.TP) { fprintf(stderr, "kvd: stage shape n=%d T=%d TP=%d\n", a.pro.n, a.T, a.TP); abort(); }
    switch (a.pro.kind) {
    case PRO_PLAIN: hipLaunchKernelGGL(k_stage<PRO_PLAIN>, dim3(a.TP), dim3(512), lds, s, a); break;
    case PRO_NORM:  hipLaunchKernelGGL(k_stage<PRO_NORM>, dim3(a.TP), dim3(512), lds, s, a); break;
    default:        hipLaunchKernelGGL(k_stage<PRO_RESID>, dim3(a.TP), dim3(512), lds, s, a); break;
    }
}

bool gemm_supported(const DevW &w) {
    return !w.wide && w.rows % 64 == 0 && w.cols % 256 == 0;
}

void launch_gemm(const GemmArgs &a, int nrows_total, hipStream_t s) {
    const bool paired = a.act != ACT_NONE;
    for (int i = 0; i < a.nseg; i++)
        if (!gemm_supported(a.seg[i].w) || a.seg[i].w.cols != a.cols) {
            fprintf(stderr, "kvd: GEMM segment %d shape %dx%d not supported\n", i, a.seg[i].w.rows, a.seg[i].w.cols); abort();
        }
    if (nrows_total % 64 || a.TP % 32 || a.T > a.TP) { fprintf(stderr, "kvd: GEMM rows %d T %d TP %d\n", nrows_total, a.T, a.TP); abort(); }
    const dim3 grid(nrows_total / 64, a.TP / 32);
    if (paired) hipLaunchKernelGGL(k_gemm_q4b<true>, grid, dim3(256), 0, s, a);
    else        hipLaunchKernelGGL(k_gemm_q4b<false>, grid, dim3(256), 0, s, a);
}

}  // namespace kvd
