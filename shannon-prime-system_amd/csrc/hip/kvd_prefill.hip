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
// A workgroup (4 waves) owns 64 rows x 16 or 32 tokens; a wave owns 16 rows
// and one or two 16-token MFMA tiles that share its A operand (the unpacked
// weight codes).
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
    __shared__ double red[RED_SLOTS * RED_WAVES];
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

// One group of U blocks of a wave's operands, loaded a group ahead of use:
// weight codes (one dword per lane and block), the activation planes of its TT
// token tiles, and the f16 block scales of the lane's output row.
template <bool PAIRED, int TT, int U> struct GemmBuf {
    uint32_t A[U], A2[PAIRED ? U : 1];
    long B[U][TT][3];
    uint32_t S[U / 2], S2[PAIRED ? U / 2 : 1];
};


// d = sum_k code_k * xq_k over one 32-column block for a 16-token x 16-row
// tile: one independent MFMA per digit plane, combined as
// (p2 * 256 + p1) * 256 + p0 (|d| < 2^31, exact in int32)
__device__ __forceinline__ v4i block_dot(const long (&b)[3], long w) {
    const v4i z = {0, 0, 0, 0};
    const v4i p0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(b[0], w, z, 0, 0, 0);
    const v4i p1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(b[1], w, z, 0, 0, 0);
    const v4i p2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(b[2], w, z, 0, 0, 0);
    return (((p2 << 8) + p1) << 8) + p0;
}

// raw buffer access: a wave-uniform base in the resource, a fixed per-lane
// byte offset, the per-iteration offset in a scalar register; reads past
// `bytes` return zero
constexpr int BUF_WORD3 = 0x00020000;                  // 32-bit data format, raw access
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, BUF_WORD3);
}
__device__ __forceinline__ uint32_t buf_ld32(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
__device__ __forceinline__ long buf_ld64(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(long, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

// A wave owns 16 weight rows x TT 16-token tiles.  The activations are the
// MFMA's A operand and the weight codes its B operand, so a lane's outputs are
// one weight row (16-lane index) x 4 tokens, and each block's scale is decoded
// once per lane: the exact integer Ms = M * 2^(e - ebase) = f16 * 2^-ebase
// (below 2^31 for every row the GEMM takes); each block adds d * Ms to the
// int64 total.  Loads use a wave-uniform base and a 32-bit lane offset.
template <bool PAIRED, int TT>
__global__ __launch_bounds__(256) void k_gemm_q4b(GemmArgs a) {
    constexpr int U = 4;
    typedef GemmBuf<PAIRED, TT, U> Buf;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c16 = lane & 15, g = lane >> 4;
    // row tile -> segment (segment row counts are multiples of 64)
    int tile_row = blockIdx.x * 64, s = 0;
    if (!PAIRED) while (s < a.nseg - 1 && tile_row >= a.seg[s].w.rows) { tile_row -= a.seg[s].w.rows; s++; }
    const DevW &wa = a.seg[s].w;
    const DevW &wb = a.seg[PAIRED ? 1 : s].w;
    const int nblk = wa.nblk, TP = a.TP;
    const int rb = wa.cols / 2;
    const int rbase = tile_row + wave * 16;              // this wave's 16 rows
    const int t0 = blockIdx.y * 16 * TT;
    const int row = rbase + c16;                         // this lane's output row
    // this wave's 16 rows of codes and scales, the workgroup's token columns of
    // the planes (all offsets below 2^31: checked by the launcher)
    const __amdgpu_buffer_rsrc_t rca = buf_rsrc(wa.codes + (size_t)rbase * rb, 16u * rb);
    const __amdgpu_buffer_rsrc_t rcb = buf_rsrc(wb.codes + (size_t)rbase * rb, 16u * rb);
    const int lo_c = c16 * rb + 4 * g;
    const int pstride = nblk * TP * 32;                  // bytes per plane
    const __amdgpu_buffer_rsrc_t rpl = buf_rsrc(a.planes + (size_t)t0 * 32, 3u * pstride - 32u * t0);
    const int lo_p = c16 * 32 + 8 * g;
    const __amdgpu_buffer_rsrc_t rsa = buf_rsrc(wa.bs + (size_t)rbase * nblk, 32u * nblk);
    const __amdgpu_buffer_rsrc_t rsb = buf_rsrc(wb.bs + (size_t)rbase * nblk, 32u * nblk);
    const int lo_s = c16 * nblk * 2;
    const int eb_a = wa.ebase[row], eb_b = PAIRED ? wb.ebase[row] : 0;
    const float sc_a = ldexpf(1.0f, -eb_a), sc_b = ldexpf(1.0f, -eb_b);
    int64_t acc_a[TT][4], acc_b[TT][4];
    #pragma unroll
    for (int j = 0; j < TT; j++)
        #pragma unroll
        for (int i = 0; i < 4; i++) { acc_a[j][i] = 0; acc_b[j][i] = 0; }

    auto load = [&](Buf &X, int b0_) {
        // the block index is wave-uniform: keep every scalar offset in SGPRs
        // (a VGPR offset would need a per-lane loop and a full wait).  Groups
        // past the end re-read the last group (never used): every iteration
        // issues the same loads, so the waits count exactly the groups ahead
        const int b0 = __builtin_amdgcn_readfirstlane(b0_ < nblk - U ? b0_ : nblk - U);
        #pragma unroll
        for (int u = 0; u < U; u++) {
            X.A[u] = buf_ld32(rca, lo_c, (b0 + u) * 16);
            if constexpr (PAIRED) X.A2[u] = buf_ld32(rcb, lo_c, (b0 + u) * 16);
            #pragma unroll
            for (int j = 0; j < TT; j++)
                #pragma unroll
                for (int p = 0; p < 3; p++)
                    X.B[u][j][p] = buf_ld64(rpl, lo_p, p * pstride + ((b0 + u) * TP + 16 * j) * 32);
        }
        static_assert(U == 4, "scales: one 8-byte load per lane and group");
        const long sa2 = buf_ld64(rsa, lo_s, b0 * 2);
        X.S[0] = (uint32_t)sa2; X.S[1] = (uint32_t)((unsigned long)sa2 >> 32);
        if constexpr (PAIRED) {
            const long sb2 = buf_ld64(rsb, lo_s, b0 * 2);
            X.S2[0] = (uint32_t)sb2; X.S2[1] = (uint32_t)((unsigned long)sb2 >> 32);
        }
    };
    auto compute = [&](const Buf &X) {
        #pragma unroll
        for (int u = 0; u < U; u++) {
            const long wA = unpack_codes(X.A[u]);
            const unsigned short h = (unsigned short)(X.S[u >> 1] >> (16 * (u & 1)));
            const int32_t ms_a = (int32_t)((float)__builtin_bit_cast(_Float16, h) * sc_a);
            #pragma unroll
            for (int j = 0; j < TT; j++) {
                const v4i d = block_dot(X.B[u][j], wA);
                #pragma unroll
                for (int i = 0; i < 4; i++) acc_a[j][i] += (int64_t)d[i] * ms_a;
            }
            if constexpr (PAIRED) {
                const long wB = unpack_codes(X.A2[u]);
                const unsigned short h2 = (unsigned short)(X.S2[u >> 1] >> (16 * (u & 1)));
                const int32_t ms_b = (int32_t)((float)__builtin_bit_cast(_Float16, h2) * sc_b);
                #pragma unroll
                for (int j = 0; j < TT; j++) {
                    const v4i d = block_dot(X.B[u][j], wB);
                    #pragma unroll
                    for (int i = 0; i < 4; i++) acc_b[j][i] += (int64_t)d[i] * ms_b;
                }
            }
        }
    };
    // a ring of register buffers: with one tile per wave, three groups' loads
    // are in flight while the fourth runs through the matrix cores (the loads'
    // latency under load is several times one group's work); two tiles per
    // wave double the work per group and leave room for two buffers
    if constexpr (TT == 1) {
        Buf X0, X1, X2, X3;
        load(X0, 0);
        load(X1, U);
        load(X2, 2 * U);
        for (int b0 = 0; b0 < nblk; b0 += 4 * U) {
            load(X3, b0 + 3 * U);
            compute(X0);
            if (b0 + U >= nblk) break;
            load(X0, b0 + 4 * U);
            compute(X1);
            if (b0 + 2 * U >= nblk) break;
            load(X1, b0 + 5 * U);
            compute(X2);
            if (b0 + 3 * U >= nblk) break;
            load(X2, b0 + 6 * U);
            compute(X3);
        }
    } else {
        Buf X, Y;
        load(X, 0);
        for (int b0 = 0; b0 < nblk; b0 += 2 * U) {
            load(Y, b0 + U);
            compute(X);
            if (b0 + U >= nblk) break;
            load(X, b0 + 2 * U);
            compute(Y);
        }
    }
    // outputs: lane holds row `row` for tokens t0 + 16j + 4g + i
    #pragma unroll
    for (int j = 0; j < TT; j++)
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + 16 * j + 4 * g + i;
            if (t >= a.T) continue;
            const int sh = a.sh[t];
            const float ya = sh == SH_ZERO ? 0.0f : rne_i64_scaled(acc_a[j][i], eb_a - sh);
            if (PAIRED) {
                const float yb = sh == SH_ZERO ? 0.0f : rne_i64_scaled(acc_b[j][i], eb_b - sh);
                const size_t o = (size_t)t * wa.rows + row;
                a.seg[0].out[o] = ya; a.seg[1].out[o] = yb;
                a.act_out[o] = act_apply(ya, yb, a.act, a.mode);
            } else {
                a.seg[s].out[(size_t)t * wa.rows + row] = ya;
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
    // the kernel's buffer offsets are 32-bit: planes (3 x nblk x TP x 32 bytes)
    // and one 16-row slice of codes / scales
    if ((size_t)3 * (a.cols / 32) * a.TP * 32 >= ((size_t)1 << 31)) { fprintf(stderr, "kvd: GEMM planes too large\n"); abort(); }
    // 32-token tiles per wave (codes unpacked and scales decoded once for two
    // tiles) when that still gives >= 512 workgroups, else 16-token tiles
    if ((nrows_total / 64) * (a.TP / 32) < 512) {
        const dim3 grid(nrows_total / 64, a.TP / 16);
        if (paired) hipLaunchKernelGGL((k_gemm_q4b<true, 1>), grid, dim3(256), 0, s, a);
        else        hipLaunchKernelGGL((k_gemm_q4b<false, 1>), grid, dim3(256), 0, s, a);
    } else {
        const dim3 grid(nrows_total / 64, a.TP / 32);
        if (paired) hipLaunchKernelGGL((k_gemm_q4b<true, 2>), grid, dim3(256), 0, s, a);
        else        hipLaunchKernelGGL((k_gemm_q4b<false, 2>), grid, dim3(256), 0, s, a);
    }
}

}  // namespace kvd
