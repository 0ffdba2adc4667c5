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
// and one or two 16-token MFMA tiles that share its unpacked weight codes.
// The activation planes, which all four waves read, go through LDS once per
// workgroup; each wave streams its own codes and scales.
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

// d = sum_k code_k * xq_k over one 32-column block for a 16-token x 16-row
// tile: one independent MFMA per digit plane, combined as
// (p2 * 256 + p1) * 256 + p0 (|d| < 2^31, exact in int32)
__device__ __forceinline__ v4i block_dot(long b0, long b1, long b2, long w) {
    const v4i z = {0, 0, 0, 0};
    const v4i p0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(b0, w, z, 0, 0, 0);
    const v4i p1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(b1, w, z, 0, 0, 0);
    const v4i p2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(b2, w, z, 0, 0, 0);
    return (((p2 << 8) + p1) << 8) + p0;
}

// raw buffer access: a wave-uniform base in the resource, a fixed per-lane
// byte offset, the per-iteration offset in a scalar register; reads past
// `bytes` return zero
constexpr int BUF_WORD3 = 0x00020000;                  // 32-bit data format, raw access
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, BUF_WORD3);
}
__device__ __forceinline__ uint4 buf_ld128(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const u4 v = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
    return make_uint4(v.x, v.y, v.z, v.w);
}
// 4 x 4 transpose across the four 16-lane rows of a wave: afterwards lane row
// r, register k holds what lane row k held in register r (same lane in the row)
__device__ __forceinline__ void transpose4(uint4 &v) {
    const auto a = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    v = make_uint4(c[0], c[1], d[0], d[1]);
}

constexpr int GEMM_KC = 8;                // 32-column blocks per pipeline chunk
constexpr int GEMM_AG = GEMM_KC / 4;      // 16-byte code loads per lane and chunk
constexpr int GEMM_SPLIT_TARGET = 2048;   // workgroups a split-K launch aims for

// A wave's own operands of one chunk: the codes of its 16 rows (a lane loads
// 16 bytes = 4 blocks of its row; transpose4 turns that into one dword per
// block), the 8 f16 scales of the lane's row.
template <bool PAIRED> struct WaveChunk {
    uint4 A[GEMM_AG], A2[PAIRED ? GEMM_AG : 1];
    uint4 S, S2;
};

// A workgroup (4 waves) owns 64 weight rows x TT 16-token tiles; a wave owns
// 16 rows.  The activations are the MFMA's A operand and the weight codes its
// B operand, so a lane's outputs are one weight row (16-lane index) x 4
// tokens, and each block's scale is decoded once per lane: the exact integer
// Ms = M * 2^(e - ebase) = f16 * 2^-ebase (below 2^31 for every row the GEMM
// takes); each block adds d * Ms to the int64 total.
//
// The K dimension runs in chunks of GEMM_KC blocks.  A chunk's activation
// planes (3 planes x TT tiles x 512 bytes per block), which all four waves
// read, are loaded once per workgroup with 16-byte loads, parked in registers
// for one chunk and written to one of two LDS buffers; the MFMAs read them
// back with ds_read_b64.  Each wave loads its own codes 16 bytes per lane and
// its scales 16 bytes per lane (8 blocks) one chunk ahead.  All buffer
// offsets are 32-bit (checked by the launcher).
template <bool PAIRED, int TT, bool SPLIT>
__global__ __launch_bounds__(256) void k_gemm_q4b(GemmArgs a) {
    constexpr int KC = GEMM_KC, AG = GEMM_AG;
    constexpr int SEG = 3 * TT;                        // 512-byte tiles per block (planes x token tiles)
    constexpr int PPT = KC * SEG * 32 / 256;           // 16-byte staging pieces per thread and chunk
    __shared__ uint4 Bs[2][KC * SEG * 32];             // [buf][(kb * 3 + p) * TT + j][32 pieces]
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c16 = lane & 15, g = lane >> 4;
    // row tile -> segment (segment row counts are multiples of 64)
    int tile_row = blockIdx.x * 64, s = 0;
    if (!PAIRED) while (s < a.nseg - 1 && tile_row >= a.seg[s].w.rows) { tile_row -= a.seg[s].w.rows; s++; }
    const DevW &wa = a.seg[s].w;
    const DevW &wb = a.seg[PAIRED ? 1 : s].w;
    const int nblk = wa.nblk, TP = a.TP, rb = wa.cols / 2;
    // split K: this workgroup's chunks [ckb, ckb + nck) of the nblk / KC
    const int kper = (nblk / KC + (int)gridDim.z - 1) / (int)gridDim.z;
    const int ckb = (int)blockIdx.z * kper;
    const int nck = nblk / KC - ckb < kper ? nblk / KC - ckb : kper;
    const int rbase = tile_row + wave * 16, t0 = blockIdx.y * 16 * TT, row = rbase + c16;
    const __amdgpu_buffer_rsrc_t rca = buf_rsrc(wa.codes + (size_t)rbase * rb, 16u * rb);
    const __amdgpu_buffer_rsrc_t rcb = buf_rsrc(wb.codes + (size_t)rbase * rb, 16u * rb);
    const int lo_c = c16 * rb + 16 * g;                // lane's 16 bytes of a 4-block group of its row
    const int pstride = nblk * TP * 32;                // bytes per plane
    const __amdgpu_buffer_rsrc_t rpl = buf_rsrc(a.planes + (size_t)t0 * 32, 3u * pstride - 32u * t0);
    const __amdgpu_buffer_rsrc_t rsa = buf_rsrc(wa.bs + (size_t)rbase * nblk, 32u * nblk);
    const __amdgpu_buffer_rsrc_t rsb = buf_rsrc(wb.bs + (size_t)rbase * nblk, 32u * nblk);
    const int lo_s = c16 * nblk * 2;
    const int eb_a = wa.ebase[row], eb_b = PAIRED ? wb.ebase[row] : 0;
    const float sc_a = ldexpf(1.0f, -eb_a), sc_b = ldexpf(1.0f, -eb_b);
    // staging piece q = tid + 256 r: tile q / 32, 16 bytes at (q % 32) * 16
    int goff[PPT];
    #pragma unroll
    for (int r = 0; r < PPT; r++) {
        const int q = tid + 256 * r, sg = q / 32, kb = sg / SEG, p = (sg % SEG) / TT, j = sg % TT;
        goff[r] = p * pstride + (kb * TP + 16 * j) * 32 + (q % 32) * 16;
    }
    auto stage_load = [&](uint4 (&st)[PPT], int ck) {
        const int so = __builtin_amdgcn_readfirstlane((ckb + ck) * KC * TP * 32);
        #pragma unroll
        for (int r = 0; r < PPT; r++) st[r] = buf_ld128(rpl, goff[r], so);
    };
    auto stage_store = [&](const uint4 (&st)[PPT], int buf) {
        #pragma unroll
        for (int r = 0; r < PPT; r++) Bs[buf][tid + 256 * r] = st[r];
    };
    auto wave_load = [&](WaveChunk<PAIRED> &w, int ck) {
        const int b0 = __builtin_amdgcn_readfirstlane((ckb + ck) * KC);
        #pragma unroll
        for (int q = 0; q < AG; q++) {
            w.A[q] = buf_ld128(rca, lo_c, (b0 + 4 * q) * 16);
            if constexpr (PAIRED) w.A2[q] = buf_ld128(rcb, lo_c, (b0 + 4 * q) * 16);
        }
        w.S = buf_ld128(rsa, lo_s, b0 * 2);
        if constexpr (PAIRED) w.S2 = buf_ld128(rsb, lo_s, b0 * 2);
    };
    int64_t acc_a[TT][4], acc_b[TT][4];
    #pragma unroll
    for (int j = 0; j < TT; j++)
        #pragma unroll
        for (int i = 0; i < 4; i++) { acc_a[j][i] = 0; acc_b[j][i] = 0; }
    auto pick = [](const uint4 &v, int k) { return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w; };
    auto compute = [&](const WaveChunk<PAIRED> &w, int buf) {
        uint4 At[AG], A2t[PAIRED ? AG : 1];
        #pragma unroll
        for (int q = 0; q < AG; q++) {
            At[q] = w.A[q]; transpose4(At[q]);
            if constexpr (PAIRED) { A2t[q] = w.A2[q]; transpose4(A2t[q]); }
        }
        const uint32_t sa[4] = {w.S.x, w.S.y, w.S.z, w.S.w};
        const uint32_t sb[4] = {w.S2.x, w.S2.y, w.S2.z, w.S2.w};
        #pragma unroll
        for (int kb = 0; kb < KC; kb++) {
            const long wA = unpack_codes(pick(At[kb / 4], kb & 3));
            const unsigned short h = (unsigned short)(sa[kb >> 1] >> (16 * (kb & 1)));
            const int32_t ms_a = (int32_t)((float)__builtin_bit_cast(_Float16, h) * sc_a);
            long B[TT][3];
            #pragma unroll
            for (int j = 0; j < TT; j++)
                #pragma unroll
                for (int p = 0; p < 3; p++)
                    B[j][p] = ((const long *)&Bs[buf][((kb * 3 + p) * TT + j) * 32])[c16 * 4 + g];
            #pragma unroll
            for (int j = 0; j < TT; j++) {
                const v4i d = block_dot(B[j][0], B[j][1], B[j][2], wA);
                #pragma unroll
                for (int i = 0; i < 4; i++) acc_a[j][i] += (int64_t)d[i] * ms_a;
            }
            if constexpr (PAIRED) {
                const long wB = unpack_codes(pick(A2t[kb / 4], kb & 3));
                const unsigned short h2 = (unsigned short)(sb[kb >> 1] >> (16 * (kb & 1)));
                const int32_t ms_b = (int32_t)((float)__builtin_bit_cast(_Float16, h2) * sc_b);
                #pragma unroll
                for (int j = 0; j < TT; j++) {
                    const v4i d = block_dot(B[j][0], B[j][1], B[j][2], wB);
                    #pragma unroll
                    for (int i = 0; i < 4; i++) acc_b[j][i] += (int64_t)d[i] * ms_b;
                }
            }
            // keep each block's products in order: reassociating the int64 sums
            // across blocks would hold every block's MFMA results live at once
            #pragma unroll
            for (int j = 0; j < TT; j++)
                #pragma unroll
                for (int i = 0; i < 4; i++) {
                    asm volatile("" : "+v"(acc_a[j][i]));
                    if constexpr (PAIRED) asm volatile("" : "+v"(acc_b[j][i]));
                }
        }
    };
    // pipeline: chunk ck computes from LDS buffer ck % 2 while the next
    // chunk's activation pieces wait in registers for the other buffer; a
    // wave's codes and scales are requested right after their registers' use.
    // Every buffer write is separated from the previous reads of that buffer
    // by the barrier that published the other buffer.
    // Without split K the loads for chunks past the last are issued too, as
    // repeats of the last chunk (cache hits, values unused): a load under a
    // condition is not counted by the compiler's waits, and the waits for the
    // chunk being computed would then wait for the next chunk's loads as well.
    // A split's few chunks end in a hand-off that waits for every load, so
    // there the extra loads would only delay it: they stay conditional.
    auto cl = [&](int ck) { return ck < nck ? ck : nck - 1; };
    auto want = [&](int ck) { return !SPLIT || ck < nck; };
    uint4 st0[PPT], st1[PPT];
    WaveChunk<PAIRED> w0, w1;
    stage_load(st0, 0);
    wave_load(w0, 0);
    if (want(1)) { stage_load(st1, cl(1)); wave_load(w1, cl(1)); }
    stage_store(st0, 0);
    __syncthreads();
    for (int ck = 0; ck < nck; ck += 2) {
        if (want(ck + 2)) stage_load(st0, cl(ck + 2));
        compute(w0, 0);
        if (want(ck + 2)) wave_load(w0, cl(ck + 2));
        if (ck + 1 >= nck) break;
        stage_store(st1, 1);
        __syncthreads();
        if (want(ck + 3)) stage_load(st1, cl(ck + 3));
        compute(w1, 1);
        if (want(ck + 3)) wave_load(w1, cl(ck + 3));
        if (ck + 2 >= nck) break;
        stage_store(st0, 0);
        __syncthreads();
    }
    if constexpr (SPLIT) {
        // split K: every split stores its exact partials in its own slice
        // (agent-scope stores, coherent across the XCDs' L2s); the last split
        // of the tile to arrive adds the others' to its own
        const int grow = (int)blockIdx.x * 64 + wave * 16 + c16;   // the row among the launch's rows
        const size_t zs = (size_t)TP * a.arows;
        int64_t *mine = a.part + blockIdx.z * zs;
        #pragma unroll
        for (int j = 0; j < TT; j++)
            #pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = t0 + 16 * j + 4 * g + i;
                st_agent(&mine[(size_t)t * a.arows + grow], acc_a[j][i]);
                if constexpr (PAIRED) st_agent(&mine[(size_t)t * a.arows + a.arows / 2 + grow], acc_b[j][i]);
            }
        mem_complete();
        __shared__ int last;
        __syncthreads();
        int *cnt = a.cnt + blockIdx.y * gridDim.x + blockIdx.x;
        if (threadIdx.x == 0) last = arrive(cnt) == (int)gridDim.z - 1;
        __syncthreads();
        if (!last) return;
        for (int z = 0; z < (int)gridDim.z; z++) {
            if (z == (int)blockIdx.z) continue;
            const int64_t *other = a.part + z * zs;
            #pragma unroll
            for (int j = 0; j < TT; j++)
                #pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = t0 + 16 * j + 4 * g + i;
                    acc_a[j][i] += ld_agent(&other[(size_t)t * a.arows + grow]);
                    if constexpr (PAIRED) acc_b[j][i] += ld_agent(&other[(size_t)t * a.arows + a.arows / 2 + grow]);
                }
        }
        if (threadIdx.x == 0) reset_counter(cnt);
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
    if (a.pro.n % 32 || a.TP % 32 || a.T > a.TP) { launch_fail("GEMM staging shape outside the kernel's limits"); return; }
    switch (a.pro.kind) {
    case PRO_PLAIN: hipLaunchKernelGGL(k_stage<PRO_PLAIN>, dim3(a.TP), dim3(512), lds, s, a); break;
    case PRO_NORM:  hipLaunchKernelGGL(k_stage<PRO_NORM>, dim3(a.TP), dim3(512), lds, s, a); break;
    default:        hipLaunchKernelGGL(k_stage<PRO_RESID>, dim3(a.TP), dim3(512), lds, s, a); break;
    }
}

bool gemm_supported(const DevW &w) {
    return !w.wide && w.rows % 64 == 0 && w.cols % (32 * GEMM_KC) == 0;
}

void launch_gemm(const GemmArgs &a, int nrows_total, hipStream_t s) {
    const bool paired = a.act != ACT_NONE;
    for (int i = 0; i < a.nseg; i++)
        if (!gemm_supported(a.seg[i].w) || a.seg[i].w.cols != a.cols) {
            launch_fail("GEMM segment shape not supported"); return;
        }
    if (nrows_total % 64 || a.TP % 32 || a.T > a.TP) { launch_fail("GEMM rows or token count outside the kernel's limits"); return; }
    // the kernel's buffer offsets are 32-bit: planes (3 x nblk x TP x 32 bytes)
    // and one 16-row slice of codes / scales
    if ((size_t)3 * (a.cols / 32) * a.TP * 32 >= ((size_t)1 << 31)) { launch_fail("GEMM activation planes exceed 2 GiB"); return; }
    // 32-token tiles per wave (codes unpacked and scales decoded once for two
    // tiles) when that still gives >= 512 workgroups, else 16-token tiles
    // (LDS: 24 KiB per workgroup with 16-token tiles, 48 KiB with 32)
    const bool tt2 = (nrows_total / 64) * (a.TP / 32) >= 512;
    dim3 grid(nrows_total / 64, a.TP / (tt2 ? 32 : 16), 1);
    // split K where the tiles alone leave the device under two workgroups per
    // CU (about eight wanted), with at least two chunks per split and the
    // splits' partial slices inside the buffer
    GemmArgs g = a;
    g.arows = nrows_total * (paired ? 2 : 1);
    const int nck = a.cols / 32 / GEMM_KC, tiles = (int)(grid.x * grid.y);
    int ks = 1;
    if (a.part && a.cnt && tiles <= a.cnt_cap && tiles < GEMM_SPLIT_TARGET / 4) {
        ks = (GEMM_SPLIT_TARGET + tiles - 1) / tiles;
        if (ks > nck / 2) ks = nck / 2;
        const size_t slice = (size_t)a.TP * g.arows;
        if (ks > 1 && (size_t)ks * slice > a.part_cap) ks = (int)(a.part_cap / slice);
        if (ks < 1) ks = 1;
        const int kper = (nck + ks - 1) / ks;
        ks = (nck + kper - 1) / kper;                  // every split holds chunks
    }
    grid.z = ks;
    const int inst = (paired ? 4 : 0) + (tt2 ? 2 : 0) + (ks > 1 ? 1 : 0);
    switch (inst) {
    case 0: hipLaunchKernelGGL((k_gemm_q4b<false, 1, false>), grid, dim3(256), 0, s, g); break;
    case 1: hipLaunchKernelGGL((k_gemm_q4b<false, 1, true>), grid, dim3(256), 0, s, g); break;
    case 2: hipLaunchKernelGGL((k_gemm_q4b<false, 2, false>), grid, dim3(256), 0, s, g); break;
    case 3: hipLaunchKernelGGL((k_gemm_q4b<false, 2, true>), grid, dim3(256), 0, s, g); break;
    case 4: hipLaunchKernelGGL((k_gemm_q4b<true, 1, false>), grid, dim3(256), 0, s, g); break;
    case 5: hipLaunchKernelGGL((k_gemm_q4b<true, 1, true>), grid, dim3(256), 0, s, g); break;
    case 6: hipLaunchKernelGGL((k_gemm_q4b<true, 2, false>), grid, dim3(256), 0, s, g); break;
    default: hipLaunchKernelGGL((k_gemm_q4b<true, 2, true>), grid, dim3(256), 0, s, g); break;
    }
}

}  // namespace kvd
