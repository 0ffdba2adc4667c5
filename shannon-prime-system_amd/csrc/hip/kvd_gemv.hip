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
#include "kvd_vec.h"
#include <hip/hip_ext.h>
#include <cstdio>
#include <cstdlib>

namespace kvd {

// ------------------------------------------------------- prologue
// Builds the GEMV input (input_transform) and the digit planes of the
// workgroup's column split [b_lo, b_hi) blocks (in dig, indexed from b_lo).
// Returns sh, or SH_ZERO for an all-zero input.
// xq = rne(x * 2^sh) as six balanced base-16 digits, 8 columns per dword and
// plane.  u = xq + 0x888888 has the digits + 8 as its plain nibbles (|xq| <=
// 2^22 keeps 0 <= u < 16^6), so digit & 15 = nibble ^ 8.  x * 2^sh is exact in
// float for every result that can round to a non-zero integer.
// The 6 x 8 nibble transpose runs on bytes: v_perm_b32 gathers byte b of the
// even columns (D0[b]) and of the odd columns (D1[b]); the low nibbles of
// D0[b] | D1[b] << 4 are then plane 2b in column order, the high nibbles plane
// 2b + 1 (one bitfield insert each).
__device__ __forceinline__ void digits8(const float v[8], int sh, uint32_t dw[NDIG]) {
    uint32_t u[8];
    #pragma unroll
    for (int j = 0; j < 8; j++) u[j] = (uint32_t)((int32_t)rintf(ldexpf(v[j], sh)) + 0x888888);
    // bytes 0..2 of columns a, b, c, d, in that order, one dword per byte
    auto gather = [](uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t (&D)[3]) {
        const uint32_t p01 = __builtin_amdgcn_perm(b, a, 0x05010400u);   // a.0 b.0 a.1 b.1
        const uint32_t p2 = __builtin_amdgcn_perm(b, a, 0x0C0C0602u);    // a.2 b.2 0 0
        const uint32_t q01 = __builtin_amdgcn_perm(d, c, 0x05010400u);
        const uint32_t q2 = __builtin_amdgcn_perm(d, c, 0x0C0C0602u);
        D[0] = __builtin_amdgcn_perm(q01, p01, 0x05040100u);
        D[1] = __builtin_amdgcn_perm(q01, p01, 0x07060302u);
        D[2] = __builtin_amdgcn_perm(q2, p2, 0x05040100u);
    };
    uint32_t D0[3], D1[3];
    gather(u[0], u[2], u[4], u[6], D0);
    gather(u[1], u[3], u[5], u[7], D1);
    #pragma unroll
    for (int b = 0; b < 3; b++) {
        dw[2 * b] = ((D0[b] & 0x0F0F0F0Fu) | ((D1[b] << 4) & 0xF0F0F0F0u)) ^ 0x88888888u;
        dw[2 * b + 1] = (((D0[b] >> 4) & 0x0F0F0F0Fu) | (D1[b] & 0xF0F0F0F0u)) ^ 0x88888888u;
    }
}

// The prologue's global loads (pro_load, plus for PRO_PLAIN this thread's
// first 8 input columns of the split), issued before the weight prefetch.
struct GemvLoads { ProLoads pro; float4 c0, c1; };
template <int PRO>
__device__ __forceinline__ void gemv_pro_load(const ProArgs &p, int mode, GemvLoads &L, int b_lo, int b_hi) {
    pro_load<PRO>(p, mode, L.pro);
    if constexpr (PRO == PRO_PLAIN) {
        const int g = b_lo * 4 + (int)threadIdx.x, gc = g < b_hi * 4 ? g : b_lo * 4;   // in range: read, used only if g is
        L.c0 = *(const float4 *)(p.x + gc * 8);
        L.c1 = *(const float4 *)(p.x + gc * 8 + 4);
    }
}

template <int PRO>
__device__ __forceinline__ int gemv_prologue(const ProArgs &p, int mode, const GemvLoads &L, float *xf, uint4 *dig, int b_lo, int b_hi, void *red) {
    const int T = blockDim.x, tid = threadIdx.x;
    DigOut dout{dig, b_lo, b_hi - b_lo, false};
    const int sh = input_transform<PRO>(p, mode, L.pro, xf, red, blockIdx.x == 0, b_lo * 32, b_hi * 32,
                                        PRO == PRO_PLAIN ? nullptr : &dout);
    if (sh == SH_ZERO || dout.done) return sh;
    // digits: one thread per 8 consecutive columns (one nibble-dword per plane);
    // the column count is a multiple of 32, so a group never runs past n
    const float *src = PRO == PRO_PLAIN ? p.x : xf;
    const int g_lo = b_lo * 4, g_hi = b_hi * 4, nb = b_hi - b_lo;
    auto put = [&](int g, const float4 &v0, const float4 &v1) {
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        uint32_t dw[NDIG];
        digits8(v, sh, dw);
        const int b = (g >> 2) - b_lo, q = g & 3;
        #pragma unroll
        for (int k = 0; k < NDIG; k++) ((uint32_t *)&dig[k * nb + b])[q] = dw[k];
    };
    int g = g_lo + tid;
    if constexpr (PRO == PRO_PLAIN) {
        // the preloaded first group, outside the loop: a loop body shared with
        // loaded groups would make its waits cover the weight prefetch
        if (g < g_hi) put(g, L.c0, L.c1);
        g += T;
    }
    for (; g < g_hi; g += T) put(g, *(const float4 *)(src + g * 8), *(const float4 *)(src + g * 8 + 4));
    __syncthreads();
    return sh;
}

// ------------------------------------------------------- main kernel
constexpr int64_t SPLIT_TAG = (int64_t)1 << 62;          // marks a parked split partial
__device__ __forceinline__ int32_t dot_digits(const uint4 c, const uint4 *D) {
    // sum over the 32 codes of code * xq, xq = sum_k 16^k digit_k, Horner form
    // folded into the dot accumulator: a = 16 a + dots of plane k (|a| < 2^30
    // at the end; 32-bit wrap-around in between cancels exactly)
    int32_t a = 0;
    #pragma unroll
    for (int k = NDIG - 1; k >= 0; k--) {
        a = (int32_t)((uint32_t)a << 4);
        a = __builtin_amdgcn_sdot8((int)c.x, (int)D[k].x, a, false);
        a = __builtin_amdgcn_sdot8((int)c.y, (int)D[k].y, a, false);
        a = __builtin_amdgcn_sdot8((int)c.z, (int)D[k].z, a, false);
        a = __builtin_amdgcn_sdot8((int)c.w, (int)D[k].w, a, false);
    }
    return a;
}

// The exact block multiplier Ms = M * 2^(e - ebase) of an f16 scale M * 2^e
// relative to its row's smallest block exponent: an integer below 2^31 for
// every row that is not WIDE (the host sets WIDE when a row's exponent spread
// could exceed 21 - ceil(log2 nblk); one block has no spread).  The f16 -> f32
// conversion, the scaling by 2^-ebase and the conversion to int32 are exact.
__device__ __forceinline__ int32_t block_mult(uint32_t h, int ebase) {
    return (int32_t)ldexpf((float)__builtin_bit_cast(_Float16, (unsigned short)h), -ebase);
}

// Cross-lane moves without LDS round trips (CDNA4 VALU lane permutes):
// v_permlane32_swap swaps the upper half of its first operand with the lower
// half of its second; v_permlane16_swap the odd 16-lane rows of the first with
// the even rows of the second.
struct U32Pair { uint32_t a, b; };
__device__ __forceinline__ U32Pair swap32(uint32_t x, uint32_t y) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
    return {r[0], r[1]};
}
__device__ __forceinline__ U32Pair swap16(uint32_t x, uint32_t y) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, y, false, false);
    return {r[0], r[1]};
}
// x from lane l ^ 32
__device__ __forceinline__ uint32_t xor32_u(uint32_t x, int lane) {
    const U32Pair p = swap32(x, x);          // a: lanes 0..31 of x twice, b: lanes 32..63 twice
    return lane < 32 ? p.b : p.a;
}
__device__ __forceinline__ float xor32_f(float x, int lane) { return __uint_as_float(xor32_u(__float_as_uint(x), lane)); }
__device__ __forceinline__ int xor32_i(int x, int lane) { return (int)xor32_u((uint32_t)x, lane); }
// lanes 0..31: x(l) + x(l + 32); lanes 32..63: y(l - 32) + y(l)
__device__ __forceinline__ int64_t fold32(int64_t x, int64_t y) {
    const U32Pair lo = swap32((uint32_t)x, (uint32_t)y), hi = swap32((uint32_t)((uint64_t)x >> 32), (uint32_t)((uint64_t)y >> 32));
    return (int64_t)(((uint64_t)hi.a << 32) | lo.a) + (int64_t)(((uint64_t)hi.b << 32) | lo.b);
}
// rows 0, 2: x(row) + x(row + 1); rows 1, 3: y(row - 1) + y(row)
__device__ __forceinline__ int64_t fold16(int64_t x, int64_t y) {
    const U32Pair lo = swap16((uint32_t)x, (uint32_t)y), hi = swap16((uint32_t)((uint64_t)x >> 32), (uint32_t)((uint64_t)y >> 32));
    return (int64_t)(((uint64_t)hi.a << 32) | lo.a) + (int64_t)(((uint64_t)hi.b << 32) | lo.b);
}

// Sum GEMV_R = 8 per-lane int64 partials over the wave: each step halves the
// rows a lane carries (lane halves, then 16-lane rows, then half rows), and
// the last three sum within groups of 8 lanes.  Afterwards lane l holds the
// total of row ((l>>5)&1)*4 + ((l>>4)&1)*2 + ((l>>3)&1) (all lanes of an
// aligned group of 8 agree).
__device__ __forceinline__ int64_t transpose_reduce8(const int64_t v[8], int lane) {
    const bool hi8 = lane & 8;
    int64_t w[4], x[2];
    #pragma unroll
    for (int r = 0; r < 4; r++) w[r] = fold32(v[r], v[r + 4]);      // lanes >= 32 carry rows 4..7
    #pragma unroll
    for (int r = 0; r < 2; r++) x[r] = fold16(w[r], w[r + 2]);      // odd rows carry rows +2
    // half rows: lane l keeps its row (bit 3) and takes the other row from l ^ 8
    const uint64_t keep = (uint64_t)(hi8 ? x[1] : x[0]), send = (uint64_t)(hi8 ? x[0] : x[1]);
    int64_t y = (int64_t)(keep + dpp64<0x128, 0xF>(send, 0));        // row_ror:8
    y += (int64_t)dpp64<0xB1, 0xF>((uint64_t)y, 0);                  // quad_perm 1,0,3,2
    y += (int64_t)dpp64<0x4E, 0xF>((uint64_t)y, 0);                  // quad_perm 2,3,0,1
    y += (int64_t)dpp64<0x141, 0xF>((uint64_t)y, 0);                 // row_half_mirror
    return y;
}

// One wave task: GEMV_R rows (paired: HR gate + HR up rows) over the
// workgroup's column split.  All fields are wave-uniform.
struct Task { int seg, row0, nvalid, grow0; };

template <bool PAIRED>
__device__ __forceinline__ Task task_of(const GemvArgs &a, int grp) {
    Task t;
    if (PAIRED) {
        const int rows0 = a.seg[0].w.rows;
        t.seg = 0; t.row0 = grp * (GEMV_R / 2);
        t.nvalid = rows0 - t.row0 < GEMV_R / 2 ? rows0 - t.row0 : GEMV_R / 2;
        t.grow0 = t.row0;
    } else {
        // a group never straddles segments (segment row counts are multiples
        // of GEMV_R, checked by the host), so its rows are consecutive
        int g = grp * GEMV_R, s = 0, off = 0, rows = a.seg[0].w.rows;
        while (s < a.nseg - 1 && g >= rows) { g -= rows; off += rows; s++; rows = a.seg[s].w.rows; }
        t.seg = s; t.row0 = g; t.grow0 = off + g;
        t.nvalid = rows - g < GEMV_R ? rows - g : GEMV_R;
    }
    t.seg = __builtin_amdgcn_readfirstlane(t.seg);
    t.row0 = __builtin_amdgcn_readfirstlane(t.row0);
    t.nvalid = __builtin_amdgcn_readfirstlane(t.nvalid);
    t.grow0 = __builtin_amdgcn_readfirstlane(t.grow0);
    return t;
}

// 16 B of codes and the f16 scale of block b for each of the task's rows.
// Every load is issued, at a valid address (rows past the end re-read the
// task's first row, b >= b_hi re-reads block b_lo): a conditional load would
// leave the compiler unsure how many loads are in flight, and its waits for
// earlier loads would then wait for these too.  Users ignore those values
// (b >= b_hi is skipped, rows past the end are never written).
template <bool PAIRED>
__device__ __forceinline__ void load_iter(const GemvArgs &a, const Task &t, int b, int b_lo, int b_hi,
                                          uint4 c[GEMV_R], uint32_t h[GEMV_R]) {
    const int per = PAIRED ? GEMV_R / 2 : GEMV_R;
    const DevW &wa = a.seg[t.seg].w;
    const DevW &wb = a.seg[PAIRED ? 1 : t.seg].w;
    const int nblk = wa.nblk;
    const size_t rb = (size_t)(wa.cols + 1) / 2;
    const int bc = b < b_hi ? b : b_lo;
    #pragma unroll
    for (int r = 0; r < GEMV_R; r++) {
        const int rr = r % per;
        const int row = t.row0 + (rr < t.nvalid ? rr : 0);
        const bool second = PAIRED && r >= per;
        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
        const DevW &w = second ? wb : wa;
        const uint8_t *cp = w.codes + (size_t)row * rb + (size_t)bc * 16;
        const u32x4 v = __builtin_nontemporal_load((const u32x4 *)cp);
        c[r] = make_uint4(v.x, v.y, v.z, v.w);
    }
    // the scales from the interleaved copy: one load per matrix (paired: the
    // 4-row groups of gate and up; rows past the end are zero padding)
    if constexpr (PAIRED) {
        const size_t gi = ((size_t)(t.row0 >> 2) * nblk + bc) * 4;
        const uint2 ga = *(const uint2 *)(wa.bs8 + gi), gb = *(const uint2 *)(wb.bs8 + gi);
        h[0] = ga.x & 0xffffu; h[1] = ga.x >> 16; h[2] = ga.y & 0xffffu; h[3] = ga.y >> 16;
        h[4] = gb.x & 0xffffu; h[5] = gb.x >> 16; h[6] = gb.y & 0xffffu; h[7] = gb.y >> 16;
    } else {
        const uint4 g = *(const uint4 *)(wa.bs8 + ((size_t)(t.row0 >> 3) * nblk + bc) * 8);
        h[0] = g.x & 0xffffu; h[1] = g.x >> 16; h[2] = g.y & 0xffffu; h[3] = g.y >> 16;
        h[4] = g.z & 0xffffu; h[5] = g.z >> 16; h[6] = g.w & 0xffffu; h[7] = g.w >> 16;
    }
}

// The task's row exponent bases, row r's in byte r (paired: gate rows, then
// up rows): one load per half.  The host pads every ebase array by 8 bytes,
// so the read may run past the last row; those rows are never written.
template <bool PAIRED, bool WIDE>
__device__ __forceinline__ uint64_t load_eb(const GemvArgs &a, const Task &t) {
    if constexpr (WIDE) return 0;
    if constexpr (PAIRED) {
        const uint32_t lo = *(const uint32_t *)(a.seg[0].w.ebase + t.row0);
        const uint32_t hi = *(const uint32_t *)(a.seg[1].w.ebase + t.row0);
        return (uint64_t)hi << 32 | lo;
    }
    return *(const uint64_t *)(a.seg[t.seg].w.ebase + t.row0);
}
__device__ __forceinline__ int eb_of(uint64_t ebw, int r) { return (int)(int8_t)(ebw >> (8 * r)); }

// The matrix pass.  Workgroup w works on column split s = w % nsplit (blocks
// [s*bps, min(nblk, (s+1)*bps)) ); its waves take row groups in a grid stride.
// With nsplit > 1 every task adds its exact int64 row partials atomically into
// accbuf (order-free, so still bit-exact); the wave that completes a group's
// last split converts the totals, writes the outputs and clears accbuf/gcnt
// for the next launch.  Two splits of unpaired rows need no counter: each row's
// partials meet through one atomic exchange on its accbuf slot.  The first weights are requested before the prologue
// (after the prologue's own loads), and each task requests the next task's
// weights before its own epilogue.
// PAIRED (gate/up) and the plain-input instances (O, down) hold one workgroup
// per CU (the plan sees to it) and may use 256 registers: a task over two
// 64-block units keeps both in flight; the residual and norm instances (QKV,
// LM head) run up to 4 waves per SIMD, two workgroups per CU.
template <int PRO, bool PAIRED, bool WIDE>
__global__ __launch_bounds__(512, (PAIRED || PRO == PRO_PLAIN) ? 2 : 4) void k_gemv(GemvArgs a) {
    extern __shared__ uint4 smem4[];
    const int nblk = (a.cols + 31) / 32, nsplit = a.nsplit, bps = a.bps;
    const int split = blockIdx.x % nsplit;
    const int b_lo = split * bps, b_hi = b_lo + bps < nblk ? b_lo + bps : nblk, nb = b_hi - b_lo;
    uint4 *dig = smem4;                                   // NDIG * nb
    float *xf = (float *)(dig + NDIG * nb);               // pro.n floats (norm prologues only)
    __shared__ double red[RED_SLOTS * RED_WAVES];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;
    constexpr int HR = GEMV_R / 2;
    constexpr int per = PAIRED ? HR : GEMV_R;
    const int gstride = (gridDim.x / nsplit) * nwaves;
    int grp = (blockIdx.x / nsplit) * nwaves + wave;

    // the prologue's loads first, then the weights: its waits then need only
    // its own data, and the weight prefetch streams in under its work
    GemvLoads L;
    gemv_pro_load<PRO>(a.pro, a.mode, L, b_lo, b_hi);
    __builtin_amdgcn_sched_barrier(0);
    Task t = task_of<PAIRED>(a, grp < a.groups ? grp : 0);
    uint4 c[GEMV_R];
    uint32_t h[GEMV_R];
    uint64_t ebn = load_eb<PAIRED, WIDE>(a, t);            // first: the task's start waits for it alone
    load_iter<PAIRED>(a, t, b_lo + lane, b_lo, b_hi, c, h);
    __builtin_amdgcn_sched_barrier(0);

    const int sh = gemv_prologue<PRO>(a.pro, a.mode, L, xf, dig, b_lo, b_hi, red);
    const int nit = (nb + 63) / 64;
    StatAcc sacc;                                          // this thread's outputs, for stat_out
    // PAIRED: the exact activation (a few hundred instructions on the holder
    // lanes) runs once per two tasks: a task's (gate, up, row) waits parked in
    // lanes 32.. until the next task's gate rows (lanes 0..31) join it
    bool parked = false;                                   // wave-uniform
    float pg = 0.0f, pu = 0.0f;
    int pj = -1;

    for (; grp < a.groups; grp += gstride) {
        const uint64_t ebw = ebn;                          // this task's (ebn is reloaded for the next)
        typedef typename std::conditional<WIDE, i128, int64_t>::type acc_t;
        acc_t acc[GEMV_R];
        #pragma unroll
        for (int r = 0; r < GEMV_R; r++) acc[r] = 0;
        auto iter = [&](int b, const uint4 (&cc)[GEMV_R], const uint32_t (&hh)[GEMV_R]) {
            if (b < b_hi && sh != SH_ZERO) {
                uint4 D[NDIG];
                #pragma unroll
                for (int k = 0; k < NDIG; k++) D[k] = dig[k * nb + (b - b_lo)];
                #pragma unroll
                for (int r = 0; r < GEMV_R; r++) {
                    const int32_t d = dot_digits(cc[r], D);
                    if constexpr (WIDE) {
                        int32_t M; int e; f16_parts(hh[r], M, e);
                        const int64_t p = (int64_t)d * (int64_t)M;
                        acc[r] += (i128)((u128)(i128)p << (e + 24));
                    } else {
                        // (d * M) << (e - ebase) == d * Ms: one 32 x 32 + 64 multiply-add
                        acc[r] += (int64_t)d * (int64_t)block_mult(hh[r], eb_of(ebw, r));
                    }
                }
            }
        };
        if ((PAIRED || PRO == PRO_PLAIN) && !WIDE && nit == 2) {
            // the second unit is requested before the first is used (these
            // instances have the registers for both)
            uint4 c2[GEMV_R];
            uint32_t h2[GEMV_R];
            load_iter<PAIRED>(a, t, b_lo + 64 + lane, b_lo, b_hi, c2, h2);
            __builtin_amdgcn_sched_barrier(0);
            iter(b_lo + lane, c, h);
            iter(b_lo + 64 + lane, c2, h2);
        } else {
            for (int it = 0; it < nit; it++) {
                const int b = b_lo + it * 64 + lane;
                if (it > 0) load_iter<PAIRED>(a, t, b, b_lo, b_hi, c, h);
                iter(b, c, h);
            }
        }
        // request the next task's first weights before this task's epilogue
        const int ngrp = grp + gstride;
        const Task tn = task_of<PAIRED>(a, ngrp < a.groups ? ngrp : 0);
        ebn = load_eb<PAIRED, WIDE>(a, tn);
        load_iter<PAIRED>(a, tn, b_lo + lane, b_lo, b_hi, c, h);

        if constexpr (WIDE) {
            // int128 rows: whole rows per task (nsplit == 1, enforced by the host)
            float y[GEMV_R];
            #pragma unroll
            for (int r = 0; r < GEMV_R; r++) {
                const i128 tt = wave_sum128(acc[r]);
                y[r] = sh == SH_ZERO ? 0.0f : rne_i128_scaled(tt, -24 - sh);
            }
            // lane r < nvalid writes row r (its value is the statistic's input)
            float yv = 0.0f;
            const bool mine = lane < t.nvalid;
            #pragma unroll
            for (int r = 0; r < GEMV_R; r++) if (lane == r) yv = y[r];
            if (PAIRED) {
                float yu = 0.0f;
                #pragma unroll
                for (int r = 0; r < HR; r++) if (lane == r) yu = y[r + HR];
                if (mine) {
                    const int j = t.row0 + lane;
                    a.seg[0].out[j] = yv; a.seg[1].out[j] = yu;
                    yv = act_apply(yv, yu, a.act, a.mode);
                    a.act_out[j] = yv;
                }
            } else if (mine) {
                a.seg[t.seg].out[t.row0 + lane] = yv;
            }
            if (mine) sacc.add(yv);
        } else {
            int64_t tot = transpose_reduce8(acc, lane);
            const int myrow = ((lane >> 5) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 3) & 1);
            const int rr = myrow % per;
            const bool holder = (lane & 7) == 0 && rr < t.nvalid;
            bool finish = true;                                // per lane on the two-split path
            if (!PAIRED && nsplit == 2) {
                // one atomic exchange per row: the first split to arrive
                // leaves its partial, tagged with 2^62 (|partial| < 2^62: at
                // most 2^lg blocks of |d| <= 2^30 times Ms < 2^(32-lg)), and
                // is done; the second takes it, finishes the row and clears
                // the slot
                int64_t *slot = a.accbuf + t.grow0 + myrow;
                int64_t other = 0;
                if (holder)
                    other = (int64_t)__hip_atomic_exchange((unsigned long long *)slot, (unsigned long long)(tot + SPLIT_TAG),
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                finish = other != 0;
                if (finish) { tot += other - SPLIT_TAG; st_agent(slot, (int64_t)0); }
            } else if (nsplit > 1) {
                int64_t *slot = a.accbuf + (PAIRED ? (myrow >= HR ? a.seg[0].w.rows : 0) + t.row0 + rr : t.grow0 + myrow);
                if (holder) atomicAdd((unsigned long long *)slot, (unsigned long long)tot);
                mem_complete();
                int prev = 0;
                if (lane == 0) prev = arrive(&a.gcnt[grp]);
                prev = __builtin_amdgcn_readlane(prev, 0);
                finish = prev == nsplit - 1;
                if (finish) {
                    if (holder) tot = (int64_t)__hip_atomic_exchange((unsigned long long *)slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (lane == 0) reset_counter(&a.gcnt[grp]);
                }
            }
            if (finish) {
                const int ebm = eb_of(ebw, myrow);
                const float y = sh == SH_ZERO ? 0.0f : rne_i64_scaled(tot, ebm - sh);
                // lane (myrow*8) owns row myrow's total; paired rows fetch their up partner
                const float partner = xor32_f(y, lane);               // row myrow^4
                if (PAIRED) {
                    // lanes 0, 8, 16, 24 hold this task's gate rows (partner:
                    // the up row); lanes 32.. the parked task's
                    const int j = holder && myrow < HR ? t.row0 + myrow : -1;
                    if (j >= 0) { a.seg[0].out[j] = y; a.seg[1].out[j] = partner; }
                    if (parked) {
                        const float g = lane < 32 ? y : pg, u = lane < 32 ? partner : pu;
                        const int jj = lane < 32 ? j : pj;
                        if (jj >= 0) {
                            const float sv = act_apply(g, u, a.act, a.mode);
                            a.act_out[jj] = sv;
                            sacc.add(sv);
                        }
                    } else {
                        // park: lane l + 32 takes lane l's gate value (its own y is the up value)
                        pg = xor32_f(y, lane); pu = y; pj = xor32_i(j, lane);
                        if (lane < 32) pj = -1;
                    }
                    parked = !parked;
                } else if (holder) {
                    a.seg[t.seg].out[t.row0 + myrow] = y;
                    sacc.add(y);
                }
            }
        }
        t = tn;
    }
    if (PAIRED && !WIDE && parked && pj >= 0) {       // the last parked task
        const float sv = act_apply(pg, pu, a.act, a.mode);
        a.act_out[pj] = sv;
        sacc.add(sv);
    }
    if (a.stat_out) stat_flush_block(a.stat_out, sacc);
}

static int g_num_cu = 0;
static int num_cu() {
    if (!g_num_cu) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_num_cu = n;
        else
            g_num_cu = 256;
    }
    return g_num_cu;
}

// Work decomposition: row groups x column splits of 64-block multiples, so
// that about two 8-wave workgroups per CU have work; the grid is a multiple
// of nsplit so that a workgroup keeps one split (and builds only its digits).
GemvPlan gemv_plan(int nrows_total, int cols, int paired, int wide, int one_per_cu) {
    GemvPlan p;
    const int nblk = (cols + 31) / 32;
    p.groups = paired ? (nrows_total + GEMV_R / 2 - 1) / (GEMV_R / 2) : (nrows_total + GEMV_R - 1) / GEMV_R;
    int cap = (one_per_cu ? 1 : 2) * num_cu();          // workgroups resident at once
    const int max_split = (nblk + 63) / 64;
    int want = (cap * GEMV_WAVES + p.groups - 1) / p.groups;
    // a split costs every task an atomic hand-off; it only pays when whole
    // rows would leave more than half of the waves idle
    if (wide || want <= 2) want = 1;
    if ((long long)p.groups * (want < max_split ? want : max_split) <= (long long)cap * GEMV_WAVES) {
        // one round of tasks: one workgroup per CU.  A second workgroup on a
        // CU runs its input transform behind the first one's (older waves
        // issue first), which costs more than the waves it adds; the split
        // then fills the CUs' waves once.
        cap = num_cu();
        want = wide ? 1 : (cap * GEMV_WAVES + p.groups - 1) / p.groups;
    }
    p.nsplit = want < max_split ? want : max_split;
    p.bps = 64 * ((max_split + p.nsplit - 1) / p.nsplit);
    p.nsplit = (nblk + p.bps - 1) / p.bps;
    int per_split = (p.groups + GEMV_WAVES - 1) / GEMV_WAVES;
    const int lim = cap / p.nsplit > 0 ? cap / p.nsplit : 1;
    if (per_split > lim) per_split = lim;
    p.grid = per_split * p.nsplit;
    return p;
}

// Kernel-tight timing: the next GEMV launch on this thread records these
// events at its own start and end (hipExtLaunchKernelGGL), instead of events
// recorded on the stream around it (two more queue packets, ~2 us).
static thread_local hipEvent_t g_t_start = nullptr, g_t_stop = nullptr;
void gemv_time_next(hipEvent_t start, hipEvent_t stop) { g_t_start = start; g_t_stop = stop; }

template <int PRO, bool PAIRED>
static void launch_pro(const GemvArgs &a, bool wide, int grid, int waves, size_t lds, hipStream_t s) {
    hipEvent_t e0 = g_t_start, e1 = g_t_stop;
    g_t_start = g_t_stop = nullptr;
    if (e0) {
        if (wide) hipExtLaunchKernelGGL((k_gemv<PRO, PAIRED, true>), dim3(grid), dim3(waves * 64), lds, s, e0, e1, 0, a);
        else      hipExtLaunchKernelGGL((k_gemv<PRO, PAIRED, false>), dim3(grid), dim3(waves * 64), lds, s, e0, e1, 0, a);
        return;
    }
    if (wide) hipLaunchKernelGGL((k_gemv<PRO, PAIRED, true>), dim3(grid), dim3(waves * 64), lds, s, a);
    else      hipLaunchKernelGGL((k_gemv<PRO, PAIRED, false>), dim3(grid), dim3(waves * 64), lds, s, a);
}

void launch_gemv(const GemvArgs &a_in, int nrows_total, hipStream_t s) {
    GemvArgs a = a_in;
    // a wave's row group must not straddle segments
    for (int i = 0; i + 1 < a.nseg; i++)
        if (a.seg[i].w.rows % GEMV_R) { launch_fail("GEMV segment rows not a multiple of the rows per wave pass"); return; }
    bool wide = false;
    for (int i = 0; i < a.nseg; i++) wide |= a.seg[i].w.wide != 0;
    const bool paired = a.act != ACT_NONE;
    for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].w.il != (paired ? 4 : 8)) { launch_fail("GEMV scale interleave does not match the row pairing"); return; }
    GemvPlan p = gemv_plan(nrows_total, a.cols, paired, wide, paired || a.pro.kind == PRO_PLAIN);
    // A plan that leaves over half of the CUs without a workgroup runs the
    // same waves in half-size workgroups on twice as many CUs (plain inputs
    // only: the norm prologues keep the whole vector in registers of 8 waves)
    int waves = GEMV_WAVES;
    if (a.pro.kind == PRO_PLAIN && p.grid * 2 <= num_cu()) { p.grid *= 2; waves = GEMV_WAVES / 2; }
    if (p.nsplit > 1 && (!a.accbuf || !a.gcnt || nrows_total * (paired ? 2 : 1) > a.acc_rows || p.groups > a.acc_rows)) {
        launch_fail("GEMV split accumulators missing or too small"); return;
    }
    a.nsplit = p.nsplit; a.bps = p.bps; a.groups = p.groups;
    const int nb = p.bps < (a.cols + 31) / 32 ? p.bps : (a.cols + 31) / 32;
    const size_t lds = (size_t)NDIG * nb * sizeof(uint4) +
                       (a.pro.kind == PRO_PLAIN ? 0 : (size_t)a.pro.n * sizeof(float));
    switch (a.pro.kind * 2 + (paired ? 1 : 0)) {
    case PRO_PLAIN * 2:     launch_pro<PRO_PLAIN, false>(a, wide, p.grid, waves, lds, s); break;
    case PRO_PLAIN * 2 + 1: launch_pro<PRO_PLAIN, true>(a, wide, p.grid, waves, lds, s); break;
    case PRO_NORM * 2:      launch_pro<PRO_NORM, false>(a, wide, p.grid, waves, lds, s); break;
    case PRO_NORM * 2 + 1:  launch_pro<PRO_NORM, true>(a, wide, p.grid, waves, lds, s); break;
    case PRO_RESID * 2:     launch_pro<PRO_RESID, false>(a, wide, p.grid, waves, lds, s); break;
    default:                launch_pro<PRO_RESID, true>(a, wide, p.grid, waves, lds, s); break;
    }
}

}  // namespace kvd
