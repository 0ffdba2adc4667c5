// kvd_attn.hip -- per-head Q/K norm + RoPE + KV append, split-K GQA decode
// attention over the paged KV store, token embedding and greedy argmax.
//
// Reference semantics:
//   Q/K norm + RoPE   core/session/sp_session.c:292-294 / :405-407 with
//                     sp_rmsnorm_head + sp_rope_neox (forward_kernels.c:24-41)
//   KV append         sp_session.c:321-323 (post-norm/RoPE K, raw V at pos)
//   attention         sp_attn_head (forward_kernels.c:59-81): window start
//                     s0 = max(0, pos-win+1), score = dot*ascale, softmax, V-sum
//   embedding         sp_embed_row -> Q4B dequant (frobenius_lift.c:116-125),
//                     x sqrt(E) on Gemma (sp_session.c:392)
//
// KV page layout (one page = PAGE positions of one layer):
//   K part [NKV][PAGE][HD] then V part [NKV][PAGE][HD]; f32 in float mode,
//   int32 (ki = rne(k*2^16), vq = clamp(rne(v*2^16), +-(2^23-1))) in exact mode.
// Each kv-head's PAGE x HD slice is contiguous, so one workgroup streams it with
// fully coalesced 16 B lane loads.
//
// Split-K: workgroup (chunk c, kv-head h) covers the chunk-aligned positions of
// [s0, pos] in chunk c (chunks never straddle a page) for all G = NH/NKV q-heads
// of the group, so every K/V byte is read once per step.  The last workgroup to
// finish a kv-head merges the chunk partials (arrival counter, self-resetting).
#include "kvd_internal.h"
#include <hip/hip_ext.h>
#include "kvd_exact.h"
#include "kvd_qkprep.h"
#include "kvd_vec.h"
#include <cstdio>
#include <cstdlib>

namespace kvd {

// exact-mode RoPE tables (host-computed integer constants, see kvd_backend.hip)
// (constant memory: the CORDIC loop index is uniform, so these are scalar loads)
__constant__ int64_t g_atan_q60[64];
__constant__ int64_t g_kinv_q62;

constexpr int64_t TWO_PI_Q60 = 7244019458077122842LL;     // round(2*pi * 2^60)
constexpr int64_t HALF_PI_Q60 = 1811004864519280711LL;    // round(pi/2 * 2^60)

// atan: the 62 Q60 arctangents, staged in LDS by the caller (unrolled, the
// reads are issued ahead of the dependent steps instead of one constant-cache
// round trip per step)
__device__ void cordic_q62(int64_t th, int64_t &co, int64_t &si, const int64_t *atan) {
    int quad = 0;
    while (th >= HALF_PI_Q60 && quad < 3) { th -= HALF_PI_Q60; quad++; }
    int64_t x = g_kinv_q62, y = 0, z = th;
    // branch-free rotation direction: sm = -1 where z < 0, and (v ^ sm) - sm
    // is v or -v; the same integer steps as the two-sided update
    #pragma unroll
    for (int i = 0; i < 62; i++) {
        const int64_t xs = x >> i, ys = y >> i, sm = z >> 63;
        x -= (ys ^ sm) - sm;
        y += (xs ^ sm) - sm;
        z -= (atan[i] ^ sm) - sm;
    }
    switch (quad) {
        case 0: co = x;  si = y;  break;
        case 1: co = -y; si = x;  break;
        case 2: co = -x; si = -y; break;
        default: co = y; si = -x; break;
    }
}

// wave all-reductions (DPP, kvd_vec.h)
__device__ __forceinline__ float wsum(float v) { return wave_allsum(v); }
__device__ __forceinline__ double wsumd(double v) { return wave_allsum(v); }
__device__ __forceinline__ int64_t wsuml(int64_t v) { return wave_allsum(v); }
__device__ __forceinline__ float wmax(float v) { return wave_allmax(v); }

// K/V rows are streamed once per step: nontemporal 16-byte loads (measured
// ~15% more read bandwidth than cached loads for this streaming pattern).
template <typename T> __device__ __forceinline__ T ld_stream(const T *p) {
    typedef typename std::conditional<sizeof(T) == 16, int __attribute__((ext_vector_type(4))),
                                      int __attribute__((ext_vector_type(2)))>::type V;
    static_assert(sizeof(T) == sizeof(V), "8- or 16-byte rows");
    return __builtin_bit_cast(T, __builtin_nontemporal_load(gmem((const V *)p)));
}
__device__ __forceinline__ float *page_of(float *const *pages, int ring, int pos) {
    const int lp = pos / PAGE;
    return gmem(pages)[ring ? lp % ring : lp];
}

// Decode: the position comes from the step state.  Batched prefill: token t of
// the batch sits at pos0 + t and every per-token buffer is offset to its row.
template <bool BATCH>
__device__ __forceinline__ void tok_select(AttnArgs &a, int t, int &pos) {
    if constexpr (!BATCH) { pos = a.st->pos; return; }
    pos = a.tpos ? a.tpos[t] : a.pos0 + t;
    if (a.tpages) a.pages = gmem(a.tpages)[t];
    const size_t QD = (size_t)a.NH * a.HD, KVD = (size_t)a.NKV * a.HD;
    a.q += t * QD; a.k += t * KVD; a.v += t * KVD; a.qr += t * QD; a.ao += t * QD;
    a.part += t * (size_t)a.NH * a.max_chunks * a.HD;
    a.part_ml += t * (size_t)a.NH * a.max_chunks * 4;
    a.counter += t * a.NKV;
    a.zscratch += t * (size_t)a.NH * a.zstride;
    a.vacc += t * QD * VREP; a.vacc_s += t * a.NH * VREP;
    a.rope_cs += t * (size_t)a.rope_stride;
}

// Attention grid coordinates.  Decode: (chunk, kv head).  Token-batched
// launches put the token first, (token, chunk, kv head): the batch's tokens
// that read one chunk's K/V rows are dispatched together and share them
// through the caches, instead of each token streaming the whole span alone.
// A batched decode over sessions with a work list: (item, kv head), the item
// naming the token and chunk, so no workgroup is launched for a chunk past its
// session's position.
template <bool BATCH> __device__ __forceinline__ int grid_token(const AttnArgs &a) {
    return BATCH ? (a.work ? a.work[blockIdx.x].x : (int)blockIdx.x) : 0;
}
template <bool BATCH> __device__ __forceinline__ int grid_chunk(const AttnArgs &a) {
    return BATCH ? (a.work ? a.work[blockIdx.x].y : (int)blockIdx.y) : (int)blockIdx.x;
}
template <bool BATCH> __device__ __forceinline__ int grid_head(const AttnArgs &a) {
    return BATCH ? (a.work ? (int)blockIdx.y : (int)blockIdx.z) : (int)blockIdx.y;
}

// ------------------------------------------------------------------ qk_prep
// grid.x = NH (q heads) + NKV (k heads) + NKV (v heads), one wave each
template <bool BATCH>
__global__ __launch_bounds__(64) void k_qk_prep(AttnArgs a_in) {
    AttnArgs a = a_in;
    int pos;
    tok_select<BATCH>(a, blockIdx.y, pos);
    qk_prep_head<false>(head_prep_of(a), blockIdx.x, pos, threadIdx.x);
}

// Rotation table of the current position for both RoPE bases:
// out[t][0..half) = cos, out[t][half..HD) = sin, t = 0 global base, 1 window base.
// Float mode: freq = powf(base, -2i/d), theta = (float)p*freq, cosf/sinf
// (forward_kernels.c:31-41); exact mode: p*F_i mod 2*pi (Q60) by CORDIC, RNE.
// table t of a launch (decode: t = 0 at the step's position; batched: table t
// at tpos[t] or pos0 + t); every thread of the workgroup calls this
__device__ __forceinline__ void rope_table_body(int t_idx, const DState *st, int pos0, const int *tpos, int HD, int mode,
                                                const int64_t *fq_g, const int64_t *fq_l, float *out) {
    const int half = HD / 2, pos = st ? st->pos : (tpos ? tpos[t_idx] : pos0 + t_idx);
    out += (size_t)t_idx * 2 * HD;
    __shared__ int64_t atan_s[64];
    if (threadIdx.x < 64) atan_s[threadIdx.x] = g_atan_q60[threadIdx.x];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 2 * half; idx += blockDim.x) {
        const int t = idx / half, i = idx % half;
        float c, s;
        if (mode == FLOAT) {
            // the host-formed powf(base, -2i/d) after the HD/2 Q60 entries
            const float freq = ((const float *)((t ? fq_l : fq_g) + half))[i];
            const float theta = (float)pos * freq;
            c = cosf(theta); s = sinf(theta);
        } else {
            const i128 th = (i128)pos * (t ? fq_l : fq_g)[i];
            int64_t co, si; cordic_q62(umod128_64(th, TWO_PI_Q60), co, si, atan_s);
            c = rne_i64_scaled(co, -62); s = rne_i64_scaled(si, -62);
        }
        out[(size_t)t * HD + i] = c;
        out[(size_t)t * HD + half + i] = s;
    }
}
__global__ __launch_bounds__(256) void k_rope_table(const DState *st, int pos0, const int *tpos, int HD, int mode,
                                                     const int64_t *fq_g, const int64_t *fq_l, float *out) {
    rope_table_body((int)blockIdx.x, st, pos0, tpos, HD, mode, fq_g, fq_l, out);
}
void launch_rope_table(const DState *st, int HD, int mode, float base_g, float base_l,
                       const int64_t *fq_g, const int64_t *fq_l, float *out, hipStream_t s) {
    hipLaunchKernelGGL(k_rope_table, dim3(1), dim3(256), 0, s, st, 0, nullptr, HD, mode, fq_g, fq_l, out);
}
void launch_rope_table_batch(int pos0, int T, int HD, int mode, float base_g, float base_l,
                             const int64_t *fq_g, const int64_t *fq_l, float *out, hipStream_t s, const int *tpos) {
    hipLaunchKernelGGL(k_rope_table, dim3(T), dim3(256), 0, s, nullptr, pos0, tpos, HD, mode, fq_g, fq_l, out);
}
void launch_qk_prep(const AttnArgs &a, hipStream_t s) {
    if (a.nt) hipLaunchKernelGGL(k_qk_prep<true>, dim3(a.NH + 2 * a.NKV, a.nt), dim3(64), 0, s, a);
    else hipLaunchKernelGGL(k_qk_prep<false>, dim3(a.NH + 2 * a.NKV), dim3(64), 0, s, a);
}
void set_rope_tables(const int64_t atan_q60[64], int64_t kinv_q62) {
    hipMemcpyToSymbol(HIP_SYMBOL(g_atan_q60), atan_q60, 64 * sizeof(int64_t));
    hipMemcpyToSymbol(HIP_SYMBOL(g_kinv_q62), &kinv_q62, sizeof(int64_t));
}

// ------------------------------------------------------------------ attention
// chunk geometry for the current position: chunks are `chunk`-aligned absolute
// position ranges clipped to the attended window [s0, pos]
__device__ __forceinline__ void chunk_range(const AttnArgs &a, int pos, int c, int &cs, int &ce, int &nch) {
    const int s0 = (a.win >= 0 && pos - a.win + 1 > 0) ? pos - a.win + 1 : 0;
    const int c0 = s0 / a.chunk;
    nch = pos / a.chunk - c0 + 1;
    cs = (c0 + c) * a.chunk; ce = cs + a.chunk;
    if (cs < s0) cs = s0;
    if (ce > pos + 1) ce = pos + 1;
}

// Spinor-63 code rows (float mode with KVC_SPINOR): row p of kv-head h holds
// HD int8 codes and the chunk multipliers (kvd_spinor.h).  v' = code * mul of
// the coordinate's chunk; a lane's consecutive coordinates cross at most one
// chunk boundary (chunks hold at least 28 coordinates).
template <int EPL>
__device__ __forceinline__ const uint8_t *spn_row(const AttnArgs &a, const float *page, int h, int p, bool vpart) {
    constexpr int RB = spn_row_bytes(EPL * 64);
    return (const uint8_t *)page + ((vpart ? (size_t)a.NKV * PAGE : 0) + (size_t)h * PAGE + (p & (PAGE - 1))) * RB;
}
constexpr int MAXCH = ATTN_MAXCH;   // positions per chunk (LDS score buffer)
constexpr int MAXNCH = 4096;     // chunks per kv-head (combine weight buffer)
constexpr int UNR = 4;           // positions in flight per wave
// rows per V-row group of the exact V-sum (two groups in flight per wave;
// 12: global attention 96.3 -> 94.6 us at the Gemma-3-12B shape, 32k, against 8)
constexpr int VSUM_UV = 12;

// EPL consecutive int32 of a row for this lane (16, 8 or 4 bytes), streamed
template <int EPL> __device__ __forceinline__ void ld_lane_row(const int32_t *src, int32_t out[EPL]) {
    if constexpr (EPL == 4) {
        typedef int32_t v4 __attribute__((ext_vector_type(4)));
        const v4 t = ld_stream((const v4 *)src); out[0] = t.x; out[1] = t.y; out[2] = t.z; out[3] = t.w;
    } else if constexpr (EPL == 2) {
        typedef int32_t v2 __attribute__((ext_vector_type(2)));
        const v2 t = ld_stream((const v2 *)src); out[0] = t.x; out[1] = t.y;
    } else {
        out[0] = __builtin_nontemporal_load(gmem(src));
    }
}

// Rows j0 .. j0+R-1 of the chunk starting at cs (n rows) for the exact passes.
// Rows past the chunk are clamped to its last row, so every load is issued
// whatever n is: a load under a condition is not counted by the compiler's
// waits, and the first use of anything loaded before it would then wait for
// every row in flight (loads complete in order).  The R <= PAGE consecutive
// positions span at most two pages, looked up once per group.
template <int EPL, int R>
__device__ __forceinline__ void load_rows_c(const AttnArgs &a, int h, int cs, int n, int j0, bool vpart, int lane,
                                            int32_t out[R][EPL]) {
    static_assert(R <= PAGE, "a row group spans at most two pages");
    constexpr int HD = EPL * 64;
    const int p0 = __builtin_amdgcn_readfirstlane(cs + (j0 < n ? j0 : n - 1));
    const int p1 = __builtin_amdgcn_readfirstlane(cs + (j0 + R - 1 < n ? j0 + R - 1 : n - 1));
    // the row base is uniform (scalar), only the lane offset is per lane
    const size_t off = (vpart ? (size_t)a.NKV * PAGE * HD : 0) + (size_t)__builtin_amdgcn_readfirstlane(h) * PAGE * HD;
    const int32_t *b0 = (const int32_t *)page_of(a.pages, a.ring_pages, p0) + off;
    const int32_t *b1 = (const int32_t *)page_of(a.pages, a.ring_pages, p1) + off;
    #pragma unroll
    for (int u = 0; u < R; u++) {
        const int p = cs + (j0 + u < n ? j0 + u : n - 1);
        const int32_t *row = (p / PAGE == p0 / PAGE ? b0 : b1) + (size_t)(p & (PAGE - 1)) * HD;
        ld_lane_row<EPL>(row + lane * EPL, out[u]);
    }
}

// Row-quad layout for the score passes: a wave takes 16 consecutive positions
// at a time, lane = 4 * row + quarter; in load i a quarter reads 16 B at
// byte 64 i + 16 quarter of its row (each row's four lanes read 64
// contiguous bytes), so every lane owns HD/4 dimensions of one row and the
// dot product needs a 4-lane reduction only.  q sits in LDS and is read with
// broadcast.  The 16 rows span at most two pages, looked up once per group.
// p0: first position of the group, plast: last position the chunk holds
__device__ __forceinline__ const float *quad_page(const AttnArgs &a, int p0, int plast, int p) {
    const int pu0 = __builtin_amdgcn_readfirstlane(p0);
    const int pu1 = __builtin_amdgcn_readfirstlane(p0 + 15 < plast ? p0 + 15 : plast);
    const float *pg0 = page_of(a.pages, a.ring_pages, pu0);
    const float *pg1 = page_of(a.pages, a.ring_pages, pu1);
    return p / PAGE == pu0 / PAGE ? pg0 : pg1;
}
template <int EPL, typename T>
__device__ __forceinline__ const T *quad_row(const AttnArgs &a, int h, int p0, int plast, int p, bool vpart) {
    const float *pg = quad_page(a, p0, plast, p);
    const int HD = EPL * 64;
    return (const T *)(pg + (vpart ? (size_t)a.NKV * PAGE * HD : 0) + ((size_t)h * PAGE + (p & (PAGE - 1))) * HD);
}
// One row group of the exact score pass (LPR lanes per row, 64 / LPR rows
// from j0): row j0 + r, clamped to the chunk's last row like load_rows_c, so
// the loads are issued unconditionally.
template <int EPL, int LPR>
__device__ __forceinline__ void load_kgroup(const AttnArgs &a, int h, int cs, int n, int j0, int r, int k4,
                                            int4 kv[EPL * 16 / LPR]) {
    const int jc = j0 < n ? j0 : n - 1, j = j0 + r < n ? j0 + r : n - 1;
    const int32_t *row = quad_row<EPL, int32_t>(a, h, cs + jc, cs + n - 1, cs + j, false) + 4 * k4;
    #pragma unroll
    for (int i = 0; i < EPL * 16 / LPR; i++) kv[i] = ld_stream((const int4 *)(row + 4 * LPR * i));
}

template <int EPL, int G, bool BATCH, bool SPN>
__global__ __launch_bounds__(256) void k_attn_float(AttnArgs a_in) {
    AttnArgs a = a_in;
    int pos;
    tok_select<BATCH>(a, grid_token<BATCH>(a_in), pos);
    const int HD = EPL * 64, c = grid_chunk<BATCH>(a_in), h = grid_head<BATCH>(a_in);
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int cs, ce, nch;
    chunk_range(a, pos, c, cs, ce, nch);
    if (c >= nch) return;
    __shared__ float sc[G][MAXCH + UNR];             // 0 past the chunk (plain rows' V-sum)
    __shared__ float ored[4][G][EPL * 64];
    __shared__ float wk[MAXNCH];
    __shared__ float redf[4];
    __shared__ int is_last;
    __shared__ float4 qs[G][EPL * 16];
    for (int i = threadIdx.x; i < G * HD / 4; i += 256) {
        const int g = i / (HD / 4), d4 = i % (HD / 4);
        qs[g][d4] = *(const float4 *)(a.qr + (size_t)(h * G + g) * HD + 4 * d4);
    }
    __syncthreads();
    const int n = ce - cs;
    // scores in the row-quad layout (16 positions per wave and group)
    const int r = lane >> 2, k4 = lane & 3;
    for (int j0 = wave * 16; j0 < n; j0 += 64) {
        const int j = j0 + r;
        float acc[G];
        #pragma unroll
        for (int g = 0; g < G; g++) acc[g] = 0.0f;
        if (SPN && j < n) {
            // code rows: quarter k4 takes the 16 coordinates 64 i + 16 k4 .. + 15
            constexpr int NB = spn_blocks(HD), NM4 = (4 * NB + 15) / 16;
            const uint8_t *row = spn_row<EPL>(a, quad_page(a, cs + j0, ce - 1, cs + j), h, cs + j, false);
            uint4 cw[EPL];
            #pragma unroll
            for (int i = 0; i < EPL; i++) cw[i] = ld_stream((const uint4 *)(row + 64 * i + 16 * k4));
            float mu[4 * NM4];
            #pragma unroll
            for (int t = 0; t < NM4; t++) {
                const float4 m4 = *gmem((const float4 *)(row + HD + 16 * t));
                mu[4 * t] = m4.x; mu[4 * t + 1] = m4.y; mu[4 * t + 2] = m4.z; mu[4 * t + 3] = m4.w;
            }
            #pragma unroll
            for (int i = 0; i < EPL; i++) {
                const int d0 = 64 * i + 16 * k4, b = spn_block_of(HD, d0), bnd = spn_block_start(HD, b + 1);
                float m0 = mu[0], m1 = mu[0];
                #pragma unroll
                for (int bb = 1; bb < NB; bb++) { if (b == bb) m0 = mu[bb]; if (b + 1 == bb) m1 = mu[bb]; }
                const uint32_t cwv[4] = {cw[i].x, cw[i].y, cw[i].z, cw[i].w};
                #pragma unroll
                for (int t4 = 0; t4 < 4; t4++) {
                    float kv[4];
                    #pragma unroll
                    for (int t = 0; t < 4; t++)
                        kv[t] = (float)(int32_t)(int8_t)(cwv[t4] >> (8 * t)) * (d0 + 4 * t4 + t < bnd ? m0 : m1);
                    #pragma unroll
                    for (int g = 0; g < G; g++) {
                        const float4 q = qs[g][16 * i + 4 * k4 + t4];
                        acc[g] += q.x * kv[0] + q.y * kv[1] + q.z * kv[2] + q.w * kv[3];
                    }
                }
            }
        } else if (j < n) {
            const float *row = quad_row<EPL, float>(a, h, cs + j0, ce - 1, cs + j, false) + 4 * k4;
            float4 kv[4 * EPL];
            #pragma unroll
            for (int i = 0; i < 4 * EPL; i++) kv[i] = ld_stream((const float4 *)(row + 16 * i));
            #pragma unroll
            for (int i = 0; i < 4 * EPL; i++)
                #pragma unroll
                for (int g = 0; g < G; g++) {
                    const float4 q = qs[g][4 * i + k4];
                    acc[g] += q.x * kv[i].x + q.y * kv[i].y + q.z * kv[i].z + q.w * kv[i].w;
                }
        }
        #pragma unroll
        for (int g = 0; g < G; g++) {
            acc[g] = quad_sum(acc[g]);
        }
        if (j < n && k4 < G) {
            float d = acc[0];
            #pragma unroll
            for (int g = 1; g < G; g++) if (k4 == g) d = acc[g];
            sc[k4][j] = d * a.ascale;
        }
    }
    __syncthreads();
    float m[G], l[G];
    #pragma unroll
    for (int g = 0; g < G; g++) {
        float mv = -INFINITY;
        for (int j = lane; j < n; j += 64) mv = fmaxf(mv, sc[g][j]);
        m[g] = wmax(mv);
    }
    __syncthreads();
    // softmax numerators once per (head, position), in place
    for (int i = threadIdx.x; i < G * n; i += 256) {
        const int g = i / n, j = i % n;
        sc[g][j] = expf(sc[g][j] - m[g]);
    }
    if ((int)threadIdx.x < G * UNR) sc[threadIdx.x / UNR][n + threadIdx.x % UNR] = 0.0f;
    __syncthreads();
    #pragma unroll
    for (int g = 0; g < G; g++) {
        float lv = 0.0f;
        for (int j = lane; j < n; j += 64) lv += sc[g][j];
        l[g] = wsum(lv);
    }
    if constexpr (SPN) {
        // code rows: lane = CPR * r + col takes codes 16 col .. 16 col + 15 of
        // row r of a group of RPL rows (one 16-byte load per lane and row
        // group), two groups in flight per wave; the RPL row partials of a
        // column meet by lane exchange at the end
        constexpr int CPR = HD / 16, RPL = 64 / CPR;
        const int rr = lane / CPR, d0 = 16 * (lane % CPR);
        const int b0 = spn_block_of(HD, d0), bnd = spn_block_start(HD, b0 + 1);
        const int b1 = bnd < d0 + 16 ? b0 + 1 : b0;
        float o[G][16];
        #pragma unroll
        for (int g = 0; g < G; g++)
            #pragma unroll
            for (int t = 0; t < 16; t++) o[g][t] = 0.0f;
        for (int j0 = wave * RPL; j0 < n; j0 += 8 * RPL) {
            uint4 cw[2];
            float m0[2], m1[2];
            #pragma unroll
            for (int k = 0; k < 2; k++) {
                const int j = j0 + 4 * RPL * k + rr;
                cw[k] = make_uint4(0, 0, 0, 0); m0[k] = m1[k] = 0.0f;
                if (j < n) {
                    const uint8_t *row = spn_row<EPL>(a, quad_page(a, cs + j0 + 4 * RPL * k, ce - 1, cs + j), h, cs + j, true);
                    cw[k] = ld_stream((const uint4 *)(row + d0));
                    m0[k] = gmem((const float *)(row + HD))[b0];
                    m1[k] = gmem((const float *)(row + HD))[b1];
                }
            }
            #pragma unroll
            for (int k = 0; k < 2; k++) {
                const int j = j0 + 4 * RPL * k + rr;
                if (j >= n) continue;
                float p[G];
                #pragma unroll
                for (int g = 0; g < G; g++) p[g] = sc[g][j];
                const uint32_t w[4] = {cw[k].x, cw[k].y, cw[k].z, cw[k].w};
                #pragma unroll
                for (int t = 0; t < 16; t++) {
                    const float x = (float)(int32_t)(int8_t)(w[t >> 2] >> (8 * (t & 3))) * (d0 + t < bnd ? m0[k] : m1[k]);
                    #pragma unroll
                    for (int g = 0; g < G; g++) o[g][t] += p[g] * x;
                }
            }
        }
        #pragma unroll
        for (int s = CPR; s < 64; s <<= 1)
            #pragma unroll
            for (int g = 0; g < G; g++)
                #pragma unroll
                for (int t = 0; t < 16; t++) o[g][t] += __shfl_xor(o[g][t], s, 64);
        if (rr == 0)
            #pragma unroll
            for (int g = 0; g < G; g++)
                #pragma unroll
                for (int t = 0; t < 16; t++) ored[wave][g][d0 + t] = o[g][t];
    } else {
        float o[G][EPL];
        #pragma unroll
        for (int g = 0; g < G; g++)
            #pragma unroll
            for (int e = 0; e < EPL; e++) o[g][e] = 0.0f;
        // rows as in the exact V-sum: every load issued (rows past the chunk
        // clamped, meeting the zero numerators after it), the next group in
        // the other buffer; rows are added in the same order as before
        int32_t va[UNR][EPL], vb[UNR][EPL];
        auto vsum = [&](const int32_t (&v)[UNR][EPL], int j0) {
            #pragma unroll
            for (int u = 0; u < UNR; u++) {
                #pragma unroll
                for (int g = 0; g < G; g++) {
                    const float p = sc[g][j0 + u];
                    #pragma unroll
                    for (int e = 0; e < EPL; e++) o[g][e] += p * __int_as_float(v[u][e]);
                }
            }
        };
        load_rows_c<EPL, UNR>(a, h, cs, n, wave * UNR, true, lane, va);
        __builtin_amdgcn_sched_barrier(0);
        for (int j0 = wave * UNR; j0 < n; j0 += 8 * UNR) {
            load_rows_c<EPL, UNR>(a, h, cs, n, j0 + 4 * UNR, true, lane, vb);
            __builtin_amdgcn_sched_barrier(0);
            vsum(va, j0);
            if (j0 + 4 * UNR >= n) break;
            load_rows_c<EPL, UNR>(a, h, cs, n, j0 + 8 * UNR, true, lane, va);
            __builtin_amdgcn_sched_barrier(0);
            vsum(vb, j0 + 4 * UNR);
        }
        #pragma unroll
        for (int g = 0; g < G; g++)
            #pragma unroll
            for (int e = 0; e < EPL; e++) ored[wave][g][lane * EPL + e] = o[g][e];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        st_agent(&a.part[((size_t)(h * G + g) * a.max_chunks + c) * HD + d], ored[0][g][d] + ored[1][g][d] + ored[2][g][d] + ored[3][g][d]);
    }
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        st_agent(&a.part_ml[((size_t)(h * G + g) * a.max_chunks + c) * 2 + 0], m[g]);
        st_agent(&a.part_ml[((size_t)(h * G + g) * a.max_chunks + c) * 2 + 1], l[g]);
    }
    // ---- the last workgroup of this kv-head merges the chunks ----
    mem_complete();
    __syncthreads();
    if (threadIdx.x == 0) is_last = (arrive(&a.counter[h]) == nch - 1);
    __syncthreads();
    if (!is_last) return;
    StatAcc sacc;
    for (int g = 0; g < G; g++) {
        const size_t base = (size_t)(h * G + g) * a.max_chunks;
        const float *pml = a.part_ml + base * 2;
        float mv = -INFINITY;
        for (int k = threadIdx.x; k < nch; k += 256) mv = fmaxf(mv, ld_agent(&pml[k * 2]));
        mv = wmax(mv);
        if (lane == 0) redf[wave] = mv;
        __syncthreads();
        const float M = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
        __syncthreads();
        float lv = 0.0f;
        for (int k = threadIdx.x; k < nch; k += 256) { const float w = expf(ld_agent(&pml[k * 2]) - M); wk[k] = w; lv += ld_agent(&pml[k * 2 + 1]) * w; }
        lv = wsum(lv);
        if (lane == 0) redf[wave] = lv;
        __syncthreads();
        const float L = redf[0] + redf[1] + redf[2] + redf[3];
        const float *po = a.part + base * HD;
        for (int d = threadIdx.x; d < HD; d += 256) {
            float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
            int k = 0;
            for (; k + 4 <= nch; k += 4) {
                acc0 += ld_agent(&po[(size_t)k * HD + d]) * wk[k];
                acc1 += ld_agent(&po[(size_t)(k + 1) * HD + d]) * wk[k + 1];
                acc2 += ld_agent(&po[(size_t)(k + 2) * HD + d]) * wk[k + 2];
                acc3 += ld_agent(&po[(size_t)(k + 3) * HD + d]) * wk[k + 3];
            }
            for (; k < nch; k++) acc0 += ld_agent(&po[(size_t)k * HD + d]) * wk[k];
            const float o = ((acc0 + acc1) + (acc2 + acc3)) / L;
            a.ao[(size_t)(h * G + g) * HD + d] = o;
            sacc.add(o);
        }
        __syncthreads();
    }
    if (a.stat_out) stat_flush_block(a.stat_out, sacc);       // max |ao| for the O GEMV
    if (threadIdx.x == 0) reset_counter(&a.counter[h]);
}

// The step's head preparation inside the exact score pass (decode): wave g < G
// normalizes and rotates q head h*G + g into qs; in the workgroup holding pos,
// wave G % 4 prepares the new K row (paged store + kn) and wave (G + 1) % 4
// appends the new V row (and keeps a copy in vn when given).  prep_load
// requests the inputs, prep_finish computes and stores.
template <int EPL> struct PrepIn { HeadIn q, k; float v[EPL]; };
template <int EPL, int G>
__device__ __forceinline__ void prep_load(const AttnArgs &a, int h, int pos, int wave, int lane, bool holds_pos, PrepIn<EPL> &in) {
    static_assert(G <= 4, "one wave per q head of the group");
    constexpr int HD = EPL * 64;
    const HeadPrep hp = head_prep_of(a);
    if (wave < G) head_load<false, EPL>(hp, a.q + (size_t)(h * G + wave) * HD, a.q_norm, lane, in.q);
    if (holds_pos && wave == G % 4) head_load<false, EPL>(hp, a.k + (size_t)h * HD, a.k_norm, lane, in.k);
    if (holds_pos && wave == (G + 1) % 4) {
        #pragma unroll
        for (int j = 0; j < EPL; j++) in.v[j] = a.v[(size_t)h * HD + lane + 64 * j];
    }
}
template <int EPL, int G>
__device__ __forceinline__ void prep_finish(const AttnArgs &a, int h, int pos, int wave, int lane, bool holds_pos,
                                            const PrepIn<EPL> &in, int4 (*qs)[EPL * 16], int4 *kn, int32_t *vn = nullptr) {
    constexpr int HD = EPL * 64;
    const HeadPrep hp = head_prep_of(a);
    float out[8];
    if (wave < G) {
        head_norm_rope_in<EPL>(hp, in.q, lane, out);
        #pragma unroll
        for (int j = 0; j < EPL; j++) ((int *)qs[wave])[lane + 64 * j] = (int)rintf(out[j] * 65536.0f);
    }
    if (holds_pos) {
        float *page = qk_page_of(a.pages, a.ring_pages, pos);
        const size_t rowoff = ((size_t)h * PAGE + pos % PAGE) * HD;
        if (wave == G % 4) {
            head_norm_rope_in<EPL>(hp, in.k, lane, out);
            if (a.kvc == KVC_SPINOR) spinor_head<EPL>(out, lane, false, nullptr);   // the codec's decoded values
            #pragma unroll
            for (int j = 0; j < EPL; j++) {
                const int32_t ki = kv_code_k(out[j]);
                gmem((int32_t *)(page + rowoff))[lane + 64 * j] = ki;
                ((int *)kn)[lane + 64 * j] = ki;
            }
        }
        if (wave == (G + 1) % 4) {
            int32_t *dst = (int32_t *)(page + (size_t)a.NKV * PAGE * HD + rowoff);
            float x[8];
            #pragma unroll
            for (int j = 0; j < EPL; j++) x[j] = in.v[j];
            if (a.kvc == KVC_SPINOR) spinor_head<EPL>(x, lane, false, nullptr);
            bool cl = false;
            #pragma unroll
            for (int j = 0; j < EPL; j++) {
                const int32_t vi = kv_code_v(x[j], cl);
                gmem(dst)[lane + 64 * j] = vi;
                if (vn) vn[lane + 64 * j] = vi;
            }
            count_v_clamp(a.vclamp, cl);
        }
    }
}

// ---- exact mode: pass 1, integer scores on the softmax grid + chunk max ----
// PREP (decode): the kernel also does the step's head preparation -- every
// workgroup normalizes and rotates its G q heads itself (wave g, head h*G+g)
// straight into LDS, and the workgroup of the last chunk, which holds pos,
// appends the new K (after norm and RoPE) and V rows to the paged store and
// scores position pos from the new K row it keeps in LDS (its own loads of
// that row may predate the append).  Same arithmetic as k_qk_prep.
// LPR lanes per row, 16 bytes each per load: a load instruction takes LPR * 16
// contiguous bytes of each of the wave's RPW = 64 / LPR rows.  8 lanes read
// a whole 128-byte line of a row per load (long chunks: half the line requests
// of 4 lanes); 4 lanes let the four waves cover a 64-position chunk in one pass.
template <int EPL, int G, bool BATCH, bool PREP, int LPR>
__global__ __launch_bounds__(256) void k_attn_exact_scores(AttnArgs a_in) {
    static_assert(!(BATCH && PREP), "head preparation is fused for decode only");
    AttnArgs a = a_in;
    int pos;
    tok_select<BATCH>(a, grid_token<BATCH>(a_in), pos);
    const int HD = EPL * 64, c = grid_chunk<BATCH>(a_in), h = grid_head<BATCH>(a_in);
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int cs, ce, nch;
    chunk_range(a, pos, c, cs, ce, nch);
    if (c >= nch) return;
    __shared__ int zmax[4][G];
    __shared__ int4 qs[G][EPL * 16];                 // qi = rne(q * 2^16), 4 dims per entry
    __shared__ int4 kn[PREP ? EPL * 16 : 1];         // PREP, last chunk: the new K row (ki)
    static_assert(LPR == 4 || LPR == 8, "4 or 8 lanes per row");
    constexpr int RPW = 64 / LPR, NLD = EPL * 16 / LPR;
    const int r = lane / LPR, k4 = lane % LPR;
    const int n = ce - cs;
    const bool holds_pos = PREP && c == nch - 1;     // chunk ranges end at pos
    // The head preparation's inputs are requested first, then the wave's first
    // row group: the preparation then runs while the rows stream in.
    PrepIn<EPL> pin;
    if constexpr (PREP) prep_load<EPL, G>(a, h, pos, wave, lane, holds_pos, pin);
    __builtin_amdgcn_sched_barrier(0);
    int4 kv[NLD];
    load_kgroup<EPL, LPR>(a, h, cs, n, wave * RPW, r, k4, kv);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PREP) {
        prep_finish<EPL, G>(a, h, pos, wave, lane, holds_pos, pin, qs, kn);
    } else {
        for (int i = threadIdx.x; i < G * HD / 4; i += 256) {
            const int g = i / (HD / 4), d4 = i % (HD / 4);
            const float *qp = a.qr + (size_t)(h * G + g) * HD + 4 * d4;
            qs[g][d4] = make_int4((int)rintf(qp[0] * 65536.0f), (int)rintf(qp[1] * 65536.0f),
                                  (int)rintf(qp[2] * 65536.0f), (int)rintf(qp[3] * 65536.0f));
        }
    }
    __syncthreads();
    int mx = INT32_MIN;                              // lane with k4 == g tracks head g
    // one row group's scores (rows j0 + r): the new K row of pos from LDS in
    // the workgroup that holds it
    auto score = [&](int4 (&kr)[NLD], int j0) {
        const int j = j0 + r;
        int64_t acc[G];
        #pragma unroll
        for (int g = 0; g < G; g++) acc[g] = 0;
        if (j < n) {
            if (holds_pos && cs + j == pos) {
                #pragma unroll
                for (int i = 0; i < NLD; i++) kr[i] = kn[LPR * i + k4];
            }
            #pragma unroll
            for (int i = 0; i < NLD; i++)
                #pragma unroll
                for (int g = 0; g < G; g++) {
                    const int4 q = qs[g][LPR * i + k4];
                    acc[g] += (int64_t)q.x * kr[i].x + (int64_t)q.y * kr[i].y + (int64_t)q.z * kr[i].z + (int64_t)q.w * kr[i].w;
                }
        }
        #pragma unroll
        for (int g = 0; g < G; g++) {
            acc[g] = group_sum<LPR>(acc[g]);
        }
        if (j < n && k4 < G) {
            int64_t tot = acc[0];
            #pragma unroll
            for (int g = 1; g < G; g++) if (k4 == g) tot = acc[g];
            const float scv = (float)((double)tot / 4294967296.0) * a.ascale;
            const int32_t z = (int32_t)llround_pow2<14>(scv);
            a.zscratch[(size_t)(h * G + k4) * a.zstride + (size_t)(cs + j)] = z;
            mx = z > mx ? z : mx;
        }
    };
    // the next row group is requested before the current one is scored, into
    // the other buffer (every load issued, clamped past the chunk)
    int4 kw[NLD];
    for (int j0 = wave * RPW; j0 < n; j0 += 8 * RPW) {
        load_kgroup<EPL, LPR>(a, h, cs, n, j0 + 4 * RPW, r, k4, kw);
        __builtin_amdgcn_sched_barrier(0);
        score(kv, j0);
        if (j0 + 4 * RPW >= n) break;
        load_kgroup<EPL, LPR>(a, h, cs, n, j0 + 8 * RPW, r, k4, kv);
        __builtin_amdgcn_sched_barrier(0);
        score(kw, j0 + 4 * RPW);
    }
    // per-head maximum over this wave
    int mxg[G];
    #pragma unroll
    for (int g = 0; g < G; g++) {
        int t = k4 == g ? mx : INT32_MIN;
        t = wave_allmax_i(t);
        mxg[g] = t;
    }
    if (lane == 0) for (int g = 0; g < G; g++) zmax[wave][g] = mxg[g];
    __syncthreads();
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        int t = zmax[0][g];
        for (int w = 1; w < 4; w++) t = zmax[w][g] > t ? zmax[w][g] : t;
        ((int32_t *)a.part_ml)[((size_t)(h * G + g) * a.max_chunks + c) * 4] = t;
    }
}

// ---- exact mode: the join of a kv head's chunks ----
// The chunk's V-sums (ored: one row per wave, summed here) join the kv head's
// totals, exactly and in any order, in VREP replicas (chunk c adds into
// replica c % VREP, where its softmax denominators were added too); the last
// of the head's nch workgroups to arrive reads and clears the totals, divides
// and writes ao, and resets the head's counter.  Every thread of the
// workgroup calls this, last.
template <int EPL, int G>
__device__ __forceinline__ void exact_join(const AttnArgs &a, int h, int c, int nch, int64_t (*ored)[G][EPL * 64]) {
    constexpr int HD = EPL * 64;
    const size_t QDh = (size_t)a.NH * HD;
    int64_t *vrep = a.vacc + (size_t)(c % VREP) * QDh;
    for (int i = threadIdx.x; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        const int64_t t = ored[0][g][d] + ored[1][g][d] + ored[2][g][d] + ored[3][g][d];
        atomicAdd((unsigned long long *)&vrep[(size_t)(h * G + g) * HD + d], (unsigned long long)t);
    }
    mem_complete();
    __syncthreads();
    __shared__ int is_last;
    if (threadIdx.x == 0) is_last = (arrive(&a.counter[h]) == nch - 1);
    __syncthreads();
    if (!is_last) return;
    // the totals are read and cleared for the next launch in one atomic step;
    // every exchange (denominators and V-sums) is issued before any total is
    // used: one round trip
    __shared__ int64_t Sg[G];
    int64_t S = 0;
    if (threadIdx.x < G)
        #pragma unroll
        for (int r = 0; r < VREP; r++)
            S += (int64_t)__hip_atomic_exchange((unsigned long long *)&a.vacc_s[(size_t)r * a.NH + h * G + threadIdx.x], 0ull,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    constexpr int PT = (G * EPL * 64 + 255) / 256;   // elements per thread
    int64_t tot[PT];
    #pragma unroll
    for (int k = 0; k < PT; k++) {
        const int i = threadIdx.x + 256 * k;
        tot[k] = 0;
        if (i < G * HD)
            #pragma unroll
            for (int r = 0; r < VREP; r++)
                tot[k] += (int64_t)__hip_atomic_exchange((unsigned long long *)&a.vacc[(size_t)r * QDh + (size_t)h * G * HD + i], 0ull,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x < G) Sg[threadIdx.x] = S;
    __syncthreads();
    StatAcc sacc;
    #pragma unroll
    for (int k = 0; k < PT; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i >= G * HD) break;
        const float o = rne_div_to_float((i128)tot[k], Sg[i / HD], 16);
        a.ao[(size_t)h * G * HD + i] = o;
        sacc.add(o);
    }
    if (a.stat_out) stat_flush_block(a.stat_out, sacc);      // max |ao| for the O GEMV
    if (threadIdx.x == 0) reset_counter(&a.counter[h]);
}

// ---- exact mode: pass 2, exp weights on the island grid, exact V-sum ----
template <int EPL, int G, bool BATCH, int UV>
__global__ __launch_bounds__(256) void k_attn_exact_vsum(AttnArgs a_in) {
    AttnArgs a = a_in;
    int pos;
    tok_select<BATCH>(a, grid_token<BATCH>(a_in), pos);
    const int HD = EPL * 64, c = grid_chunk<BATCH>(a_in), h = grid_head<BATCH>(a_in);
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // decode may sum V over longer chunks than the score pass's (vchunk, a
    // multiple of chunk): fewer workgroups arrive on each kv head's counter.
    // The maxima stay per score chunk (nsc of them).
    int cs, ce, nch, nsc;
    chunk_range(a, pos, 0, cs, ce, nsc);
    if (!BATCH && a.vchunk > a.chunk) a.chunk = a.vchunk;
    chunk_range(a, pos, c, cs, ce, nch);
    if (c >= nch) return;
    __shared__ int32_t ew[G][MAXCH + UV];           // island weights in Q22 (<= 2^22), 0 past the chunk
    __shared__ int64_t ored[4][G][EPL * 64];
    __shared__ int redi[4][G];
    __shared__ int64_t redl[4][G];
    const int n = ce - cs;
    // This chunk's scores and the chunk maxima are requested first, then the
    // first UV V rows of each wave: the global-max reduction and the weights
    // then overlap the rows' latency.  Every one of these loads is issued
    // (indices past the end clamped, the values unused), so that the waits
    // for the scores leave the rows in flight.
    constexpr int ZPT = G * MAXCH / 256;              // score slots per thread
    int32_t zr[ZPT];                                  // slot j >= n: unused
    #pragma unroll
    for (int k = 0; k < ZPT; k++) {
        const int i = threadIdx.x + 256 * k;
        const int g = i / MAXCH, j = i % MAXCH;
        zr[k] = a.zscratch[(size_t)(h * G + g) * a.zstride + (size_t)(cs + (j < n ? j : n - 1))];
    }
    const int32_t *pml = (const int32_t *)a.part_ml;
    int pm0[G];
    #pragma unroll
    for (int g = 0; g < G; g++) {
        const int v = pml[((size_t)(h * G + g) * a.max_chunks + ((int)threadIdx.x < nsc ? threadIdx.x : 0)) * 4];
        pm0[g] = (int)threadIdx.x < nsc ? v : INT32_MIN;
    }
    __builtin_amdgcn_sched_barrier(0);
    int32_t va[UV][EPL], vb[UV][EPL];                 // row groups in flight, alternating
    load_rows_c<EPL, UV>(a, h, cs, n, wave * UV, true, lane, va);
    __builtin_amdgcn_sched_barrier(0);
    // global max of the attended window over every chunk's maximum
    int M[G];
    #pragma unroll
    for (int g = 0; g < G; g++) {
        int t = pm0[g];
        for (int k = threadIdx.x + 256; k < nsc; k += 256) {
            const int v = pml[((size_t)(h * G + g) * a.max_chunks + k) * 4];
            t = v > t ? v : t;
        }
        t = wave_allmax_i(t);
        if (lane == 0) redi[wave][g] = t;
    }
    __syncthreads();
    #pragma unroll
    for (int g = 0; g < G; g++) {
        int t = redi[0][g];
        for (int w = 1; w < 4; w++) t = redi[w][g] > t ? redi[w][g] : t;
        M[g] = t;
    }
    #pragma unroll
    for (int k = 0; k < ZPT; k++) {
        const int i = threadIdx.x + 256 * k;
        const int g = i / MAXCH, j = i % MAXCH;
        if (j < n) ew[g][j] = (int32_t)(exp_fixed((((int64_t)zr[k] - (int64_t)M[g]) * ONE) >> 14) >> 8);
    }
    if ((int)threadIdx.x < G * UV) ew[threadIdx.x / UV][n + threadIdx.x % UV] = 0;
    __syncthreads();
    // The V-sum of this wave's rows in FP64, exactly: weights are Q22 (<= 2^22)
    // and |vq| < 2^23, so every product is below 2^45 and every partial sum of
    // a wave's rows (ceil(MAXCH / (4 UV)) groups of UV, fewer than 2^8 rows) is
    // an integer below 2^53 -- one exact FMA per term instead of an emulated
    // 64-bit multiply-add.
    static_assert((MAXCH + 4 * UV - 1) / (4 * UV) * UV < 256, "a wave's exact FP64 V-sum covers under 2^8 rows");
    double o[G][EPL];
    #pragma unroll
    for (int g = 0; g < G; g++)
        #pragma unroll
        for (int e = 0; e < EPL; e++) o[g][e] = 0.0;
    // every row of the group is read, without conditions (rows past the end
    // meet the zero weights after the chunk's, which add exactly nothing): a
    // row left unread on some path would count as still in flight, and
    // reusing its registers would wait for every load
    auto vsum = [&](const int32_t (&v)[UV][EPL], int j0) {
        #pragma unroll
        for (int u = 0; u < UV; u++) {
            #pragma unroll
            for (int g = 0; g < G; g++) {
                const double w = (double)ew[g][j0 + u];
                #pragma unroll
                for (int e = 0; e < EPL; e++) o[g][e] = fma(w, (double)v[u][e], o[g][e]);
            }
        }
    };
    // the next row group is requested before the current one is summed, into
    // the other buffer (no register copies, whose waits would be total)
    for (int j0 = wave * UV; j0 < n; j0 += 8 * UV) {
        load_rows_c<EPL, UV>(a, h, cs, n, j0 + 4 * UV, true, lane, vb);
        __builtin_amdgcn_sched_barrier(0);
        vsum(va, j0);
        if (j0 + 4 * UV >= n) break;
        load_rows_c<EPL, UV>(a, h, cs, n, j0 + 8 * UV, true, lane, va);
        __builtin_amdgcn_sched_barrier(0);
        vsum(vb, j0 + 4 * UV);
    }
    #pragma unroll
    for (int g = 0; g < G; g++)
        #pragma unroll
        for (int e = 0; e < EPL; e++) ored[wave][g][lane * EPL + e] = (int64_t)o[g][e];
    // the chunk's softmax denominators, all heads of the group in one round
    #pragma unroll
    for (int g = 0; g < G; g++) {
        int64_t S = 0;
        for (int j = threadIdx.x; j < n; j += 256) S += ew[g][j];
        S = wsuml(S);
        if (lane == 0) redl[wave][g] = S;
    }
    __syncthreads();
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        atomicAdd((unsigned long long *)&a.vacc_s[(size_t)(c % VREP) * a.NH + h * G + g],
                  (unsigned long long)(redl[0][g] + redl[1][g] + redl[2][g] + redl[3][g]));
    }
    exact_join<EPL, G>(a, h, c, nch, ored);
}

// ---- exact mode, window layers (decode): both passes in one launch ----
// A window layer attends over at most (W-1)/64 + 2 64-position chunks per kv
// head (at most WIN_MAXCH here), and the host launches this kernel only when
// its whole grid fits the device at once, four times over (one launch per
// hardware queue).  Workgroup (c, h) scores chunk c of kv head h into LDS and
// hands data to the head's other workgroups through tagged slots in a.wslot:
// each value is stored with a non-zero tag (WTAG added: the values are far
// below 2^52), its single reader polls until every value it needs is
// non-zero, then clears them.  Every slot is zero when a launch starts (zeroed
// with the buffer, cleared by its reader in every launch), so there are no
// counters, fences or resets: one store and one poll per hand-off.
//   1. chunk maxima: workgroup c stores its G maxima into every reader's row
//      (mx[h][r][g][c], r < nch); wave g of workgroup r polls mx[h][r][g][*]
//      for the window maximum of head g;
//   2. V partials: workgroup c stores its G*HD exact V-sums and its G softmax
//      denominators (one copy per reader) into pv[h][c][*]; workgroup s
//      finishes slice s of the head's G*HD outputs (ceil(G*HD / nch) each):
//      sums the slice over the chunks, divides by the summed denominators
//      (RNE) and writes ao.
// The arithmetic is that of k_attn_exact_scores (PREP, 4 lanes per row)
// followed by k_attn_exact_vsum, bit for bit: the sums are exact integers.
// The polls are bounded (2^20 rounds), so every wave exits whatever happens;
// with the grid resident the bound is never reached.
constexpr int WIN_MAXCH = WIN_MAXCH_HOST;
constexpr int64_t WTAG = (int64_t)1 << 62;
template <int EPL, int G> constexpr size_t win_slots_per_head() {
    return (size_t)WIN_MAXCH * G * WIN_MAXCH + (size_t)WIN_MAXCH * (G * EPL * 64 + WIN_MAXCH * G);
}
size_t window_slot_bytes(int NKV, int HD, int G) {
    return (size_t)NKV * WIN_MAXCH * G * (2 * WIN_MAXCH + HD) * sizeof(int64_t);
}

template <int EPL, int G>
__global__ __launch_bounds__(256) void k_attn_exact_window(AttnArgs a_in) {
    constexpr int HD = EPL * 64, LPR = 4, RPW = 64 / LPR, NLD = EPL * 16 / LPR, UV = 2 * UNR;
    constexpr int PVROW = G * HD + WIN_MAXCH * G;    // partial row: G*HD V-sums, then G denominators per reader
    constexpr int PPT = (G * HD + WIN_MAXCH * (1 + G) + 255) / 256;   // polled values per thread (finisher)
    static_assert(8 * UV == 64, "two V row groups per wave cover a 64-position chunk");
    static_assert(G * HD + WIN_MAXCH * (1 + G) <= 4 * G * HD, "the finisher's values fit the V-sum LDS");
    static_assert(win_slots_per_head<EPL, G>() == (size_t)WIN_MAXCH * G * (2 * WIN_MAXCH + HD), "slot layout");
    AttnArgs a = a_in;
    const int pos = a.st->pos, c = blockIdx.x, h = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int cs, ce, nch;
    chunk_range(a, pos, c, cs, ce, nch);
    if (c >= nch) return;
    __shared__ int4 qs[G][EPL * 16];
    __shared__ int4 kn[EPL * 16];
    __shared__ int32_t vn[HD];
    __shared__ int32_t zs[G][64];
    __shared__ int32_t ew[G][64];
    __shared__ int zmax[4][G];
    __shared__ int64_t Sl[G];
    __shared__ int64_t ored[4][G][EPL * 64];
    const int r = lane / LPR, k4 = lane % LPR, n = ce - cs;
    const bool holds_pos = c == nch - 1;             // chunk ranges end at pos
    int64_t *mxh = a.wslot + (size_t)h * win_slots_per_head<EPL, G>();      // [reader][g][chunk]
    int64_t *pvh = mxh + (size_t)WIN_MAXCH * G * WIN_MAXCH;                 // [chunk][PVROW]
    // requests: the preparation's inputs, the wave's K rows, then its first V
    // row group (rows wave*UV.., clamped like every load); the second group
    // ((wave+4)*UV..) follows the scores, in the K rows' registers
    PrepIn<EPL> pin;
    prep_load<EPL, G>(a, h, pos, wave, lane, holds_pos, pin);
    __builtin_amdgcn_sched_barrier(0);
    int4 kv[NLD];
    load_kgroup<EPL, LPR>(a, h, cs, n, wave * RPW, r, k4, kv);
    int32_t va[UV][EPL], vb[UV][EPL];
    load_rows_c<EPL, UV>(a, h, cs, n, wave * UV, true, lane, va);
    __builtin_amdgcn_sched_barrier(0);
    prep_finish<EPL, G>(a, h, pos, wave, lane, holds_pos, pin, qs, kn, vn);
    __syncthreads();
    // scores on the softmax grid: row wave*RPW + r, one pass covers the chunk
    int mx = INT32_MIN;                              // lane with k4 == g tracks head g
    {
        const int j = wave * RPW + r;
        int64_t acc[G];
        #pragma unroll
        for (int g = 0; g < G; g++) acc[g] = 0;
        if (j < n) {
            if (holds_pos && cs + j == pos) {
                #pragma unroll
                for (int i = 0; i < NLD; i++) kv[i] = kn[LPR * i + k4];
            }
            #pragma unroll
            for (int i = 0; i < NLD; i++)
                #pragma unroll
                for (int g = 0; g < G; g++) {
                    const int4 q = qs[g][LPR * i + k4];
                    acc[g] += (int64_t)q.x * kv[i].x + (int64_t)q.y * kv[i].y + (int64_t)q.z * kv[i].z + (int64_t)q.w * kv[i].w;
                }
        }
        #pragma unroll
        for (int g = 0; g < G; g++) acc[g] = group_sum<LPR>(acc[g]);
        if (j < n && k4 < G) {
            int64_t tot = acc[0];
            #pragma unroll
            for (int g = 1; g < G; g++) if (k4 == g) tot = acc[g];
            const float scv = (float)((double)tot / 4294967296.0) * a.ascale;
            const int32_t z = (int32_t)llround_pow2<14>(scv);
            zs[k4][j] = z;
            mx = z;
        }
    }
    #pragma unroll
    for (int g = 0; g < G; g++) {
        const int t = wave_allmax_i(k4 == g ? mx : INT32_MIN);
        if (lane == 0) zmax[wave][g] = t;
    }
    __syncthreads();
    // 1. this chunk's maxima into every reader's row, then the second V group
    if ((int)threadIdx.x < nch * G) {
        const int rd = threadIdx.x / G, g = threadIdx.x % G;
        int t = zmax[0][g];
        for (int w = 1; w < 4; w++) t = zmax[w][g] > t ? zmax[w][g] : t;
        st_agent(&mxh[((size_t)rd * G + g) * WIN_MAXCH + c], WTAG | (int64_t)(uint32_t)t);
    }
    load_rows_c<EPL, UV>(a, h, cs, n, (wave + 4) * UV, true, lane, vb);
    // wave g < G: the window maximum of head g from this reader's row (lane k:
    // chunk k, nch <= WIN_MAXCH <= 64), the row cleared; the island weights
    // (0 past the chunk) and the chunk's softmax denominator
    if (wave < G) {
        const int g = wave;
        int64_t *row = mxh + ((size_t)c * G + g) * WIN_MAXCH;
        const bool mine = lane < nch;
        int64_t v = WTAG;
        for (int spins = 0; spins < (1 << 20); spins++) {
            if (mine) v = ld_agent(&row[lane]);
            if (__ballot(v == 0) == 0) break;
            __builtin_amdgcn_s_sleep(1);
        }
        if (mine) st_agent(&row[lane], (int64_t)0);
        const int M = wave_allmax_i(mine ? (int)(uint32_t)v : INT32_MIN);
        const int32_t w = lane < n ? (int32_t)(exp_fixed((((int64_t)zs[g][lane] - (int64_t)M) * ONE) >> 14) >> 8) : 0;
        ew[g][lane] = w;
        const int64_t S = wsuml((int64_t)w);
        if (lane == 0) Sl[g] = S;
    }
    // the workgroup holding pos sums the new V row from LDS (its own loads of
    // that row predate the append)
    if (holds_pos) {
        const int jp = pos - cs, u0 = jp % UV;
        #pragma unroll
        for (int u = 0; u < UV; u++)
            if (u == u0) {
                #pragma unroll
                for (int e = 0; e < EPL; e++) {
                    if (jp / UV == wave) va[u][e] = vn[lane * EPL + e];
                    if (jp / UV == wave + 4) vb[u][e] = vn[lane * EPL + e];
                }
            }
    }
    __syncthreads();
    // the exact FP64 V-sum of k_attn_exact_vsum over the wave's 2 * UV rows
    double o[G][EPL];
    #pragma unroll
    for (int g = 0; g < G; g++)
        #pragma unroll
        for (int e = 0; e < EPL; e++) o[g][e] = 0.0;
    auto vsum = [&](const int32_t (&v)[UV][EPL], int j0) {
        #pragma unroll
        for (int u = 0; u < UV; u++) {
            #pragma unroll
            for (int g = 0; g < G; g++) {
                const double w = (double)ew[g][j0 + u];
                #pragma unroll
                for (int e = 0; e < EPL; e++) o[g][e] = fma(w, (double)v[u][e], o[g][e]);
            }
        }
    };
    vsum(va, wave * UV);
    vsum(vb, (wave + 4) * UV);
    #pragma unroll
    for (int g = 0; g < G; g++)
        #pragma unroll
        for (int e = 0; e < EPL; e++) ored[wave][g][lane * EPL + e] = (int64_t)o[g][e];
    __syncthreads();
    // 2. this chunk's V-sums and (one copy per reader) denominators
    int64_t *prow = pvh + (size_t)c * PVROW;
    for (int i = threadIdx.x; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        st_agent(&prow[i], ored[0][g][d] + ored[1][g][d] + ored[2][g][d] + ored[3][g][d] + WTAG);
    }
    if ((int)threadIdx.x < nch * G) st_agent(&prow[G * HD + threadIdx.x], Sl[threadIdx.x % G] + WTAG);
    // this workgroup's slice [e0, e0 + nl) of the head's G*HD outputs: value p
    // of the nch x (nl + G) it needs is element e0 + j (j < nl) or
    // denominator j - nl of chunk p / (nl + G)
    const int L = (G * HD + nch - 1) / nch, e0 = c * L;
    const int nl = e0 >= G * HD ? 0 : (G * HD - e0 < L ? G * HD - e0 : L), pw = nl + G, P = nch * pw;
    int64_t pv[PPT];
    int64_t *addr[PPT];
    #pragma unroll
    for (int k = 0; k < PPT; k++) {
        const int p = threadIdx.x + 256 * k, ck = p / pw, j = p % pw;
        addr[k] = pvh + (size_t)ck * PVROW + (j < nl ? e0 + j : G * HD + c * G + (j - nl));
        pv[k] = p < P ? 0 : WTAG;
    }
    for (int spins = 0; spins < (1 << 20); spins++) {
        bool ok = true;
        #pragma unroll
        for (int k = 0; k < PPT; k++)
            if (pv[k] == 0) pv[k] = ld_agent(addr[k]);
        #pragma unroll
        for (int k = 0; k < PPT; k++) ok &= pv[k] != 0;
        if (__syncthreads_and(ok)) break;
        __builtin_amdgcn_s_sleep(1);
    }
    int64_t *vals = &ored[0][0][0];                  // [nch][pw], untagged
    #pragma unroll
    for (int k = 0; k < PPT; k++) {
        const int p = threadIdx.x + 256 * k;
        if (p < P) { vals[p] = pv[k] - WTAG; st_agent(addr[k], (int64_t)0); }
    }
    __syncthreads();
    __shared__ int64_t Sg[G];
    if ((int)threadIdx.x < G) {
        int64_t S = 0;
        for (int ck = 0; ck < nch; ck++) S += vals[ck * pw + nl + threadIdx.x];
        Sg[threadIdx.x] = S;
    }
    __syncthreads();
    StatAcc sacc;
    for (int j = threadIdx.x; j < nl; j += 256) {
        int64_t tot = 0;
        for (int ck = 0; ck < nch; ck++) tot += vals[ck * pw + j];
        const int e = e0 + j;
        const float o = rne_div_to_float((i128)tot, Sg[e / HD], 16);
        a.ao[(size_t)h * G * HD + e] = o;
        sacc.add(o);
    }
    if (a.stat_out) stat_flush_block(a.stat_out, sacc);      // max |ao| for the O GEMV
}

// Kernel-tight timing of the calling thread's next attention dispatch: its
// first launch records `start` at the kernel's start, its last `stop` at the
// last kernel's end (hipExtLaunchKernelGGL).
static thread_local hipEvent_t g_at_start = nullptr, g_at_stop = nullptr;
void attn_time_next(hipEvent_t start, hipEvent_t stop) { g_at_start = start; g_at_stop = stop; }
template <typename K> static void launch_ev(K kernel, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const AttnArgs &a) {
    if (e0 || e1) hipExtLaunchKernelGGL(kernel, grid, dim3(256), 0, s, e0, e1, 0, a);
    else hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, a);
}

// decode (B = false: position from the step state) and batched prefill
// (B = true: token grid dimension) are separate instances
template <int EPL, int G, bool B> static void attn_dispatch_b(const AttnArgs &a, int grid_chunks, bool prep, hipStream_t s) {
    const dim3 grid = B ? (a.work ? dim3(a.nwork, a.NKV, 1) : dim3(a.nt, grid_chunks, a.NKV)) : dim3(grid_chunks, a.NKV, 1);
    const hipEvent_t e0 = g_at_start, e1 = g_at_stop;
    g_at_start = g_at_stop = nullptr;
    if (a.mode == FLOAT && a.kvc == KVC_SPINOR) launch_ev(k_attn_float<EPL, G, B, true>, grid, s, e0, e1, a);
    else if (a.mode == FLOAT) launch_ev(k_attn_float<EPL, G, B, false>, grid, s, e0, e1, a);
    else {
        const bool wide = a.chunk > 64;
        if (!B && prep && a.one_launch && a.wslot && a.chunk == 64 && grid_chunks <= WIN_MAXCH) {
            launch_ev(k_attn_exact_window<EPL, G>, grid, s, e0, e1, a);
            return;
        }
        if (!B && prep) {
            if (wide) launch_ev(k_attn_exact_scores<EPL, G, B, !B, 8>, grid, s, e0, nullptr, a);
            else launch_ev(k_attn_exact_scores<EPL, G, B, !B, 4>, grid, s, e0, nullptr, a);
        } else {
            if (wide) launch_ev(k_attn_exact_scores<EPL, G, B, false, 8>, grid, s, e0, nullptr, a);
            else launch_ev(k_attn_exact_scores<EPL, G, B, false, 4>, grid, s, e0, nullptr, a);
        }
        dim3 gv = grid;
        // V-sum chunks of vchunk positions: the span of grid_chunks score
        // chunks meets at most grid_chunks * chunk / vchunk + 2 of them
        if (!B && a.vchunk > a.chunk) gv.x = grid_chunks * a.chunk / a.vchunk + 2;
        launch_ev(k_attn_exact_vsum<EPL, G, B, VSUM_UV>, gv, s, nullptr, e1, a);
    }
}
template <int EPL, int G> static void attn_dispatch(const AttnArgs &a, int grid_chunks, bool prep, hipStream_t s) {
    if (a.nt) attn_dispatch_b<EPL, G, true>(a, grid_chunks, false, s);
    else attn_dispatch_b<EPL, G, false>(a, grid_chunks, prep, s);
}

static void attention_go(const AttnArgs &a, int grid_chunks, bool prep, hipStream_t s) {
    const int G = a.NH / a.NKV;
    if (a.chunk > MAXCH || a.chunk % 16 || grid_chunks > MAXNCH || grid_chunks < 1) {
        launch_fail("attention chunk or chunk count outside the kernel's limits"); return;
    }
    if (a.vchunk && (a.vchunk > MAXCH || a.vchunk % a.chunk)) {
        launch_fail("V-sum chunk not a multiple of the score chunk within the kernel's limits"); return;
    }
    if (a.HD == 256 && G == 2) attn_dispatch<4, 2>(a, grid_chunks, prep, s);
    else if (a.HD == 128 && G == 2) attn_dispatch<2, 2>(a, grid_chunks, prep, s);
    else if (a.HD == 128 && G == 4) attn_dispatch<2, 4>(a, grid_chunks, prep, s);
    else if (a.HD == 64 && G == 2) attn_dispatch<1, 2>(a, grid_chunks, prep, s);
    else if (a.HD == 256 && G == 4) attn_dispatch<4, 4>(a, grid_chunks, prep, s);
    else if (a.HD == 64 && G == 4) attn_dispatch<1, 4>(a, grid_chunks, prep, s);
}
void launch_attention(const AttnArgs &a, int grid_chunks, hipStream_t s) {
    if (prefill_attention_tiled(a)) return launch_prefill_attention(a, s);
    attention_go(a, grid_chunks, false, s);
}

// Workgroups of the exact decode attention (score pass and V-sum) the device
// holds at once, the smaller of the two (0: no such instance).  The host sizes
// global-layer chunks so that a launch is one round of them where it can.
template <int EPL, int G> static int attn_cap_t() {
    int a = 0, b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, k_attn_exact_scores<EPL, G, false, true, 8>, 256, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k_attn_exact_vsum<EPL, G, false, VSUM_UV>, 256, 0) != hipSuccess)
        return 0;
    return a < b ? a : b;
}
template <int EPL, int G> static int window_cap_t() {
    int a = 0;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, k_attn_exact_window<EPL, G>, 256, 0) == hipSuccess ? a : 0;
}
int window_capacity(int HD, int G) {
    int nb = 0, dev = 0, ncu = 0;
    if (HD == 256 && G == 2) nb = window_cap_t<4, 2>();
    else if (HD == 128 && G == 2) nb = window_cap_t<2, 2>();
    else if (HD == 128 && G == 4) nb = window_cap_t<2, 4>();
    else if (HD == 64 && G == 2) nb = window_cap_t<1, 2>();
    else if (HD == 256 && G == 4) nb = window_cap_t<4, 4>();
    else if (HD == 64 && G == 4) nb = window_cap_t<1, 4>();
    if (nb <= 0 || hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return nb * ncu;
}
int attn_capacity(int HD, int G) {
    int nb = 0, dev = 0, ncu = 0;
    if (HD == 256 && G == 2) nb = attn_cap_t<4, 2>();
    else if (HD == 128 && G == 2) nb = attn_cap_t<2, 2>();
    else if (HD == 128 && G == 4) nb = attn_cap_t<2, 4>();
    else if (HD == 64 && G == 2) nb = attn_cap_t<1, 2>();
    else if (HD == 256 && G == 4) nb = attn_cap_t<4, 4>();
    else if (HD == 64 && G == 4) nb = attn_cap_t<1, 4>();
    if (nb <= 0 || hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return nb * ncu;
}


// The step's head preparation and attention: exact-mode decode runs the
// preparation inside the score pass; float mode and batched tokens launch
// k_qk_prep first.
bool attention_fuses_prep(const AttnArgs &a) { return a.mode == EXACT && !a.nt && !a.rec_r; }
void launch_prep_attention(const AttnArgs &a, int grid_chunks, hipStream_t s) {
    if (!attention_fuses_prep(a)) launch_qk_prep(a, s);
    attention_go(a, grid_chunks, attention_fuses_prep(a), s);
}

// ------------------------------------------------------------------ embedding
__device__ __forceinline__ void embed_body(int t_idx, DevW w, const DState *st, const int *tokbuf, int pos0, const int *toks,
                                           float *x, float scale, VecStat *stats, int nstats) {
    // a decode step starts here: clear the step's vector statistics (plain
    // stores; the step's later kernels accumulate into them)
    static_assert(sizeof(VecStat) == 16, "one 16-byte store per statistic replica");
    for (int i = threadIdx.x; i < nstats; i += blockDim.x) ((uint4 *)stats)[i] = make_uint4(0, 0, 0, 0);
    // decode: the step's token; batched: workgroup t embeds toks[t] (several
    // sessions) or tokbuf[pos0 + t] (one session's prefill) into row t
    const int tok = st ? (st->drive == DRIVE_STREAM ? tokbuf[st->pos] : st->tok)
                       : (toks ? toks[t_idx] : tokbuf[pos0 + t_idx]), E = w.cols;
    x += (size_t)t_idx * E;
    const uint8_t *rc = w.codes + (size_t)tok * ((E + 1) / 2);
    const uint16_t *bs = w.bs + (size_t)tok * w.nblk;
    if ((E & 7) == 0) {
        // 8 columns per thread and step: one 4-byte code load, one scale; the
        // steps' loads are independent, so they are all in flight together
        for (int g = threadIdx.x; g < E / 8; g += blockDim.x) {
            const uint32_t c8 = *(const uint32_t *)(rc + 4 * g);
            const float sv = (float)__builtin_bit_cast(_Float16, (unsigned short)bs[g >> 2]);
            float v[8];
            #pragma unroll
            for (int j = 0; j < 8; j++) {
                const int nib = (c8 >> (4 * j)) & 15;           // low nibble = even column
                v[j] = (float)(nib >= 8 ? nib - 16 : nib) * sv;
                if (scale != 0.0f) v[j] *= scale;
            }
            *(float4 *)(x + 8 * g) = make_float4(v[0], v[1], v[2], v[3]);
            *(float4 *)(x + 8 * g + 4) = make_float4(v[4], v[5], v[6], v[7]);
        }
    } else {
        for (int i = threadIdx.x; i < E; i += blockDim.x) {
            const int nib = (rc[i >> 1] >> ((i & 1) * 4)) & 15;
            const int q = nib >= 8 ? nib - 16 : nib;
            const uint32_t hb = bs[i >> 5];
            const float sv = (float)__builtin_bit_cast(_Float16, (unsigned short)hb);
            float v = (float)q * sv;
            if (scale != 0.0f) v *= scale;
            x[i] = v;
        }
    }
}
__global__ __launch_bounds__(256) void k_embed(DevW w, const DState *st, const int *tokbuf, int pos0, const int *toks,
                                                float *x, float scale, VecStat *stats, int nstats) {
    embed_body((int)blockIdx.x, w, st, tokbuf, pos0, toks, x, scale, stats, nstats);
}
// decode: the step's embedding (workgroup 0) and its rotation tables
// (workgroup 1, independent of it) in one launch
__global__ __launch_bounds__(256) void k_embed_rope(DevW w, const DState *st, const int *tokbuf, float *x, float scale,
                                                     VecStat *stats, int nstats, int HD, int mode, const int64_t *fq_g,
                                                     const int64_t *fq_l, float *rope) {
    if (blockIdx.x == 0) embed_body(0, w, st, tokbuf, 0, nullptr, x, scale, stats, nstats);
    else rope_table_body(0, st, 0, nullptr, HD, mode, fq_g, fq_l, rope);
}
void launch_embed(const DevW &embd, const DState *st, const int *tokbuf, float *x, float scale, hipStream_t s,
                  VecStat *stats, int nstats) {
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, s, embd, st, tokbuf, 0, nullptr, x, scale, stats, nstats);
}
void launch_embed_rope(const DevW &embd, const DState *st, const int *tokbuf, float *x, float scale, VecStat *stats,
                       int nstats, int HD, int mode, const int64_t *fq_g, const int64_t *fq_l, float *rope, hipStream_t s) {
    hipLaunchKernelGGL(k_embed_rope, dim3(2), dim3(256), 0, s, embd, st, tokbuf, x, scale, stats, nstats, HD, mode,
                       fq_g, fq_l, rope);
}
void launch_embed_batch(const DevW &embd, const int *tokbuf, int pos0, int T, float *x, float scale, hipStream_t s,
                        const int *toks) {
    hipLaunchKernelGGL(k_embed, dim3(T), dim3(256), 0, s, embd, nullptr, tokbuf, pos0, toks, x, scale, nullptr, 0);
}
__global__ void k_advance(DState *st) {
    if (threadIdx.x == 0 && st->drive == DRIVE_STREAM) st->pos = st->pos + 1;
}
void launch_advance(DState *st, hipStream_t s) { hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, st); }

// ------------------------------------------------------------------ argmax
// lowest index among the maxima (strict '>' scan order of the reference callers)
__device__ __forceinline__ void amax_merge(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}
__global__ __launch_bounds__(256) void k_argmax(const float *lg, int V, float *pv, int *pi, int *counter, DState *st, int *gen_log) {
    __shared__ float sv[4]; __shared__ int si[4]; __shared__ int is_last;
    float v = -INFINITY; int idx = 0x7FFFFFFF;
    for (int j = blockIdx.x * 256 + threadIdx.x; j < V; j += gridDim.x * 256) amax_merge(v, idx, lg[j], j);
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax_merge(v, idx, __shfl_xor(v, o, 64), __shfl_xor(idx, o, 64));
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = v; si[threadIdx.x >> 6] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) amax_merge(v, idx, sv[w], si[w]);
        st_agent(&pv[blockIdx.x], v); st_agent(&pi[blockIdx.x], idx);
        mem_complete();
        is_last = arrive(counter) == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (!is_last) return;
    // the last workgroup merges the per-workgroup maxima, one per thread
    float bv = -INFINITY; int bi = 0x7FFFFFFF;
    for (int b = threadIdx.x; b < (int)gridDim.x; b += 256) amax_merge(bv, bi, ld_agent(&pv[b]), ld_agent(&pi[b]));
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax_merge(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int w = 1; w < 4; w++) amax_merge(bv, bi, sv[w], si[w]);
    if (bi == 0x7FFFFFFF) bi = 0;
    st->tok = bi;
    if (gen_log) gen_log[st->pos] = bi;
    if (st->drive == DRIVE_GREEDY) st->pos = st->pos + 1;
    reset_counter(counter);
}
// greedy token of each of T logit rows (lowest index among the maxima); one
// 1024-thread workgroup per row, 16-byte loads with four in flight per thread
constexpr int AMR_T = 1024;
__global__ __launch_bounds__(AMR_T) void k_argmax_rows(const float *lg, int V, int *out) {
    __shared__ float sv[AMR_T / 64]; __shared__ int si[AMR_T / 64];
    const float *row = lg + (size_t)blockIdx.x * V;
    const int tid = threadIdx.x;
    float v = -INFINITY; int idx = 0x7FFFFFFF;
    if ((V & 3) == 0) {                              // rows start 16-byte aligned
        const float4 *r4 = (const float4 *)row;
        const int V4 = V >> 2;
        int j = tid;
        for (; j + 3 * AMR_T < V4; j += 4 * AMR_T) {
            float4 q[4];
            #pragma unroll
            for (int u = 0; u < 4; u++) q[u] = r4[j + u * AMR_T];
            #pragma unroll
            for (int u = 0; u < 4; u++) {
                const int b = 4 * (j + u * AMR_T);
                amax_merge(v, idx, q[u].x, b); amax_merge(v, idx, q[u].y, b + 1);
                amax_merge(v, idx, q[u].z, b + 2); amax_merge(v, idx, q[u].w, b + 3);
            }
        }
        for (; j < V4; j += AMR_T) {
            const float4 q = r4[j];
            amax_merge(v, idx, q.x, 4 * j); amax_merge(v, idx, q.y, 4 * j + 1);
            amax_merge(v, idx, q.z, 4 * j + 2); amax_merge(v, idx, q.w, 4 * j + 3);
        }
    } else {
        for (int j = tid; j < V; j += AMR_T) amax_merge(v, idx, row[j], j);
    }
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax_merge(v, idx, __shfl_xor(v, o, 64), __shfl_xor(idx, o, 64));
    if ((tid & 63) == 0) { sv[tid >> 6] = v; si[tid >> 6] = idx; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < AMR_T / 64; w++) amax_merge(v, idx, sv[w], si[w]);
        out[blockIdx.x] = idx == 0x7FFFFFFF ? 0 : idx;
    }
}
void launch_argmax_rows(const float *logits, int V, int T, int *out, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_rows, dim3(T), dim3(AMR_T), 0, s, logits, V, out);
}

int argmax_blocks(int V) { int b = (V + 2047) / 2048; return b < 1 ? 1 : (b > 256 ? 256 : b); }
void launch_argmax(const float *logits, int V, float *pval, int *pidx, int *counter, DState *st,
                   int *gen_log, int nblocks, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax, dim3(nblocks), dim3(256), 0, s, logits, V, pval, pidx, counter, st, gen_log);
}

}  // namespace kvd
