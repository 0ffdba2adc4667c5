// kvd_pattn.hip -- exact-mode attention of one session's batched prefill on
// the global (full-context) layers: the batch's tokens share every K and V row
// they read instead of each token streaming the whole context.
//
// The arithmetic is the decode attention's (kvd_attn.hip), so every token's
// scores, weights and output are bit-identical to a decode step's:
//   ip = <qi, ki> exact, qi = rne(q 2^16), ki the stored int32 K;
//   z = llround(((float)((double)ip / 2^32) * ascale) * 2^14);
//   w = exp_fixed(((z - M) 2^30) >> 14) >> 8 (Q22), M the token-head's max;
//   out = RNE(sum_p w vq / (sum_p w * 2^16)).
//
// Score pass, on the int8 matrix cores: qi and ki are split into four balanced
// base-256 digits; every digit pair (a, b) is one int8 MFMA product with an
// exact int32 sum (|sum| <= HD 2^14), and ip = sum_{a,b} 2^(8(a+b)) P_ab in
// int64 -- the same integer as the decode kernels' int64 dot product.  A
// workgroup scores 64 positions for 64 token-heads (one 16 x 16 tile row per
// wave); the positions' K digits are staged once in LDS.  A workgroup whose q
// or K values do not fit four balanced digits (|x| > 127 (1 + 2^8 + 2^16 +
// 2^24)) scores its tile on the vector units instead, with the same result.
//
// V-sum pass: a workgroup takes a 2048-position chunk for a group of tokens:
// each V row is read once for all of the group's token-heads (FP64 FMAs on
// integers below 2^53, as in decode), partial sums go to the tokens' int64
// totals by order-free atomics, and the group's last workgroup divides.
//
// Sliding-window layers (win >= 0): token t attends [s0(t), pos(t)], s0(t) =
// max(0, pos(t) - win + 1), as in decode; chunks are absolute position ranges
// from the batch's lowest window start, each pass masks a token's positions
// below s0(t), and a workgroup whose chunk lies below its token group's
// earliest window start does nothing.
#include "kvd_internal.h"
#include "kvd_exact.h"
#include "kvd_vec.h"
#include "kvd_spinor.h"

namespace kvd {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int PS_CH = 64;            // positions per score workgroup (and per chunk maximum)
constexpr int PV_CH = 2048;          // positions per V-sum workgroup (full-context layers)
constexpr int PV_SUB = 512;          // ... in sub-chunks of 128 rows per wave (FP64 sums below 2^53)
constexpr int DIG_MAX = 127 * (1 + 256 + 65536 + 16777216);   // largest |x| of four balanced digits

__device__ __forceinline__ const float *pg(const AttnArgs &a, int pos) {
    const int lp = pos / PAGE;
    return gmem(a.pages)[a.ring_pages ? lp % a.ring_pages : lp];
}
// the first position token t of the batch attends
__host__ __device__ __forceinline__ int win_start(const AttnArgs &a, int t) {
    const int q = a.pos0 + t - a.win + 1;
    return a.win >= 0 && q > 0 ? q : 0;
}

// x = d0 + 2^8 d1 + 2^16 d2 + 2^24 d3, d in [-128, 127] (|x| <= DIG_MAX)
__device__ __forceinline__ void digits4(int32_t x, int32_t d[4]) {
    #pragma unroll
    for (int k = 0; k < 4; k++) {
        d[k] = ((x + 128) & 255) - 128;
        x = (x - d[k]) >> 8;
    }
}

// ---------------------------------------------------------------- score pass
// grid: (token groups of 64 / G tokens, 64-position chunks, kv heads); the
// token group runs fastest, so the groups reading one chunk's K run together.
// zscratch and the chunk maxima are laid out per token as for the decode
// kernels: token t's scores at zscratch + t NH zstride, its maximum of chunk c
// of token-head q at part_ml + t NH max_chunks 4 + (q max_chunks + c) 4.
template <int EPL, int G>
__global__ __launch_bounds__(256) void k_pattn_scores(AttnArgs a) {
    constexpr int HD = EPL * 64, KS = HD / 32, TPW = 16 / G, TWG = 4 * TPW, KROW = HD + 16;
    const int tg = blockIdx.x, c = win_start(a, 0) / PS_CH + (int)blockIdx.y, h = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t0 = tg * TWG;
    const int tend = t0 + TWG < a.nt ? t0 + TWG : a.nt;
    const int pos_hi = a.pos0 + tend - 1;               // the group's last token attends up to here
    const int cs = c * PS_CH;
    if (t0 >= a.nt || cs > pos_hi || cs + PS_CH <= win_start(a, t0)) return;
    const int np = pos_hi - cs + 1 < PS_CH ? pos_hi - cs + 1 : PS_CH;
    __shared__ __align__(16) int8_t kd[4][PS_CH][KROW];   // K digits [digit][position][dim]
    __shared__ int s_wide;
    if (threadIdx.x == 0) s_wide = 0;
    const size_t QD = (size_t)a.NH * HD;
    // this wave's 16 token-heads: lane row m = lane % 16 -> token t0 + wave TPW + m / G, head h G + m % G
    const int m = lane & 15, j = lane >> 4;
    const int tq = t0 + wave * TPW + m / G;
    const float *qp = a.qr + (size_t)(tq < a.nt ? tq : 0) * QD + (size_t)(h * G + m % G) * HD + 8 * j;
    int32_t qi[KS][8];
    bool wide = false;
    #pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const float4 v0 = *(const float4 *)(qp + 32 * ks), v1 = *(const float4 *)(qp + 32 * ks + 4);
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        #pragma unroll
        for (int e = 0; e < 8; e++) {
            qi[ks][e] = tq < a.nt ? (int32_t)rintf(v[e] * 65536.0f) : 0;
            wide |= qi[ks][e] > DIG_MAX || qi[ks][e] < -DIG_MAX;
        }
    }
    __syncthreads();                                    // s_wide is cleared
    // K rows of the chunk as digit planes: thread i takes 16 consecutive dims of
    // a row.  The chunk is one page (PS_CH == PAGE, chunks aligned), looked up
    // once; every row load is requested before the first is used, rows past
    // the group's last position clamped to it (their scores are never stored,
    // and a copy of a row changes no range check)
    static_assert(PS_CH == PAGE && PS_CH * (HD / 16) % 256 == 0, "one page per chunk, whole row pieces per thread");
    constexpr int KIT = PS_CH * (HD / 16) / 256;
    const int32_t *kpage = (const int32_t *)pg(a, cs) + (size_t)h * PAGE * HD;
    int4 kx[KIT][4];
    #pragma unroll
    for (int it = 0; it < KIT; it++) {
        const int i = threadIdx.x + 256 * it, pl = i / (HD / 16), d0 = (i % (HD / 16)) * 16;
        const int32_t *row = kpage + (size_t)(pl < np ? pl : np - 1) * HD + d0;
        #pragma unroll
        for (int q = 0; q < 4; q++) kx[it][q] = *gmem((const int4 *)(row + 4 * q));
    }
    // every row is requested before any is used: the conversion below takes
    // its inputs through a zero the compiler cannot see through, produced
    // after the loads (otherwise it hoists the conversion between them, and
    // each iteration waits for its own rows before the next is requested)
    int32_t after_loads;
    asm volatile("v_mov_b32 %0, 0" : "=v"(after_loads) : : "memory");
    #pragma unroll
    for (int it = 0; it < KIT; it++) {
        const int i = threadIdx.x + 256 * it, pl = i / (HD / 16), d0 = (i % (HD / 16)) * 16;
        int32_t x[16];
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            x[4 * q] = kx[it][q].x ^ after_loads; x[4 * q + 1] = kx[it][q].y ^ after_loads;
            x[4 * q + 2] = kx[it][q].z ^ after_loads; x[4 * q + 3] = kx[it][q].w ^ after_loads;
        }
        uint32_t w[4][4] = {};
        #pragma unroll
        for (int e = 0; e < 16; e++) {
            wide |= x[e] > DIG_MAX || x[e] < -DIG_MAX;
            int32_t d[4];
            digits4(x[e], d);
            #pragma unroll
            for (int b = 0; b < 4; b++) w[b][e >> 2] |= (uint32_t)(d[b] & 255) << (8 * (e & 3));
        }
        #pragma unroll
        for (int b = 0; b < 4; b++) *(uint4 *)&kd[b][pl][d0] = make_uint4(w[b][0], w[b][1], w[b][2], w[b][3]);
    }
    if (__any(wide) && lane == 0) s_wide = 1;
    __syncthreads();
    const bool mfma = s_wide == 0;

    // this wave's A operands: digit a of qi at dims 32 ks + 8 j .. +8 (byte e = dim 8 j + e)
    long A[4][KS];
    #pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        uint32_t lo[4] = {}, hi[4] = {};
        #pragma unroll
        for (int e = 0; e < 8; e++) {
            int32_t d[4];
            digits4(qi[ks][e], d);
            #pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint32_t byte = (uint32_t)(d[b] & 255) << (8 * (e & 3));
                if (e < 4) lo[b] |= byte; else hi[b] |= byte;
            }
        }
        #pragma unroll
        for (int b = 0; b < 4; b++) A[b][ks] = (long)(((uint64_t)hi[b] << 32) | lo[b]);
    }
    int mx[4] = {INT32_MIN, INT32_MIN, INT32_MIN, INT32_MIN};
    const int rowq = 4 * j;                              // output rows 4 j .. 4 j + 3 of the tile
    for (int nt = 0; nt < PS_CH / 16; nt++) {
        if (nt * 16 >= np) break;
        const int p = cs + nt * 16 + m;                  // this lane's output column (position)
        int64_t ip[4] = {0, 0, 0, 0};
        if (mfma) {
            v4i acc[16];
            #pragma unroll
            for (int k = 0; k < 16; k++) acc[k] = (v4i){0, 0, 0, 0};
            #pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                long B[4];
                #pragma unroll
                for (int b = 0; b < 4; b++) B[b] = *(const long *)&kd[b][nt * 16 + m][32 * ks + 8 * j];
                #pragma unroll
                for (int a2 = 0; a2 < 4; a2++)
                    #pragma unroll
                    for (int b = 0; b < 4; b++)
                        acc[a2 * 4 + b] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[a2][ks], B[b], acc[a2 * 4 + b], 0, 0, 0);
            }
            #pragma unroll
            for (int i = 0; i < 4; i++)
                #pragma unroll
                for (int a2 = 0; a2 < 4; a2++)
                    #pragma unroll
                    for (int b = 0; b < 4; b++) ip[i] += (int64_t)acc[a2 * 4 + b][i] * ((int64_t)1 << (8 * (a2 + b)));
        } else {
            // out-of-range magnitudes: the tile on the vector units, from the
            // digits (x = sum_b 2^(8b) d_b exactly holds only in range, so the
            // int32 values are rebuilt from the rows themselves)
            #pragma unroll
            for (int i = 0; i < 4; i++) {
                const int mm = rowq + i;
                const int tt = t0 + wave * TPW + mm / G;
                if (tt >= a.nt || p > pos_hi) continue;
                const float *q2 = a.qr + (size_t)tt * QD + (size_t)(h * G + mm % G) * HD;
                const int32_t *krow = (const int32_t *)pg(a, p) + ((size_t)h * PAGE + (p & (PAGE - 1))) * HD;
                int64_t s = 0;
                for (int d = 0; d < HD; d++) s += (int64_t)(int32_t)rintf(q2[d] * 65536.0f) * gmem(krow)[d];
                ip[i] = s;
            }
        }
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const int mm = rowq + i;
            const int tt = t0 + wave * TPW + mm / G;
            if (tt < a.nt && p <= a.pos0 + tt && p >= win_start(a, tt)) {
                const float scv = (float)((double)ip[i] / 4294967296.0) * a.ascale;
                const int32_t z = (int32_t)llround_pow2<14>(scv);
                a.zscratch[(size_t)tt * a.NH * a.zstride + (size_t)(h * G + mm % G) * a.zstride + p] = z;
                mx[i] = z > mx[i] ? z : mx[i];
            }
        }
    }
    // chunk maxima: over the 16 lanes of a row group
    #pragma unroll
    for (int i = 0; i < 4; i++) {
        int v = mx[i];
        #pragma unroll
        for (int o = 1; o < 16; o <<= 1) { const int w = __shfl_xor(v, o, 64); v = w > v ? w : v; }
        mx[i] = v;
    }
    if (m == 0) {
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const int mm = rowq + i;
            const int tt = t0 + wave * TPW + mm / G;
            if (tt < a.nt && cs <= a.pos0 + tt && cs + PS_CH > win_start(a, tt))
                ((int32_t *)a.part_ml)[(size_t)tt * a.NH * a.max_chunks * 4 + ((size_t)(h * G + mm % G) * a.max_chunks + c) * 4] = mx[i];
        }
    }
}

// --------------------------------------------------------------- V-sum pass
// grid: (token groups of TT tokens, 2048-position chunks, kv heads).  NQ =
// TT G token-heads share each V row.  Token t's totals are its decode-layout
// accumulators (vacc + t QD VREP, vacc_s + t NH VREP, replica 0) and its
// group's arrivals count on counter[t0 NKV + h].
// WIN (sliding-window layers): one 8-wave workgroup per (token group, kv
// head) takes the group's whole span (at most win + TT - 1 rows), adds the
// waves' partials in LDS and divides: no cross-workgroup exchange.
template <int EPL, int G, int TT, bool WIN>
__global__ __launch_bounds__(WIN ? 512 : 256) void k_pattn_vsum(AttnArgs a) {
    constexpr int HD = EPL * 64, NQ = TT * G, UV = WIN ? 8 : 4, NW = WIN ? 8 : 4, NT = 64 * NW;
    const int VC = PV_CH;
    const int tg = blockIdx.x, c = win_start(a, 0) / VC + (int)blockIdx.y, h = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t0 = tg * TT;
    const int tend = t0 + TT < a.nt ? t0 + TT : a.nt;
    const int pos_hi = a.pos0 + tend - 1;
    const int s0g = win_start(a, t0);                   // the group's lowest window start
    const int nch = WIN ? 1 : pos_hi / VC - s0g / VC + 1;   // chunks of this group (the arrival count)
    if (t0 >= a.nt || (!WIN && (c < s0g / VC || c > pos_hi / VC))) return;
    // this workgroup's rows: [cs, cs + np) within the chunk and the group's span
    const int cs = WIN ? s0g : (c * VC > s0g ? c * VC : s0g);
    const int np = WIN ? pos_hi - s0g + 1 : (pos_hi < c * VC + VC - 1 ? pos_hi : c * VC + VC - 1) - cs + 1;
    const size_t QD = (size_t)a.NH * HD;
    __shared__ int32_t ew[NQ][PV_SUB + UV];              // island weights (Q22) of a sub-chunk, 0 where masked and past it
    __shared__ int s_M[NQ];
    __shared__ int64_t ored[NQ][HD];                      // the waves' partials, added in LDS (order-free)
    __shared__ int64_t sred[NQ];
    __shared__ int is_last;
    for (int i = threadIdx.x; i < NQ * HD; i += NT) ored[i / HD][i % HD] = 0;
    if (threadIdx.x < NQ) sred[threadIdx.x] = 0;
    if (threadIdx.x < NQ * UV) ew[threadIdx.x / UV][PV_SUB + threadIdx.x % UV] = 0;
    // each token-head's maximum over its 64-position chunk maxima (wave w: token-heads w, w+4, ..)
    for (int q = wave; q < NQ; q += NW) {
        const int tt = t0 + q / G;
        int t = INT32_MIN;
        if (tt < a.nt) {
            const int n64 = (a.pos0 + tt) / PS_CH + 1;
            const int32_t *pml = (const int32_t *)a.part_ml + (size_t)tt * a.NH * a.max_chunks * 4 +
                                 (size_t)(h * G + q % G) * a.max_chunks * 4;
            for (int k = win_start(a, tt) / PS_CH + lane; k < n64; k += 64) { const int v = pml[(size_t)k * 4]; t = v > t ? v : t; }
        }
        t = wave_allmax_i(t);
        if (lane == 0) s_M[q] = t;
    }
    __syncthreads();
    for (int sb = 0; sb < np; sb += PV_SUB) {
        const int ns = np - sb < PV_SUB ? np - sb : PV_SUB;
        // the sub-chunk's scores: every slot's load is issued first (token and
        // position clamped into range, masked slots' values unused), then the
        // weights are formed -- one round trip, not one per slot
        static_assert(NQ * PV_SUB % NT == 0, "whole slots per thread");
        constexpr int FPT = NQ * PV_SUB / NT;
        int32_t zz[FPT];
        #pragma unroll
        for (int k = 0; k < FPT; k++) {
            const int i = threadIdx.x + NT * k, q = i / PV_SUB, jj = i % PV_SUB;
            const int tt = t0 + q / G < a.nt ? t0 + q / G : a.nt - 1;
            const int p = cs + sb + (jj < ns ? jj : ns - 1);
            zz[k] = a.zscratch[(size_t)tt * a.NH * a.zstride + (size_t)(h * G + q % G) * a.zstride + p];
        }
        #pragma unroll
        for (int k = 0; k < FPT; k++) {
            const int i = threadIdx.x + NT * k, q = i / PV_SUB, jj = i % PV_SUB, tt = t0 + q / G, p = cs + sb + jj;
            int32_t w = 0;
            if (jj < ns && tt < a.nt && p <= a.pos0 + tt && p >= win_start(a, tt))
                w = (int32_t)(exp_fixed((((int64_t)zz[k] - (int64_t)s_M[q]) * ONE) >> 14) >> 8);
            ew[q][jj] = w;
        }
        __syncthreads();
        // FP64 V-sum of the sub-chunk: a wave's rows (<= 128) keep every
        // partial an integer below 2^53; the partials then add in int64
        double o[NQ][EPL];
        #pragma unroll
        for (int q = 0; q < NQ; q++)
            #pragma unroll
            for (int e = 0; e < EPL; e++) o[q][e] = 0.0;
        // UV rows per wave and step, every load issued (rows past ns clamped to
        // the last row; they meet zero weights), the step's at most two pages
        // looked up once; the next step's rows are requested before this
        // step's FMAs, into the other buffer (no register copies)
        const size_t voff = (size_t)a.NKV * PAGE * HD + (size_t)h * PAGE * HD;
        auto load_v = [&](int j0, int32_t (&v)[UV][EPL]) {
            const int pa = __builtin_amdgcn_readfirstlane(cs + sb + (j0 < ns ? j0 : ns - 1));
            const int pb = __builtin_amdgcn_readfirstlane(cs + sb + (j0 + UV - 1 < ns ? j0 + UV - 1 : ns - 1));
            const int32_t *ba = (const int32_t *)pg(a, pa) + voff, *bb = (const int32_t *)pg(a, pb) + voff;
            #pragma unroll
            for (int u = 0; u < UV; u++) {
                const int p = __builtin_amdgcn_readfirstlane(cs + sb + (j0 + u < ns ? j0 + u : ns - 1));
                const int32_t *row = (p / PAGE == pa / PAGE ? ba : bb) + (size_t)(p & (PAGE - 1)) * HD;
                const int32_t *src = row + lane * EPL;
                if constexpr (EPL == 4) {
                    const int4 t = *gmem((const int4 *)src); v[u][0] = t.x; v[u][1] = t.y; v[u][2] = t.z; v[u][3] = t.w;
                } else if constexpr (EPL == 2) {
                    const int2 t = *gmem((const int2 *)src); v[u][0] = t.x; v[u][1] = t.y;
                } else {
                    v[u][0] = *gmem(src);
                }
            }
        };
        // one row at a time (the scheduler would otherwise hoist every
        // weight of the step into registers ahead of the FMAs)
        auto vrows = [&](const int32_t (&v)[UV][EPL], int j0) {
            #pragma unroll
            for (int u = 0; u < UV; u++) {
                #pragma unroll
                for (int q = 0; q < NQ; q++) {
                    const double w = (double)ew[q][j0 + u];
                    #pragma unroll
                    for (int e = 0; e < EPL; e++) o[q][e] = fma(w, (double)v[u][e], o[q][e]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        int32_t va[UV][EPL], vb[UV][EPL];
        load_v(wave * UV, va);
        __builtin_amdgcn_sched_barrier(0);
        for (int j0 = wave * UV; j0 < ns; j0 += 2 * NW * UV) {
            load_v(j0 + NW * UV, vb);
            __builtin_amdgcn_sched_barrier(0);
            vrows(va, j0);
            if (j0 + NW * UV >= ns) break;
            load_v(j0 + 2 * NW * UV, va);
            __builtin_amdgcn_sched_barrier(0);
            vrows(vb, j0 + NW * UV);
        }
        #pragma unroll
        for (int q = 0; q < NQ; q++)
            #pragma unroll
            for (int e = 0; e < EPL; e++) atomicAdd((unsigned long long *)&ored[q][lane * EPL + e], (unsigned long long)(int64_t)o[q][e]);
        // denominators of the sub-chunk
        for (int q = wave; q < NQ; q += NW) {
            int64_t sum = 0;
            for (int jj = lane; jj < PV_SUB; jj += 64) sum += ew[q][jj];
            sum = wave_allsum(sum);
            if (lane == 0) atomicAdd((unsigned long long *)&sred[q], (unsigned long long)sum);
        }
        __syncthreads();                                 // ew is consumed
    }
    if constexpr (WIN) {
        // the whole span was this workgroup's: divide the totals
        for (int i = threadIdx.x; i < NQ * HD; i += NT) {
            const int q = i / HD, d = i % HD, tt = t0 + q / G;
            if (tt < a.nt) a.ao[(size_t)tt * QD + (size_t)(h * G + q % G) * HD + d] = rne_div_to_float((i128)ored[q][d], sred[q], 16);
        }
        return;
    }
    for (int i = threadIdx.x; i < NQ * HD; i += NT) {
        const int q = i / HD, d = i % HD, tt = t0 + q / G;
        if (tt >= a.nt) continue;
        const int64_t t = ored[q][d];
        atomicAdd((unsigned long long *)&a.vacc[(size_t)tt * QD * VREP + (size_t)(h * G + q % G) * HD + d], (unsigned long long)t);
    }
    __syncthreads();
    if (threadIdx.x < NQ) {
        const int q = threadIdx.x, tt = t0 + q / G;
        if (tt < a.nt)
            atomicAdd((unsigned long long *)&a.vacc_s[(size_t)tt * a.NH * VREP + h * G + q % G], (unsigned long long)sred[q]);
    }
    mem_complete();
    __syncthreads();
    if (threadIdx.x == 0) is_last = (arrive(&a.counter[(size_t)t0 * a.NKV + h]) == nch - 1);
    __syncthreads();
    if (!is_last) return;
    // the group's totals are read and cleared for the next launch in one atomic step
    __shared__ int64_t Sg[NQ];
    if (threadIdx.x < NQ) {
        const int q = threadIdx.x, tt = t0 + q / G;
        Sg[q] = tt < a.nt ? (int64_t)__hip_atomic_exchange((unsigned long long *)&a.vacc_s[(size_t)tt * a.NH * VREP + h * G + q % G],
                                                           0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 1;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < NQ * HD; i += NT) {
        const int q = i / HD, d = i % HD, tt = t0 + q / G;
        if (tt >= a.nt) continue;
        const int64_t tot = (int64_t)__hip_atomic_exchange(
            (unsigned long long *)&a.vacc[(size_t)tt * QD * VREP + (size_t)(h * G + q % G) * HD + d], 0ull,
            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.ao[(size_t)tt * QD + (size_t)(h * G + q % G) * HD + d] = rne_div_to_float((i128)tot, Sg[q], 16);
    }
    if (threadIdx.x == 0) reset_counter(&a.counter[(size_t)t0 * a.NKV + h]);
}

template <int EPL, int G>
void pattn_go(const AttnArgs &a, hipStream_t s) {
    constexpr int TPW = 16 / G, TWG = 4 * TPW, TT = 8 / G;
    const int pos_hi = a.pos0 + a.nt - 1, lo = win_start(a, 0);
    const dim3 g1((a.nt + TWG - 1) / TWG, pos_hi / PS_CH - lo / PS_CH + 1, a.NKV);
    hipLaunchKernelGGL((k_pattn_scores<EPL, G>), g1, dim3(256), 0, s, a);
    if (a.win >= 0) {
        hipLaunchKernelGGL((k_pattn_vsum<EPL, G, TT, true>), dim3((a.nt + TT - 1) / TT, 1, a.NKV), dim3(512), 0, s, a);
    } else {
        const dim3 g2((a.nt + TT - 1) / TT, pos_hi / PV_CH - lo / PV_CH + 1, a.NKV);
        hipLaunchKernelGGL((k_pattn_vsum<EPL, G, TT, false>), g2, dim3(256), 0, s, a);
    }
}

}  // namespace

bool prefill_attention_tiled(const AttnArgs &a) {
    const int G = a.NH / a.NKV;
    return a.mode == EXACT && a.nt > 0 && !a.tpages && !a.tpos &&
           a.kvc == KVC_PLAIN && (a.HD == 64 || a.HD == 128 || a.HD == 256) && (G == 2 || G == 4);
}

void launch_prefill_attention(const AttnArgs &a, hipStream_t s) {
    const int G = a.NH / a.NKV;
    const int pos_hi = a.pos0 + a.nt - 1;
    // the chunk maxima and score rows must hold every position of the batch
    if (!prefill_attention_tiled(a) || pos_hi / PS_CH + 1 > a.max_chunks || pos_hi >= a.zstride)
        return launch_fail("tiled prefill attention: arguments outside the kernels' limits");
    if (a.HD == 256 && G == 2) pattn_go<4, 2>(a, s);
    else if (a.HD == 256) pattn_go<4, 4>(a, s);
    else if (a.HD == 128 && G == 2) pattn_go<2, 2>(a, s);
    else if (a.HD == 128) pattn_go<2, 4>(a, s);
    else if (G == 2) pattn_go<1, 2>(a, s);
    else pattn_go<1, 4>(a, s);
}

}  // namespace kvd
