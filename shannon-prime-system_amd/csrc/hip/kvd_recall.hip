// kvd_recall.hip -- ARM recall on the device: the router (projected-score
// top-k per q head) and attention over each q head's recalled positions.
//
// Reference: core/arm/arm.c (the sequential float projection :31-45, the
// selection sinks u top-(B-W-sink) u recent-W :110-160, identity when B = 0 or
// the context is within budget) and core/forward/decode.c:740-790 (attention
// over the recall set).  The K sidecar is written at append time by the head
// preparation (kvd_qkprep.h recall_sidecar); the query projection and the
// candidate scores here are the same sequential float sums with separate
// multiply and add, so the scores -- and the selected set -- are the CPU's
// whenever q and K are (exact mode).  The top-k keeps the largest scores; at
// an exact tie on the k-th score it keeps the lowest positions (the
// reference's quickselect may keep other tied positions: the scores are float
// sums of r products and exact ties do not occur on real data).
//
// Exact mode: int64 scores, the island softmax grid and an exact V-sum, all
// integers, so the order of the recalled positions changes no bit.  Float
// mode: float scores, expf weights and float sums (within the float tolerance
// of the CPU's list-order sums).
//
// Page layout with the sidecar: K [NKV][PAGE][HD], V [NKV][PAGE][HD], then the
// sidecar [NKV][PAGE][r] floats.
#include "kvd_internal.h"
#include "kvd_exact.h"
#include "kvd_vec.h"

namespace kvd {

namespace {

__device__ __forceinline__ const float *rc_page(const RecallArgs &rc, int pos) { return gmem(rc.pages)[pos / PAGE]; }
// row of position s of kv head kvh: K (vpart = 0) or V (vpart = 1)
__device__ __forceinline__ const int32_t *rc_row(const RecallArgs &rc, int kvh, int s, int vpart) {
    return (const int32_t *)rc_page(rc, s) + (size_t)vpart * rc.NKV * PAGE * rc.HD +
           ((size_t)kvh * PAGE + (s & (PAGE - 1))) * rc.HD;
}

// float -> unsigned key with the float order (larger float, larger key), and
// back.  -0.0 takes +0.0's key: equal floats get equal keys, as the
// reference's comparisons (`>`, core/arm/arm.c:49-76) treat them.
__device__ __forceinline__ uint32_t order_key(float f) {
    uint32_t b = __float_as_uint(f);
    if (b == 0x80000000u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Selection geometry of position pos (sp_arm_select's clamps, arm.c:110-160).
struct SelGeom { int ident, sink, cand_hi, topk, m; };
__device__ __forceinline__ SelGeom sel_geom(const RecallArgs &rc, int pos) {
    SelGeom g;
    g.ident = rc.B <= 0 || pos + 1 <= rc.B;
    const int W = rc.W > pos + 1 ? pos + 1 : rc.W;
    g.sink = rc.sink > pos + 1 ? pos + 1 : rc.sink;
    g.cand_hi = pos + 1 - W;
    if (g.cand_hi < g.sink) g.cand_hi = g.sink;
    if (g.cand_hi > pos + 1) g.cand_hi = pos + 1;
    g.topk = rc.B - W - g.sink;
    if (g.topk < 0) g.topk = 0;
    if (g.topk > g.cand_hi - g.sink) g.topk = g.cand_hi - g.sink;
    g.m = g.ident ? pos + 1 : g.sink + g.topk + (pos + 1 - g.cand_hi);
    return g;
}

// ---- router 1: the candidates' projected scores (grid: score_blocks x NKV)
// One thread per candidate position: its sidecar row (r floats, contiguous in
// the page) is read once for all G q heads of the kv head; each head's score
// sum_p pq[p] * side[p] is sequential in p with separate multiply and add.
// With KVSEL (SP_RECALL_KVSEL, core/forward/decode.c:738-757) the kv head
// scores once, with the projection of its group-centroid query
// qg = ((0 + q_0) + q_1) + ... (float, in head order), formed here from the
// rotated q heads; its keys go to the group leader's row (kvh * G).
template <int RT>
__global__ __launch_bounds__(256) void k_recall_score(RecallArgs rc) {
    const int pos = rc.st->pos, kvh = blockIdx.y, G0 = rc.NH / rc.NKV;
    const SelGeom g = sel_geom(rc, pos);
    if (g.ident || g.topk == 0) return;
    const int r = RT ? RT : rc.r, HD = rc.HD;
    const int G = rc.kvsel ? 1 : G0;                     // heads scored here
    __shared__ float pq[RECALL_MAX_GROUP * 64];
    if (rc.kvsel) {
        __shared__ float qg[256];
        for (int i = threadIdx.x; i < HD; i += 256) {
            float a = 0.0f;
            for (int gh = 0; gh < G0; gh++) a = __fadd_rn(a, rc.qr[(size_t)(kvh * G0 + gh) * HD + i]);
            qg[i] = a;
        }
        __syncthreads();
        if ((int)threadIdx.x < r) {                      // sequential +-1 sum over d, as the sidecar's
            const int p = threadIdx.x, NW = HD / 32;
            float a = 0.0f;
            for (int d = 0; d < HD; d++)
                a = __fadd_rn(a, ((rc.Rb[(size_t)p * NW + (d >> 5)] >> (d & 31)) & 1u) ? qg[d] : -qg[d]);
            pq[p] = a;
        }
    } else {
        for (int i = threadIdx.x; i < G * r; i += 256) pq[i] = rc.pq[(size_t)kvh * G * r + i];
    }
    __syncthreads();
    for (int s = g.sink + blockIdx.x * 256 + threadIdx.x; s < g.cand_hi; s += gridDim.x * 256) {
        const float *side = rc.side + ((size_t)s * rc.NKV + kvh) * r;
        float row[RT ? RT : 64];
        if constexpr (RT) {
            #pragma unroll
            for (int q = 0; q < RT / 4; q++) {
                const float4 v = *gmem((const float4 *)(side + 4 * q));
                row[4 * q] = v.x; row[4 * q + 1] = v.y; row[4 * q + 2] = v.z; row[4 * q + 3] = v.w;
            }
        }
        for (int gh = 0; gh < G; gh++) {
            float a = 0.0f;
            if constexpr (RT) {
                #pragma unroll
                for (int p = 0; p < RT; p++) a = __fadd_rn(a, __fmul_rn(pq[gh * RT + p], row[p]));
            } else {
                for (int p = 0; p < r; p++) a = __fadd_rn(a, __fmul_rn(pq[gh * r + p], gmem(side)[p]));
            }
            rc.keys[(size_t)(kvh * G0 + gh) * rc.kstride + s] = order_key(a);
        }
    }
}

// inclusive prefix sum over the lanes of a wave
__device__ __forceinline__ int wave_incl_scan(int v) {
    const int lane = __lane_id();
    #pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    return v;
}

// ---- router 2: one q head's recall set (grid: NH, 1024 threads)
// The candidates' keys sit in registers, SEL_KPT consecutive positions per
// thread (tiles of SEL_TILE positions are reloaded beyond that).  The k-th
// largest key (k = B - W - sink): a histogram of SEL_BINS bins linear in the
// score between the smallest and largest candidate (monotone in the key, so
// equal keys share a bin, and spread where the keys' top bits are not: the
// scores share sign and exponent), the bin holding the k-th key by one wave's
// suffix scan, that bin's keys compacted into LDS and the k-th found by rank
// counting.  A bin too full for that (ties, degenerate ranges) is resolved by
// 8-bit radix passes over the bits below its keys' common prefix.  Then the
// list in the reference's order: sinks, the keys above the k-th, the lowest
// positions holding the k-th key itself, the recent window -- written through
// block prefix sums of each thread's counts (thread order is position order).
constexpr int SEL_T = 1024, SEL_KPT = 32, SEL_TILE = SEL_T * SEL_KPT;
constexpr int SEL_BINS = 2048, SEL_CAP = 512;

// The k-th key among the candidates whose value bin is da (all candidates
// when !use_a) that lie in [kmin, kmax]: 8-bit radix passes over the bits
// below kmin ^ kmax's common prefix, keys read from memory each pass.  need:
// in, the rank among those candidates; out, the rank among the keys equal to
// tau.  Every thread of the block calls it.
__device__ __noinline__ void radix_select(const uint32_t *keys, int lo_pos, int hi_pos, bool use_a, float fmin,
                                          float scale, int da, uint32_t kmin, uint32_t kmax, int &need, uint32_t &tau,
                                          int *hist, int &s_digit, int &s_above) {
    const int tid = threadIdx.x, lane = tid & 63;
    auto in_a = [&](uint32_t k) {
        if (!use_a) return true;
        const int b = (int)((key_float(k) - fmin) * scale);
        return (b > SEL_BINS - 1 ? SEL_BINS - 1 : (b < 0 ? 0 : b)) == da;
    };
    const int hi = 32 - __builtin_clz(kmin ^ kmax);
    uint32_t prefix = hi >= 32 ? 0u : (kmin >> hi) << hi;
    for (int lo = hi; lo > 0;) {
        const int bits = lo >= 8 ? 8 : lo, shift = lo - bits;
        for (int i = tid; i < 256; i += blockDim.x) hist[i] = 0;
        __syncthreads();
        for (int p = lo_pos + tid; p < hi_pos; p += blockDim.x) {
            const uint32_t k = keys[p];
            if (in_a(k) && (lo >= 32 || (k >> lo) == (prefix >> lo))) atomicAdd(&hist[(k >> shift) & ((1u << bits) - 1u)], 1);
        }
        __syncthreads();
        if (tid < 64) {
            const int c[4] = {hist[4 * lane], hist[4 * lane + 1], hist[4 * lane + 2], hist[4 * lane + 3]};
            const int incl = wave_incl_scan(c[0] + c[1] + c[2] + c[3]);
            const int total = __shfl(incl, 63, 64);
            int acc = total - incl, found = -1, before = 0;
            #pragma unroll
            for (int b = 3; b >= 0; b--) {
                if (found < 0 && acc + c[b] >= need) { found = 4 * lane + b; before = acc; }
                if (found < 0) acc += c[b];
            }
            const unsigned long long bal = __ballot(found >= 0);
            const int L = 63 - __builtin_clzll(bal);
            const int d = __shfl(found, L, 64), aa = __shfl(before, L, 64);
            if (lane == 0) { s_digit = d; s_above = aa; }
        }
        __syncthreads();
        prefix |= (uint32_t)s_digit << shift;
        need -= s_above;
        lo = shift;
    }
    tau = prefix;
}
__global__ __launch_bounds__(SEL_T) void k_recall_select(RecallArgs rc) {
    const int pos = rc.st->pos, h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const SelGeom g = sel_geom(rc, pos);
    int *list = rc.lists + (size_t)h * rc.lstride;
    if (tid == 0) rc.counts[h] = g.m;
    if (rc.kvsel && h % (rc.NH / rc.NKV)) return;       // KVSEL: the group leader's list serves the group
    if (g.ident) {
        for (int s = tid; s <= pos; s += SEL_T) list[s] = s;
        return;
    }
    for (int s = tid; s < g.sink; s += SEL_T) list[s] = s;
    for (int s = g.cand_hi + tid; s <= pos; s += SEL_T) list[g.sink + g.topk + (s - g.cand_hi)] = s;
    if (g.topk == 0) return;
    const uint32_t *keys = rc.keys + (size_t)h * rc.kstride;
    __shared__ int hist[SEL_BINS];
    __shared__ uint32_t ckey[SEL_CAP];
    __shared__ uint32_t red_u[2 * (SEL_T / 64)];
    __shared__ int red_i[2 * (SEL_T / 64)];
    __shared__ int s_digit, s_above, s_count;
    __shared__ uint32_t s_tau;
    const int c0 = g.sink & ~3;                          // tiles start 16-byte aligned
    const int ntiles = (g.cand_hi - c0 + SEL_TILE - 1) / SEL_TILE;
    uint32_t kr[SEL_KPT];
    auto first = [&](int t) { return c0 + t * SEL_TILE + tid * SEL_KPT; };
    auto load_tile = [&](int t) {
        const int p0 = first(t);
        #pragma unroll
        for (int q = 0; q < SEL_KPT / 4; q++) {
            // p < cand_hi <= pmax <= kstride with p and kstride multiples of 4:
            // the 16-byte load stays inside the head's keys
            const int p = p0 + 4 * q;
            const uint4 v = p < g.cand_hi ? *(const uint4 *)(keys + p) : make_uint4(0u, 0u, 0u, 0u);
            kr[4 * q] = v.x; kr[4 * q + 1] = v.y; kr[4 * q + 2] = v.z; kr[4 * q + 3] = v.w;
        }
    };
    // valid positions of thread's tile t: [lo_j, hi_j) of its SEL_KPT slots
    auto slots = [&](int t, int &jlo, int &jhi) {
        const int p0 = first(t);
        jlo = g.sink - p0; jlo = jlo < 0 ? 0 : (jlo > SEL_KPT ? SEL_KPT : jlo);
        jhi = g.cand_hi - p0; jhi = jhi < 0 ? 0 : (jhi > SEL_KPT ? SEL_KPT : jhi);
    };
    // f(key) on every valid candidate (reloading tiles when there are several)
    auto each = [&](auto f) {
        for (int t = 0; t < ntiles; t++) {
            if (ntiles > 1) load_tile(t);
            int jlo, jhi;
            slots(t, jlo, jhi);
            #pragma unroll
            for (int j = 0; j < SEL_KPT; j++)
                if (j >= jlo && j < jhi) f(kr[j]);
        }
    };
    if (ntiles == 1) load_tile(0);
    // the smallest and largest key among the candidates that pred accepts
    auto block_minmax = [&](auto pred, uint32_t &mn, uint32_t &mx) {
        mn = 0xFFFFFFFFu; mx = 0u;
        each([&](uint32_t k) { if (pred(k)) { mn = k < mn ? k : mn; mx = k > mx ? k : mx; } });
        #pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const uint32_t a = (uint32_t)__shfl_xor((int)mn, o, 64), b = (uint32_t)__shfl_xor((int)mx, o, 64);
            mn = a < mn ? a : mn; mx = b > mx ? b : mx;
        }
        __syncthreads();                                 // red_u of an earlier reduction is consumed
        if (lane == 0) { red_u[wv] = mn; red_u[SEL_T / 64 + wv] = mx; }
        __syncthreads();
        mn = red_u[0]; mx = red_u[SEL_T / 64];
        for (int w = 1; w < SEL_T / 64; w++) {
            mn = red_u[w] < mn ? red_u[w] : mn;
            mx = red_u[SEL_T / 64 + w] > mx ? red_u[SEL_T / 64 + w] : mx;
        }
    };
    // histogram of digit(k) (nbins, a multiple of 64) over the accepted
    // candidates, then the digit holding the need-th largest key and the count
    // of keys in higher digits: lane l of wave 0 sums bins [l*per, (l+1)*per),
    // a suffix scan over the lanes finds the lane (every lane at or below the
    // right one reaches need; the highest is it), which walks its bins down
    auto select_digit = [&](int nbins, auto digit, auto pred, int need_, int &d, int &above) {
        for (int i = tid; i < nbins; i += SEL_T) hist[i] = 0;
        __syncthreads();
        each([&](uint32_t k) { if (pred(k)) atomicAdd(&hist[digit(k)], 1); });
        __syncthreads();
        if (tid < 64) {
            const int per = nbins / 64;
            int sl = 0;
            for (int b = 0; b < per; b++) sl += hist[lane * per + b];
            const int incl = wave_incl_scan(sl);
            const int total = __shfl(incl, 63, 64);
            const int acc0 = total - incl;               // keys in the bins of higher lanes
            const unsigned long long bal = __ballot(acc0 + sl >= need_);
            const int L = 63 - __builtin_clzll(bal);
            if (lane == L) {
                int acc = acc0, b = per - 1;
                for (; b > 0; b--) { const int c = hist[lane * per + b]; if (acc + c >= need_) break; acc += c; }
                s_digit = lane * per + b; s_above = acc;
            }
        }
        __syncthreads();
        d = s_digit; above = s_above;
    };
    uint32_t kmin, kmax;
    block_minmax([](uint32_t) { return true; }, kmin, kmax);
    int need = g.topk;                                   // keys still to take among the accepted ones
    uint32_t tau = kmin;
    bool done = kmin == kmax;                            // one key value: every candidate ties
    const float fmin = key_float(kmin), fmax = key_float(kmax);
    const float scale = (float)SEL_BINS / (fmax - fmin);
    const bool use_a = !done && fmax > fmin && scale > 0.0f && scale < INFINITY;
    auto bin_a = [&](uint32_t k) {
        const float x = (key_float(k) - fmin) * scale;
        const int b = (int)x;
        return b > SEL_BINS - 1 ? SEL_BINS - 1 : (b < 0 ? 0 : b);
    };
    int da = 0;
    if (use_a) {
        int above;
        select_digit(SEL_BINS, bin_a, [](uint32_t) { return true; }, need, da, above);
        need -= above;
        // the chosen bin's keys into LDS
        if (tid == 0) s_count = 0;
        __syncthreads();
        each([&](uint32_t k) {
            if (bin_a(k) == da) { const int i = atomicAdd(&s_count, 1); if (i < SEL_CAP) ckey[i] = k; }
        });
        __syncthreads();
        const int cnt = s_count;
        if (cnt <= SEL_CAP) {
            // the key with (keys above it) < need <= (keys at or above it)
            for (int i = tid; i < cnt; i += SEL_T) {
                const uint32_t k = ckey[i];
                int gt = 0, ge = 0;
                for (int j = 0; j < cnt; j++) { const uint32_t x = ckey[j]; gt += x > k; ge += x >= k; }
                if (gt < need && ge >= need) { s_tau = k; s_above = gt; }   // every writer writes the same pair
            }
            __syncthreads();
            tau = s_tau; need -= s_above;
            done = true;
        } else {
            block_minmax([&](uint32_t k) { return bin_a(k) == da; }, kmin, kmax);
            tau = kmin;
            done = kmin == kmax;
        }
    }
    if (!done) {
        // too many keys in the chosen bin: radix passes over it (keys read
        // from memory: the rare path keeps its registers to itself)
        radix_select(keys, g.sink, g.cand_hi, use_a, fmin, scale, da, kmin, kmax, need, tau, hist, s_digit, s_above);
    }
    const int n_gt = g.topk - need;                      // keys strictly above tau
    int base_gt = 0, base_eq = 0;
    for (int t = 0; t < ntiles; t++) {
        if (ntiles > 1) load_tile(t);
        int jlo, jhi;
        slots(t, jlo, jhi);
        int cg = 0, ce = 0;
        #pragma unroll
        for (int j = 0; j < SEL_KPT; j++)
            if (j >= jlo && j < jhi) { cg += kr[j] > tau; ce += kr[j] == tau; }
        // block exclusive scan of (cg, ce)
        const int ig = wave_incl_scan(cg), ie = wave_incl_scan(ce);
        __syncthreads();                                 // red_i of the previous tile is consumed
        if (lane == 63) { red_i[wv] = ig; red_i[SEL_T / 64 + wv] = ie; }
        __syncthreads();
        int og = base_gt + ig - cg, oe = base_eq + ie - ce;
        for (int w = 0; w < SEL_T / 64; w++) {
            if (w < wv) { og += red_i[w]; oe += red_i[SEL_T / 64 + w]; }
            base_gt += red_i[w]; base_eq += red_i[SEL_T / 64 + w];
        }
        const int p0 = first(t);
        #pragma unroll
        for (int j = 0; j < SEL_KPT; j++) {
            if (j < jlo || j >= jhi) continue;
            if (kr[j] > tau) list[g.sink + og++] = p0 + j;
            else if (kr[j] == tau) { if (oe < need) list[g.sink + n_gt + oe] = p0 + j; oe++; }
        }
    }
}

// the row of rc.lists that q head h attends over (KVSEL: its group leader's)
__device__ __forceinline__ int list_row(const RecallArgs &rc, int h) {
    return rc.kvsel ? h - h % (rc.NH / rc.NKV) : h;
}

// ---- attention pass 1: scores of a chunk of the list + the chunk maximum
// (grid: mchunks x NH).  Row-quad layout: a wave scores 16 list entries at a
// time, lane = 4 * entry + quarter, a quarter reads 16 B at byte 64 i + 16
// quarter of its K row and the dot product needs a 4-lane reduction.
template <int EPL, bool EXACT_MODE>
__global__ __launch_bounds__(256) void k_recall_scores(RecallArgs rc) {
    constexpr int HD = EPL * 64;
    const int h = blockIdx.y, c = blockIdx.x, kvh = h / (rc.NH / rc.NKV);
    const int m = rc.counts[h];
    const int j0 = c * RECALL_CHUNK;
    if (j0 >= m) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), e = lane >> 2, k4 = lane & 3;
    __shared__ int4 qi[EPL * 16];
    __shared__ float4 qf[EPL * 16];
    __shared__ int wmi[4];
    __shared__ float wmf[4];
    for (int i = threadIdx.x; i < HD / 4; i += 256) {
        const float *qp = rc.qr + (size_t)h * HD + 4 * i;
        if constexpr (EXACT_MODE)
            qi[i] = make_int4((int)rintf(qp[0] * 65536.0f), (int)rintf(qp[1] * 65536.0f),
                              (int)rintf(qp[2] * 65536.0f), (int)rintf(qp[3] * 65536.0f));
        else qf[i] = make_float4(qp[0], qp[1], qp[2], qp[3]);
    }
    __syncthreads();
    const int j = j0 + wave * 16 + e;                    // this quad's list entry
    const bool live = j < m;
    int64_t ai = 0;
    float af = 0.0f;
    if (live) {
        const int s = rc.lists[(size_t)list_row(rc, h) * rc.lstride + j];
        const int32_t *row = rc_row(rc, kvh, s, 0) + 4 * k4;
        #pragma unroll
        for (int i = 0; i < 4 * EPL; i++) {
            const int4 kv = *gmem((const int4 *)(row + 16 * i));
            if constexpr (EXACT_MODE) {
                const int4 q = qi[4 * i + k4];
                ai += (int64_t)q.x * kv.x + (int64_t)q.y * kv.y + (int64_t)q.z * kv.z + (int64_t)q.w * kv.w;
            } else {
                const float4 q = qf[4 * i + k4];
                af += q.x * __int_as_float(kv.x) + q.y * __int_as_float(kv.y) + q.z * __int_as_float(kv.z) +
                      q.w * __int_as_float(kv.w);
            }
        }
    }
    if constexpr (EXACT_MODE) {
        ai = quad_sum(ai);
        int z = INT32_MIN;
        if (live) {
            const float scv = (float)((double)ai / 4294967296.0) * rc.ascale;
            z = (int32_t)llround_pow2<14>(scv);
            if (k4 == 0) rc.zs[(size_t)h * rc.lstride + j] = z;
        }
        z = wave_allmax_i(z);
        if (lane == 0) wmi[wave] = z;
        __syncthreads();
        if (threadIdx.x == 0) {
            int t = wmi[0];
            for (int w = 1; w < 4; w++) t = wmi[w] > t ? wmi[w] : t;
            rc.cmax[(size_t)h * rc.mchunks + c] = t;
        }
    } else {
        af = quad_sum(af);
        float sv = -INFINITY;
        if (live) {
            sv = af * rc.ascale;
            if (k4 == 0) rc.zs[(size_t)h * rc.lstride + j] = __float_as_int(sv);
        }
        sv = wave_allmax(sv);
        if (lane == 0) wmf[wave] = sv;
        __syncthreads();
        if (threadIdx.x == 0) {
            float t = wmf[0];
            for (int w = 1; w < 4; w++) t = fmaxf(t, wmf[w]);
            rc.cmax[(size_t)h * rc.mchunks + c] = __float_as_int(t);
        }
    }
}

// one V row of the list: lane holds elements lane*EPL .. +EPL-1
template <int EPL>
__device__ __forceinline__ void rc_vrow(const RecallArgs &rc, int kvh, int s, int lane, int32_t out[EPL]) {
    const int32_t *src = rc_row(rc, kvh, s, 1) + lane * EPL;
    if constexpr (EPL == 4) { const int4 t = *gmem((const int4 *)src); out[0] = t.x; out[1] = t.y; out[2] = t.z; out[3] = t.w; }
    else if constexpr (EPL == 2) { const int2 t = *gmem((const int2 *)src); out[0] = t.x; out[1] = t.y; }
    else out[0] = *gmem(src);
}

// ---- attention pass 2 (exact): island weights, exact V-sum (FP64 FMAs on
// integers below 2^53: weights <= 2^22, |vq| < 2^23, 16 rows per lane),
// order-free int64 totals; the head's last workgroup divides (RNE)
template <int EPL>
__global__ __launch_bounds__(256) void k_recall_vsum_exact(RecallArgs rc) {
    constexpr int HD = EPL * 64;
    const int h = blockIdx.y, c = blockIdx.x, kvh = h / (rc.NH / rc.NKV);
    const int m = rc.counts[h];
    const int nact = (m + RECALL_CHUNK - 1) / RECALL_CHUNK;
    if (c >= nact) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __shared__ int s_M;
    __shared__ int64_t ored[4][HD];
    __shared__ int64_t sred[4];
    __shared__ int is_last;
    __shared__ int64_t Sg;
    // Wave 0 requests the chunk maxima first; every wave then requests its 16
    // list entries (positions and scores, lanes 0..15) and all 16 rows.
    // Entries past the list are clamped to its last one and weighted 0, so
    // every load is issued and the waits for the maxima and the scores leave
    // the rows in flight.
    const int jw = c * RECALL_CHUNK + wave * 16;
    const int nw = m - jw < 0 ? 0 : (m - jw > 16 ? 16 : m - jw);
    int cm = INT32_MIN;
    if (wave == 0) {
        const int x = rc.cmax[(size_t)h * rc.mchunks + (lane < nact ? lane : nact - 1)];
        cm = lane < nact ? x : INT32_MIN;
    }
    const int jl = jw + lane < m ? jw + lane : m - 1;
    const int s_l = rc.lists[(size_t)list_row(rc, h) * rc.lstride + jl], z_l = rc.zs[(size_t)h * rc.lstride + jl];
    int32_t v[16][EPL];
    #pragma unroll
    for (int u = 0; u < 16; u++) rc_vrow<EPL>(rc, kvh, __builtin_amdgcn_readlane(s_l, u), lane, v[u]);
    if (wave == 0) {
        int t = cm;
        for (int k = 64 + lane; k < nact; k += 64) {
            const int x = rc.cmax[(size_t)h * rc.mchunks + k];
            t = x > t ? x : t;
        }
        t = wave_allmax_i(t);
        if (lane == 0) s_M = t;
    }
    __syncthreads();
    const int64_t M = s_M;
    const int64_t w_l = lane < nw ? exp_fixed((((int64_t)z_l - M) * ONE) >> 14) >> 8 : 0;     // Q22
    double o[EPL];
    #pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = 0.0;
    #pragma unroll
    for (int u = 0; u < 16; u++) {                  // entries past the list: weight 0, adds exactly nothing
        const double w = (double)__shfl(w_l, u, 64);
        #pragma unroll
        for (int e = 0; e < EPL; e++) o[e] = fma(w, (double)v[u][e], o[e]);
    }
    const int64_t S = wave_allsum(w_l);
    #pragma unroll
    for (int e = 0; e < EPL; e++) ored[wave][lane * EPL + e] = (int64_t)o[e];
    if (lane == 0) sred[wave] = S;
    __syncthreads();
    for (int d = threadIdx.x; d < HD; d += 256) {
        const int64_t t = ored[0][d] + ored[1][d] + ored[2][d] + ored[3][d];
        atomicAdd((unsigned long long *)&rc.vacc[(size_t)h * HD + d], (unsigned long long)t);
    }
    if (threadIdx.x == 0)
        atomicAdd((unsigned long long *)&rc.vs[h], (unsigned long long)(sred[0] + sred[1] + sred[2] + sred[3]));
    mem_complete();
    __syncthreads();
    if (threadIdx.x == 0) is_last = (arrive(&rc.counter[h]) == nact - 1);
    __syncthreads();
    if (!is_last) return;
    // the totals are read and cleared for the next launch in one atomic step
    if (threadIdx.x == 0)
        Sg = (int64_t)__hip_atomic_exchange((unsigned long long *)&rc.vs[h], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int64_t tot = 0;
    if ((int)threadIdx.x < HD)
        tot = (int64_t)__hip_atomic_exchange((unsigned long long *)&rc.vacc[(size_t)h * HD + threadIdx.x], 0ull,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    StatAcc sacc;
    if ((int)threadIdx.x < HD) {
        const float x = rne_div_to_float((i128)tot, Sg, 16);
        rc.ao[(size_t)h * HD + threadIdx.x] = x;
        sacc.add(x);
    }
    stat_flush_block(rc.stat_out, sacc);                    // max |ao| for the O GEMV
    if (threadIdx.x == 0) reset_counter(&rc.counter[h]);
}

// ---- attention pass 2 (float): expf weights against the head's maximum,
// chunk sums written per chunk; the head's last workgroup adds the chunks in
// order (deterministic) and divides
template <int EPL>
__global__ __launch_bounds__(256) void k_recall_vsum_float(RecallArgs rc) {
    constexpr int HD = EPL * 64;
    const int h = blockIdx.y, c = blockIdx.x, kvh = h / (rc.NH / rc.NKV);
    const int m = rc.counts[h];
    const int nact = (m + RECALL_CHUNK - 1) / RECALL_CHUNK;
    if (c >= nact) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __shared__ float s_M;
    __shared__ float ored[4][HD];
    __shared__ float sred[4];
    __shared__ int is_last;
    __shared__ float Sg;
    // loads ordered and clamped as in the exact pass; entries past the list
    // are skipped in the sums
    const int jw = c * RECALL_CHUNK + wave * 16;
    const int nw = m - jw < 0 ? 0 : (m - jw > 16 ? 16 : m - jw);
    float cm = -INFINITY;
    if (wave == 0) {
        const float x = __int_as_float(rc.cmax[(size_t)h * rc.mchunks + (lane < nact ? lane : nact - 1)]);
        cm = lane < nact ? x : -INFINITY;
    }
    const int jl = jw + lane < m ? jw + lane : m - 1;
    const int s_l = rc.lists[(size_t)list_row(rc, h) * rc.lstride + jl];
    const float z_l = __int_as_float(rc.zs[(size_t)h * rc.lstride + jl]);
    int32_t v[16][EPL];
    #pragma unroll
    for (int u = 0; u < 16; u++) rc_vrow<EPL>(rc, kvh, __builtin_amdgcn_readlane(s_l, u), lane, v[u]);
    if (wave == 0) {
        float t = cm;
        for (int k = 64 + lane; k < nact; k += 64) t = fmaxf(t, __int_as_float(rc.cmax[(size_t)h * rc.mchunks + k]));
        t = wave_allmax(t);
        if (lane == 0) s_M = t;
    }
    __syncthreads();
    const float w_l = lane < nw ? expf(z_l - s_M) : 0.0f;
    float o[EPL];
    #pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = 0.0f;
    #pragma unroll
    for (int u = 0; u < 16; u++) {
        if (u < nw) {
            const float w = __shfl(w_l, u, 64);
            #pragma unroll
            for (int e = 0; e < EPL; e++) o[e] += w * __int_as_float(v[u][e]);
        }
    }
    const float S = wave_allsum(w_l);
    #pragma unroll
    for (int e = 0; e < EPL; e++) ored[wave][lane * EPL + e] = o[e];
    if (lane == 0) sred[wave] = S;
    __syncthreads();
    float *part = rc.part + ((size_t)h * rc.mchunks + c) * HD;
    for (int d = threadIdx.x; d < HD; d += 256) st_agent(&part[d], ored[0][d] + ored[1][d] + ored[2][d] + ored[3][d]);
    if (threadIdx.x == 0) st_agent(&rc.psum[(size_t)h * rc.mchunks + c], sred[0] + sred[1] + sred[2] + sred[3]);
    mem_complete();
    __syncthreads();
    if (threadIdx.x == 0) is_last = (arrive(&rc.counter[h]) == nact - 1);
    __syncthreads();
    if (!is_last) return;
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int k = 0; k < nact; k++) t += ld_agent(&rc.psum[(size_t)h * rc.mchunks + k]);
        Sg = t;
    }
    float tot = 0.0f;
    if ((int)threadIdx.x < HD)
        for (int k = 0; k < nact; k++) tot += ld_agent(&rc.part[((size_t)h * rc.mchunks + k) * HD + threadIdx.x]);
    __syncthreads();
    StatAcc sacc;
    if ((int)threadIdx.x < HD) {
        const float x = tot / Sg;
        rc.ao[(size_t)h * HD + threadIdx.x] = x;
        sacc.add(x);
    }
    stat_flush_block(rc.stat_out, sacc);
    if (threadIdx.x == 0) reset_counter(&rc.counter[h]);
}

template <int EPL> void recall_attn(const RecallArgs &rc, hipStream_t s) {
    const dim3 grid(rc.mchunks, rc.NH);
    if (rc.mode == EXACT) {
        hipLaunchKernelGGL((k_recall_scores<EPL, true>), grid, dim3(256), 0, s, rc);
        hipLaunchKernelGGL(k_recall_vsum_exact<EPL>, grid, dim3(256), 0, s, rc);
    } else {
        hipLaunchKernelGGL((k_recall_scores<EPL, false>), grid, dim3(256), 0, s, rc);
        hipLaunchKernelGGL(k_recall_vsum_float<EPL>, grid, dim3(256), 0, s, rc);
    }
}

}  // namespace

void launch_recall_attention(const RecallArgs &rc, hipStream_t s) {
    // lstride must hold every list (mchunks chunks of RECALL_CHUNK entries
    // cover it) and the keys every candidate position (kstride >= pmax, a
    // multiple of 4 for the select's 16-byte loads)
    if (!rc.side || rc.r < 1 || rc.r > 64 || rc.NH < 1 || rc.NKV < 1 || rc.NH % rc.NKV || rc.NH / rc.NKV > RECALL_MAX_GROUP ||
        rc.mchunks < 1 || !rc.stat_out || !rc.pq || rc.mchunks * RECALL_CHUNK < rc.lstride || rc.score_blocks < 1 ||
        rc.kstride < 4 || rc.kstride % 4 || (rc.kvsel && (!rc.Rb || !rc.qr || rc.HD > 256)))
        return launch_fail("recall attention: arguments outside the kernels' limits");
    if (rc.HD != 64 && rc.HD != 128 && rc.HD != 256)
        return launch_fail("recall attention serves head_dim 64, 128 and 256");
    const dim3 sg(rc.score_blocks, rc.NKV);
    switch (rc.r) {
    case 8:  hipLaunchKernelGGL(k_recall_score<8>, sg, dim3(256), 0, s, rc); break;
    case 16: hipLaunchKernelGGL(k_recall_score<16>, sg, dim3(256), 0, s, rc); break;
    case 32: hipLaunchKernelGGL(k_recall_score<32>, sg, dim3(256), 0, s, rc); break;
    case 64: hipLaunchKernelGGL(k_recall_score<64>, sg, dim3(256), 0, s, rc); break;
    default: hipLaunchKernelGGL(k_recall_score<0>, sg, dim3(256), 0, s, rc); break;
    }
    hipLaunchKernelGGL(k_recall_select, dim3(rc.NH), dim3(SEL_T), 0, s, rc);
    switch (rc.HD) {
    case 64:  recall_attn<1>(rc, s); break;
    case 128: recall_attn<2>(rc, s); break;
    default:  recall_attn<4>(rc, s); break;
    }
}

}  // namespace kvd
