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

int recall_page_floats(int NKV, int r) { return NKV * PAGE * r; }

namespace {

__device__ __forceinline__ const float *rc_page(const RecallArgs &rc, int pos) { return rc.pages[pos / PAGE]; }
// row of position s of kv head kvh: K (vpart = 0) or V (vpart = 1)
__device__ __forceinline__ const int32_t *rc_row(const RecallArgs &rc, int kvh, int s, int vpart) {
    return (const int32_t *)rc_page(rc, s) + (size_t)vpart * rc.NKV * PAGE * rc.HD +
           ((size_t)kvh * PAGE + (s & (PAGE - 1))) * rc.HD;
}

// float -> unsigned key with the float order (larger float, larger key)
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
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

// ---- router 1: the candidates' projected scores (grid: score_blocks x NH)
__global__ __launch_bounds__(256) void k_recall_score(RecallArgs rc) {
    const int pos = rc.st->pos, h = blockIdx.y, kvh = h / (rc.NH / rc.NKV);
    const SelGeom g = sel_geom(rc, pos);
    if (g.ident || g.topk == 0) return;
    __shared__ float qs[256];
    __shared__ float pq[64];
    const int HD = rc.HD, r = rc.r, NW = HD / 32;
    for (int i = threadIdx.x; i < HD; i += 256) qs[i] = rc.qr[(size_t)h * HD + i];
    __syncthreads();
    if ((int)threadIdx.x < r) {                         // the query's projection, sequential in d
        const uint32_t *bits = rc.Rb + (size_t)threadIdx.x * NW;
        float a = 0.0f;
        for (int w = 0; w < NW; w++) {
            const uint32_t bw = bits[w];
            for (int b = 0; b < 32; b++) {
                const float x = qs[32 * w + b];
                a = __fadd_rn(a, ((bw >> b) & 1u) ? x : -x);
            }
        }
        pq[threadIdx.x] = a;
    }
    __syncthreads();
    uint32_t *keys = rc.keys + (size_t)h * rc.kstride;
    for (int s = g.sink + blockIdx.x * 256 + threadIdx.x; s < g.cand_hi; s += gridDim.x * 256) {
        const float *side = rc_page(rc, s) + (size_t)2 * rc.NKV * PAGE * HD + ((size_t)kvh * PAGE + (s & (PAGE - 1))) * r;
        float a = 0.0f;
        for (int p = 0; p < r; p++) a = __fadd_rn(a, __fmul_rn(pq[p], side[p]));
        keys[s] = order_key(a);
    }
}

// ---- router 2: one q head's recall set (grid: NH, 1024 threads)
// The topk-th largest key by a 4 x 8-bit radix select, then the list in the
// reference's order: sinks, the selected candidates (keys above the k-th, then
// the lowest positions holding the k-th key itself), the recent window.
constexpr int SEL_T = 1024;
__global__ __launch_bounds__(SEL_T) void k_recall_select(RecallArgs rc) {
    const int pos = rc.st->pos, h = blockIdx.x, tid = threadIdx.x;
    const SelGeom g = sel_geom(rc, pos);
    int *list = rc.lists + (size_t)h * rc.lstride;
    if (tid == 0) rc.counts[h] = g.m;
    if (g.ident) {
        for (int s = tid; s <= pos; s += SEL_T) list[s] = s;
        return;
    }
    const uint32_t *keys = rc.keys + (size_t)h * rc.kstride;
    __shared__ int hist[256];
    __shared__ uint32_t s_prefix;
    __shared__ int s_need;
    __shared__ int wsum[2 * (SEL_T / 64)];
    __shared__ int s_base[2];
    uint32_t prefix = 0;
    int need = g.topk;                                   // keys still to take at the prefix
    if (need > 0) {
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int i = tid; i < 256; i += SEL_T) hist[i] = 0;
            __syncthreads();
            const uint32_t mask = shift == 24 ? 0u : (0xFFFFFFFFu << (shift + 8));
            for (int s = g.sink + tid; s < g.cand_hi; s += SEL_T) {
                const uint32_t k = keys[s];
                if ((k & mask) == (prefix & mask)) atomicAdd(&hist[(k >> shift) & 255], 1);
            }
            __syncthreads();
            if (tid == 0) {                               // the digit holding the need-th largest key
                int acc = 0, d = 255;
                for (; d > 0; d--) { if (acc + hist[d] >= need) break; acc += hist[d]; }
                s_prefix = (prefix & mask) | ((uint32_t)d << shift);
                s_need = need - acc;
            }
            __syncthreads();
            prefix = s_prefix; need = s_need;
        }
    }
    const uint32_t tau = prefix;
    const int n_gt = g.topk - need;                      // keys strictly above tau
    for (int s = tid; s < g.sink; s += SEL_T) list[s] = s;
    for (int s = g.cand_hi + tid; s <= pos; s += SEL_T) list[g.sink + g.topk + (s - g.cand_hi)] = s;
    if (tid == 0) { s_base[0] = 0; s_base[1] = 0; }
    __syncthreads();
    if (g.topk == 0) return;
    const int lane = tid & 63, wv = tid >> 6, NWV = SEL_T / 64;
    const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int base = g.sink; base < g.cand_hi; base += SEL_T) {
        const int s = base + tid;
        const uint32_t k = s < g.cand_hi ? keys[s] : 0u;
        const bool gt = s < g.cand_hi && k > tau, eq = s < g.cand_hi && k == tau;
        const unsigned long long bg = __ballot(gt), be = __ballot(eq);
        if (lane == 0) { wsum[wv] = __popcll(bg); wsum[NWV + wv] = __popcll(be); }
        __syncthreads();
        int og = s_base[0], oe = s_base[1], tg = 0, te = 0;
        for (int w = 0; w < NWV; w++) {
            if (w < wv) { og += wsum[w]; oe += wsum[NWV + w]; }
            tg += wsum[w]; te += wsum[NWV + w];
        }
        og += __popcll(bg & below); oe += __popcll(be & below);
        if (gt) list[g.sink + og] = s;
        if (eq && oe < need) list[g.sink + n_gt + oe] = s;
        __syncthreads();
        if (tid == 0) { s_base[0] += tg; s_base[1] += te; }
        __syncthreads();
    }
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
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, e = lane >> 2, k4 = lane & 3;
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
        const int s = rc.lists[(size_t)h * rc.lstride + j];
        const int32_t *row = rc_row(rc, kvh, s, 0) + 4 * k4;
        #pragma unroll
        for (int i = 0; i < 4 * EPL; i++) {
            const int4 kv = *(const int4 *)(row + 16 * i);
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
    if constexpr (EPL == 4) { const int4 t = *(const int4 *)src; out[0] = t.x; out[1] = t.y; out[2] = t.z; out[3] = t.w; }
    else if constexpr (EPL == 2) { const int2 t = *(const int2 *)src; out[0] = t.x; out[1] = t.y; }
    else out[0] = src[0];
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
    const int j0 = c * RECALL_CHUNK, j1 = j0 + RECALL_CHUNK < m ? j0 + RECALL_CHUNK : m;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __shared__ int s_M;
    __shared__ int64_t ored[4][HD];
    __shared__ int64_t sred[4];
    __shared__ int is_last;
    __shared__ int64_t Sg;
    if (threadIdx.x < 64) {
        int t = INT32_MIN;
        for (int k = threadIdx.x; k < nact; k += 64) {
            const int v = rc.cmax[(size_t)h * rc.mchunks + k];
            t = v > t ? v : t;
        }
        t = wave_allmax_i(t);
        if (threadIdx.x == 0) s_M = t;
    }
    __syncthreads();
    const int64_t M = s_M;
    const int *list = rc.lists + (size_t)h * rc.lstride;
    const int *zs = rc.zs + (size_t)h * rc.lstride;
    double o[EPL];
    #pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = 0.0;
    int64_t S = 0;
    for (int j = j0 + wave; j < j1; j += 4) {
        const int s = list[j];
        const int64_t w = exp_fixed((((int64_t)zs[j] - M) * ONE) >> 14) >> 8;      // Q22
        S += w;
        int32_t v[EPL];
        rc_vrow<EPL>(rc, kvh, s, lane, v);
        #pragma unroll
        for (int e = 0; e < EPL; e++) o[e] = fma((double)w, (double)v[e], o[e]);
    }
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
        const float v = rne_div_to_float((i128)tot, Sg, 16);
        rc.ao[(size_t)h * HD + threadIdx.x] = v;
        sacc.add(v);
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
    const int j0 = c * RECALL_CHUNK, j1 = j0 + RECALL_CHUNK < m ? j0 + RECALL_CHUNK : m;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __shared__ float s_M;
    __shared__ float ored[4][HD];
    __shared__ float sred[4];
    __shared__ int is_last;
    __shared__ float Sg;
    if (threadIdx.x < 64) {
        float t = -INFINITY;
        for (int k = threadIdx.x; k < nact; k += 64) t = fmaxf(t, __int_as_float(rc.cmax[(size_t)h * rc.mchunks + k]));
        t = wave_allmax(t);
        if (threadIdx.x == 0) s_M = t;
    }
    __syncthreads();
    const float M = s_M;
    const int *list = rc.lists + (size_t)h * rc.lstride;
    const int *zs = rc.zs + (size_t)h * rc.lstride;
    float o[EPL];
    #pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = 0.0f;
    float S = 0.0f;
    for (int j = j0 + wave; j < j1; j += 4) {
        const int s = list[j];
        const float w = expf(__int_as_float(zs[j]) - M);
        S += w;
        int32_t v[EPL];
        rc_vrow<EPL>(rc, kvh, s, lane, v);
        #pragma unroll
        for (int e = 0; e < EPL; e++) o[e] += w * __int_as_float(v[e]);
    }
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
        const float v = tot / Sg;
        rc.ao[(size_t)h * HD + threadIdx.x] = v;
        sacc.add(v);
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
    // cover it) and the keys every candidate position (kstride >= pmax)
    if (rc.r < 1 || rc.r > 64 || rc.NH < 1 || rc.NKV < 1 || rc.NH % rc.NKV || rc.mchunks < 1 || !rc.stat_out ||
        rc.mchunks * RECALL_CHUNK < rc.lstride || rc.score_blocks < 1 || rc.kstride < 1)
        return launch_fail("recall attention: arguments outside the kernels' limits");
    if (rc.HD != 64 && rc.HD != 128 && rc.HD != 256)
        return launch_fail("recall attention serves head_dim 64, 128 and 256");
    hipLaunchKernelGGL(k_recall_score, dim3(rc.score_blocks, rc.NH), dim3(256), 0, s, rc);
    hipLaunchKernelGGL(k_recall_select, dim3(rc.NH), dim3(SEL_T), 0, s, rc);
    switch (rc.HD) {
    case 64:  recall_attn<1>(rc, s); break;
    case 128: recall_attn<2>(rc, s); break;
    default:  recall_attn<4>(rc, s); break;
    }
}

}  // namespace kvd
