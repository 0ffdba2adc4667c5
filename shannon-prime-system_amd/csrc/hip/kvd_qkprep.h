// kvd_qkprep.h -- one attention head's input preparation by one wave: per-head
// RMSNorm, NEOX RoPE, and the K/V append into the paged store.
//
// Reference: core/session/sp_session.c:292-294 / :405-407 (sp_rmsnorm_head +
// sp_rope_neox, forward_kernels.c:24-41) and the KV store at :321-323 (K after
// norm and RoPE, V raw).
#pragma once
#include "kvd_internal.h"
#include "kvd_exact.h"
#include "kvd_vec.h"
#include "kvd_spinor.h"

namespace kvd {

// the fields of the attention arguments the head preparation reads
struct HeadPrep {
    const float *q, *k, *v, *q_norm, *k_norm, *rope_cs;
    float *qr;
    float *const *pages;
    int ring_pages, NH, NKV, HD, mode;
    int kvc;                  // KVC_SPINOR: K/V pass the Spinor-63 codec
    float eps;
    int *vclamp;              // exact mode: count of V heads stored with a clamped element
    const uint32_t *rec_R;    // recall sidecar projection sign bits [rec_r][HD/32]
    int rec_r;                // 0: no sidecar
    float *rec_side;          // the layer's sidecar array [pmax][NKV][rec_r]
    float *rec_pq;            // routed step: q heads' projections [NH][rec_r]
};
__device__ __forceinline__ HeadPrep head_prep_of(const AttnArgs &a) {
    HeadPrep p;
    p.q = a.q; p.k = a.k; p.v = a.v; p.q_norm = a.q_norm; p.k_norm = a.k_norm; p.rope_cs = a.rope_cs;
    p.qr = a.qr; p.pages = a.pages; p.ring_pages = a.ring_pages; p.NH = a.NH; p.NKV = a.NKV; p.HD = a.HD;
    p.mode = a.mode; p.kvc = a.kvc; p.eps = a.eps; p.vclamp = a.vclamp;
    p.rec_R = a.rec_R; p.rec_r = a.rec_r; p.rec_pq = a.rec_pq; p.rec_side = a.rec_side;
    return p;
}

__device__ __forceinline__ float *qk_page_of(float *const *pages, int ring, int pos) {
    const int lp = pos / PAGE;
    return gmem(pages)[ring ? lp % ring : lp];
}

// The global inputs of one head's preparation, loaded by head_load so that a
// caller can request them before a bulk (K/V) request: vector loads complete
// in order, so inputs requested after the bulk would wait for all of it.
struct HeadIn { float v[8], w[8], c[4], s[4]; };
template <bool COHERENT, int PER>
__device__ __forceinline__ void head_load(const HeadPrep &a, const float *src, const float *nw, int lane, HeadIn &in) {
    constexpr int HD = PER * 64, half = HD / 2, per = PER;
    #pragma unroll
    for (int j = 0; j < 8; j++)
        if (j < per) {
            in.v[j] = COHERENT ? ld_agent(&src[lane + 64 * j]) : src[lane + 64 * j];
            in.w[j] = nw[lane + 64 * j];
        }
    if (per >= 2) {
        #pragma unroll
        for (int j = 0; j < 4; j++) {
            if (j >= per / 2) break;
            in.c[j] = a.rope_cs[lane + 64 * j]; in.s[j] = a.rope_cs[half + lane + 64 * j];
        }
    } else {
        const int i = lane < 32 ? lane : lane - 32;
        in.c[0] = a.rope_cs[i]; in.s[0] = a.rope_cs[half + i];
    }
}

// One q or k head's per-head RMSNorm and NEOX RoPE from what head_load read:
// lane l gets elements l + 64 j in out[j].
template <int PER>
__device__ __forceinline__ void head_norm_rope_in(const HeadPrep &a, const HeadIn &in, int lane, float out[8]) {
    constexpr int HD = PER * 64, per = PER;
    float v[8];                                                 // HD <= 512
    #pragma unroll
    for (int j = 0; j < 8; j++) if (j < per) v[j] = in.v[j];
    // per-head RMSNorm
    if (a.mode == FLOAT) {
        double ss = 0.0;
        #pragma unroll
        for (int j = 0; j < 8; j++) if (j < per) ss += (double)v[j] * (double)v[j];
        ss = wave_allsum(ss);
        const float sc = 1.0f / sqrtf((float)(ss / HD) + a.eps);
        #pragma unroll
        for (int j = 0; j < 8; j++) if (j < per) v[j] = v[j] * sc * in.w[j];
    } else {
        int64_t ss = 0;
        #pragma unroll
        for (int j = 0; j < 8; j++) if (j < per) { const int64_t xi = llround_pow2<16>(v[j]); ss += xi * xi; }
        ss = wave_allsum(ss);
        if (ss == 0) {
            #pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 0.0f;
        } else {
            const int64_t inv = rms_inv_q72(HD, ss);
            #pragma unroll
            for (int j = 0; j < 8; j++) {
                if (j >= per) break;
                const int64_t xi = llround_pow2<16>(v[j]), wi = llround_pow2<16>(in.w[j]);
                v[j] = (float)((double)mul3_lo64(xi, inv, wi) / 4503599627370496.0);
            }
        }
    }
    // NEOX RoPE on pairs (i, i + half), cos/sin from this position's table.
    // HD >= 128: both halves of a pair sit in the same lane (j and j + per/2);
    // HD == 64: the partner is lane ^ 32.
    if (per >= 2) {
        #pragma unroll
        for (int j = 0; j < 4; j++) {
            if (j >= per / 2) break;
            const float x0 = v[j], x1 = v[j + per / 2], c = in.c[j], s = in.s[j];
            const float ac = x0 * c, bs = x1 * s, as = x0 * s, bc = x1 * c;
            out[j] = ac - bs;
            out[j + per / 2] = as + bc;
        }
    } else {
        const float other = __shfl_xor(v[0], 32, 64);
        const bool first = lane < 32;
        const float x0 = first ? v[0] : other, x1 = first ? other : v[0], c = in.c[0], s = in.s[0];
        const float ac = x0 * c, bs = x1 * s, as = x0 * s, bc = x1 * c;
        out[0] = first ? ac - bs : as + bc;
    }
}

// One q or k head's per-head RMSNorm and NEOX RoPE: src holds the head's HD
// projections, nw its norm weight; lane l gets elements l + 64 j in out[j].
// COHERENT selects agent-scope loads, for projections written by other
// workgroups of the same launch.
template <bool COHERENT, int PER>
__device__ __forceinline__ void head_norm_rope(const HeadPrep &a, const float *src, const float *nw, int lane, float out[8]) {
    HeadIn in;
    head_load<COHERENT, PER>(a, src, nw, lane, in);
    head_norm_rope_in<PER>(a, in, lane, out);
}

// The stored form of a K or V element: the float itself, or in exact mode
// K ki = rne(k * 2^16) and V vq = clamp(rne(v * 2^16), +-(2^23 - 1)) (the
// bound keeps every V-sum product below 2^45); `clamped` is set when the
// clamp changed the value (|v| >= 128 - 2^-17).
__device__ __forceinline__ int32_t kv_code_k(float k) { return (int32_t)rintf(k * 65536.0f); }
__device__ __forceinline__ int32_t kv_code_v(float v, bool &clamped) {
    const float r = rintf(v * 65536.0f);
    const float c = fminf(fmaxf(r, -8388607.0f), 8388607.0f);
    clamped |= c != r;
    return (int32_t)c;
}
// one count per V head (wave) that clamped an element: the caller's flag
__device__ __forceinline__ void count_v_clamp(int *counter, bool clamped) {
    if (counter && __any(clamped) && __lane_id() == __builtin_amdgcn_readfirstlane(__lane_id()))
        atomicAdd(counter, 1);
}

// A K or V head (lane l holds coordinates l + 64 j) through the Spinor-63
// codec: per chunk the wave-wide max |v|, the int8 codes and v' = code * mul.
// Float mode stores the row of codes and multipliers (row: the head's row of
// spn_row_bytes(HD) bytes); exact mode gets v' back in place, for the int32 grid.
template <int PER>
__device__ __forceinline__ void spinor_head(float x[8], int lane, bool store, uint8_t *row) {
    constexpr int HD = PER * 64, NB = spn_blocks(HD);
    float am[NB];
    #pragma unroll
    for (int b = 0; b < NB; b++) am[b] = 0.0f;
    #pragma unroll
    for (int j = 0; j < PER; j++) {
        const int b = spn_block_of(HD, lane + 64 * j);
        #pragma unroll
        for (int bb = 0; bb < NB; bb++) if (b == bb) am[bb] = fmaxf(am[bb], fabsf(x[j]));
    }
    float mul_mine = 0.0f;
    #pragma unroll
    for (int b = 0; b < NB; b++) {
        am[b] = spn_scale(wave_allmax(am[b]));
        if (lane == b) mul_mine = am[b] / 127.0f;
    }
    #pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = lane + 64 * j, b = spn_block_of(HD, e);
        float sc = am[0];
        #pragma unroll
        for (int bb = 1; bb < NB; bb++) if (b == bb) sc = am[bb];
        const int32_t c = spn_code(x[j], sc);
        if (store) row[e] = (uint8_t)(int8_t)c;
        else x[j] = (float)c * (sc / 127.0f);
    }
    if (store && lane < NB) ((float *)(row + HD))[lane] = mul_mine;
}

// The recall projection of one K head (the sidecar) or q head (the router's
// query), core/arm/arm.c:31-45: lane p < r gets
// sum_d R[p][d] * k[d] as a sequential float sum in d (R = +-1, so each
// product is +-k[d] exactly and only the additions round, as on the CPU).
// The wave holds k at lanes l + 64 j in out[j]; readlane broadcasts each
// element in turn.
template <int PER>
__device__ __forceinline__ void recall_sidecar(const uint32_t *Rb, int r, const float out[8], float *dst, int lane) {
    constexpr int NW = PER * 2;                    // sign words per row (HD / 32)
    const int p = lane < r ? lane : 0;
    uint32_t bits[NW];
    #pragma unroll
    for (int w = 0; w < NW; w++) bits[w] = Rb[(size_t)p * NW + w];
    float acc = 0.0f;
    #pragma unroll
    for (int w = 0; w < NW; w++) {
        const int src = __float_as_int(out[w >> 1]);
        for (int b = 0; b < 32; b++) {
            const float kd = __int_as_float(__builtin_amdgcn_readlane(src, (w & 1) * 32 + b));
            acc = __fadd_rn(acc, ((bits[w] >> b) & 1u) ? kd : -kd);
        }
    }
    if (lane < r) dst[lane] = acc;
}

// hb < NH: q head hb -> qr; hb < NH + NKV: k head -> page; else v head -> page.
// src: the head's HD projections; lane l holds elements l + 64 j.
template <bool COHERENT, int PER>
__device__ __forceinline__ void qk_prep_head_t(const HeadPrep a, int hb, int pos, int lane) {
    constexpr int HD = PER * 64, per = PER;
    const bool isq = hb < a.NH, isk = !isq && hb < a.NH + a.NKV;
    const int h = isq ? hb : (isk ? hb - a.NH : hb - a.NH - a.NKV);
    float *page = qk_page_of(a.pages, a.ring_pages, pos);
    const int slot = pos % PAGE;
    const float *src = isq ? a.q + (size_t)h * HD : (isk ? a.k : a.v) + (size_t)h * HD;
    if (!isq && !isk && a.kvc == KVC_SPINOR) {                  // V through the codec
        float x[8];
        #pragma unroll
        for (int j = 0; j < 8; j++) if (j < per) x[j] = COHERENT ? ld_agent(&src[lane + 64 * j]) : src[lane + 64 * j];
        if (a.mode == FLOAT) {
            constexpr int RB = spn_row_bytes(HD);
            spinor_head<PER>(x, lane, true, (uint8_t *)page + ((size_t)a.NKV * PAGE + (size_t)h * PAGE + slot) * RB);
        } else {
            spinor_head<PER>(x, lane, false, nullptr);
            int32_t *dst = (int32_t *)page + (size_t)a.NKV * PAGE * HD + ((size_t)h * PAGE + slot) * HD;
            bool cl = false;
            #pragma unroll
            for (int j = 0; j < 8; j++) if (j < per) dst[lane + 64 * j] = kv_code_v(x[j], cl);
            count_v_clamp(a.vclamp, cl);
        }
        return;
    }
    if (!isq && !isk) {                                         // V: raw (exact: Q16 grid, clamped)
        float *dst = page + (size_t)a.NKV * PAGE * HD + ((size_t)h * PAGE + slot) * HD;
        bool cl = false;
        #pragma unroll
        for (int j = 0; j < 8; j++) {
            if (j >= per) break;
            const float v = COHERENT ? ld_agent(&src[lane + 64 * j]) : src[lane + 64 * j];
            if (a.mode == FLOAT) dst[lane + 64 * j] = v;
            else ((int32_t *)dst)[lane + 64 * j] = kv_code_v(v, cl);
        }
        if (a.mode != FLOAT) count_v_clamp(a.vclamp, cl);
        return;
    }
    float out[8];
    head_norm_rope<COHERENT, PER>(a, src, isq ? a.q_norm : a.k_norm, lane, out);
    if (isq) {
        #pragma unroll
        for (int j = 0; j < 8; j++) if (j < per) a.qr[(size_t)h * HD + lane + 64 * j] = out[j];
        if (a.rec_pq)                                           // the router's query projection
            recall_sidecar<PER>(a.rec_R, a.rec_r, out, a.rec_pq + (size_t)h * a.rec_r, lane);
        return;
    }
    if (a.rec_r)                                                // sidecar from the K before any codec
        recall_sidecar<PER>(a.rec_R, a.rec_r, out, a.rec_side + ((size_t)pos * a.NKV + h) * a.rec_r, lane);
    if (a.kvc == KVC_SPINOR && a.mode == FLOAT) {
        constexpr int RB = spn_row_bytes(HD);
        spinor_head<PER>(out, lane, true, (uint8_t *)page + ((size_t)h * PAGE + slot) * RB);
    } else {
        if (a.kvc == KVC_SPINOR) spinor_head<PER>(out, lane, false, nullptr);
        float *dst = page + ((size_t)h * PAGE + slot) * HD;
        #pragma unroll
        for (int j = 0; j < 8; j++) {
            if (j >= per) break;
            if (a.mode == FLOAT) dst[lane + 64 * j] = out[j];
            else ((int32_t *)dst)[lane + 64 * j] = kv_code_k(out[j]);
        }
    }
}
// head_dim 64 / 128 / 256 / 512: register arrays with compile-time indices
template <bool COHERENT>
__device__ __forceinline__ void qk_prep_head(const HeadPrep a, int hb, int pos, int lane) {
    switch (a.HD) {
    case 64:  qk_prep_head_t<COHERENT, 1>(a, hb, pos, lane); break;
    case 128: qk_prep_head_t<COHERENT, 2>(a, hb, pos, lane); break;
    case 256: qk_prep_head_t<COHERENT, 4>(a, hb, pos, lane); break;
    default:  qk_prep_head_t<COHERENT, 8>(a, hb, pos, lane); break;
    }
}

}  // namespace kvd
