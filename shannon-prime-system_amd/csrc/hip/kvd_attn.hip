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
#include "kvd_exact.h"

namespace kvd {

// exact-mode RoPE tables (host-computed integer constants, see kvd_backend.hip)
__device__ int64_t g_atan_q60[64];
__device__ int64_t g_kinv_q62;

constexpr int64_t TWO_PI_Q60 = 7244019458077122842LL;     // round(2*pi * 2^60)
constexpr int64_t HALF_PI_Q60 = 1811004864519280711LL;    // round(pi/2 * 2^60)

__device__ void cordic_q62(int64_t th, int64_t &co, int64_t &si) {
    int quad = 0;
    while (th >= HALF_PI_Q60 && quad < 3) { th -= HALF_PI_Q60; quad++; }
    int64_t x = g_kinv_q62, y = 0, z = th;
    for (int i = 0; i < 62; i++) {
        const int64_t xs = x >> i, ys = y >> i;
        if (z >= 0) { x -= ys; y += xs; z -= g_atan_q60[i]; }
        else        { x += ys; y -= xs; z += g_atan_q60[i]; }
    }
    switch (quad) {
        case 0: co = x;  si = y;  break;
        case 1: co = -y; si = x;  break;
        case 2: co = -x; si = -y; break;
        default: co = y; si = -x; break;
    }
}

__device__ __forceinline__ float wsum(float v) {
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ double wsumd(double v) {
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ int64_t wsuml(int64_t v) {
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wmax(float v) {
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float *page_of(float *const *pages, int ring, int pos) {
    const int lp = pos / PAGE;
    return pages[ring ? lp % ring : lp];
}

// ------------------------------------------------------------------ qk_prep
// grid.x = NH (q heads) + NKV (k heads) + NKV (v heads); block = 64 threads
// (one wave), each lane owning HD/64 pairs-halves.  float/exact by a.mode.
__global__ __launch_bounds__(64) void k_qk_prep(AttnArgs a) {
    const int64_t *freq_q60 = a.freq_q60;
    const int HD = a.HD, half = HD / 2, lane = threadIdx.x;
    const int pos = a.st->pos;
    const int hb = blockIdx.x;
    const bool isq = hb < a.NH, isk = !isq && hb < a.NH + a.NKV;
    const int h = isq ? hb : (isk ? hb - a.NH : hb - a.NH - a.NKV);
    float *page = page_of(a.pages, a.ring_pages, pos);
    const int slot = pos % PAGE;
    if (!isq && !isk) {                                        // V: raw copy
        const float *src = a.v + (size_t)h * HD;
        float *dst = page + (size_t)a.NKV * PAGE * HD + ((size_t)h * PAGE + slot) * HD;
        for (int i = lane; i < HD; i += 64) {
            if (a.mode == FLOAT) dst[i] = src[i];
            else {
                float r = rintf(src[i] * 65536.0f);
                r = fminf(fmaxf(r, -8388607.0f), 8388607.0f);
                ((int32_t *)dst)[i] = (int32_t)r;
            }
        }
        return;
    }
    const float *src = isq ? a.q + (size_t)h * HD : a.k + (size_t)h * HD;
    const float *nw = isq ? a.q_norm : a.k_norm;
    float v[8];                                                // HD <= 512
    const int per = HD / 64;
    for (int j = 0; j < per; j++) v[j] = src[lane + 64 * j];
    // per-head RMSNorm
    if (a.mode == FLOAT) {
        double ss = 0.0;
        for (int j = 0; j < per; j++) ss += (double)v[j] * (double)v[j];
        ss = wsumd(ss);
        const float sc = 1.0f / sqrtf((float)(ss / HD) + a.eps);
        for (int j = 0; j < per; j++) v[j] = v[j] * sc * nw[lane + 64 * j];
    } else {
        int64_t ss = 0;
        for (int j = 0; j < per; j++) { int64_t xi = llround_d((double)v[j] * 65536.0); ss += xi * xi; }
        ss = wsuml(ss);
        if (ss == 0) { for (int j = 0; j < per; j++) v[j] = 0.0f; }
        else {
            const int64_t inv = (int64_t)isqrt_u64(udiv128_64((u128)HD << 72, (uint64_t)ss));
            for (int j = 0; j < per; j++) {
                int64_t xi = llround_d((double)v[j] * 65536.0), wi = llround_d((double)nw[lane + 64 * j] * 65536.0);
                v[j] = (float)((double)mul3_lo64(xi, inv, wi) / 4503599627370496.0);
            }
        }
    }
    // NEOX RoPE: pairs (i, i+half).  Lane owns columns lane+64j; the partner of a
    // column in the lower half lives in the same lane (half is a multiple of 64).
    __shared__ float rot[512];
    for (int j = 0; j < per; j++) rot[lane + 64 * j] = v[j];
    __syncthreads();
    for (int i = lane; i < half; i += 64) {
        const float x0 = rot[i], x1 = rot[i + half];
        float c, s;
        if (a.mode == FLOAT) {
            const float freq = powf(a.base, -2.0f * (float)i / (float)HD);
            const float theta = (float)pos * freq;
            c = cosf(theta); s = sinf(theta);
            rot[i] = x0 * c - x1 * s;
            rot[i + half] = x0 * s + x1 * c;
        } else {
            const i128 th = (i128)pos * freq_q60[i];
            const int64_t r = umod128_64(th, TWO_PI_Q60);
            int64_t co, si; cordic_q62(r, co, si);
            c = rne_i64_scaled(co, -62); s = rne_i64_scaled(si, -62);
            const float ac = x0 * c, bs = x1 * s, as = x0 * s, bc = x1 * c;
            rot[i] = ac - bs;
            rot[i + half] = as + bc;
        }
    }
    __syncthreads();
    if (isq) {
        for (int i = lane; i < HD; i += 64) a.qr[(size_t)h * HD + i] = rot[i];
    } else {
        float *dst = page + ((size_t)h * PAGE + slot) * HD;
        for (int i = lane; i < HD; i += 64) {
            if (a.mode == FLOAT) dst[i] = rot[i];
            else ((int32_t *)dst)[i] = (int32_t)rintf(rot[i] * 65536.0f);
        }
    }
}

void launch_qk_prep(const AttnArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(k_qk_prep, dim3(a.NH + 2 * a.NKV), dim3(64), 0, s, a);
}
void set_rope_tables(const int64_t atan_q60[64], int64_t kinv_q62) {
    hipMemcpyToSymbol(HIP_SYMBOL(g_atan_q60), atan_q60, 64 * sizeof(int64_t));
    hipMemcpyToSymbol(HIP_SYMBOL(g_kinv_q62), &kinv_q62, sizeof(int64_t));
}

// ------------------------------------------------------------------ attention
// chunk geometry for the current position
__device__ __forceinline__ void chunk_range(const AttnArgs &a, int pos, int c, int &cs, int &ce, int &nch) {
    const int s0 = (a.win >= 0 && pos - a.win + 1 > 0) ? pos - a.win + 1 : 0;
    const int c0 = s0 / a.chunk;
    nch = pos / a.chunk - c0 + 1;
    cs = (c0 + c) * a.chunk; ce = cs + a.chunk;
    if (cs < s0) cs = s0;
    if (ce > pos + 1) ce = pos + 1;
}

template <int EPL, int G>
__global__ __launch_bounds__(256) void k_attn_float(AttnArgs a) {
    const int HD = EPL * 64, c = blockIdx.x, h = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int pos = a.st->pos;
    int cs, ce, nch;
    chunk_range(a, pos, c, cs, ce, nch);
    if (c >= nch) return;
    __shared__ float sc[G][PAGE];
    __shared__ float ored[4][G][EPL * 64];
    __shared__ int is_last;

    float q[G][EPL];
    #pragma unroll
    for (int g = 0; g < G; g++)
        #pragma unroll
        for (int e = 0; e < EPL; e++) q[g][e] = a.qr[(size_t)(h * G + g) * HD + lane * EPL + e];

    const float *page = page_of(a.pages, a.ring_pages, cs);
    const float *K = page + (size_t)h * PAGE * HD;
    const float *V = page + (size_t)a.NKV * PAGE * HD + (size_t)h * PAGE * HD;
    const int n = ce - cs;
    for (int j = wave; j < n; j += 4) {
        const int slot = (cs + j) % PAGE;
        float kv[EPL];
        if constexpr (EPL == 4) { float4 t = *(const float4 *)(K + (size_t)slot * HD + lane * 4); kv[0] = t.x; kv[1] = t.y; kv[2] = t.z; kv[3] = t.w; }
        else if constexpr (EPL == 2) { float2 t = *(const float2 *)(K + (size_t)slot * HD + lane * 2); kv[0] = t.x; kv[1] = t.y; }
        else { for (int e = 0; e < EPL; e++) kv[e] = K[(size_t)slot * HD + lane * EPL + e]; }
        #pragma unroll
        for (int g = 0; g < G; g++) {
            float d = 0.0f;
            #pragma unroll
            for (int e = 0; e < EPL; e++) d += q[g][e] * kv[e];
            d = wsum(d);
            if (lane == 0) sc[g][j] = d * a.ascale;
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
    #pragma unroll
    for (int g = 0; g < G; g++) {
        float lv = 0.0f;
        for (int j = lane; j < n; j += 64) { const float p = expf(sc[g][j] - m[g]); lv += p; }
        l[g] = wsum(lv);
    }
    // V-sum with p = exp(s - m) recomputed per position
    float o[G][EPL];
    #pragma unroll
    for (int g = 0; g < G; g++)
        #pragma unroll
        for (int e = 0; e < EPL; e++) o[g][e] = 0.0f;
    for (int j = wave; j < n; j += 4) {
        const int slot = (cs + j) % PAGE;
        float vv[EPL];
        if constexpr (EPL == 4) { float4 t = *(const float4 *)(V + (size_t)slot * HD + lane * 4); vv[0] = t.x; vv[1] = t.y; vv[2] = t.z; vv[3] = t.w; }
        else if constexpr (EPL == 2) { float2 t = *(const float2 *)(V + (size_t)slot * HD + lane * 2); vv[0] = t.x; vv[1] = t.y; }
        else { for (int e = 0; e < EPL; e++) vv[e] = V[(size_t)slot * HD + lane * EPL + e]; }
        #pragma unroll
        for (int g = 0; g < G; g++) {
            const float p = expf(sc[g][j] - m[g]);
            #pragma unroll
            for (int e = 0; e < EPL; e++) o[g][e] += p * vv[e];
        }
    }
    #pragma unroll
    for (int g = 0; g < G; g++)
        #pragma unroll
        for (int e = 0; e < EPL; e++) ored[wave][g][lane * EPL + e] = o[g][e];
    __syncthreads();
    for (int i = threadIdx.x; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        const float t = ored[0][g][d] + ored[1][g][d] + ored[2][g][d] + ored[3][g][d];
        a.part[((size_t)(h * G + g) * a.max_chunks + c) * HD + d] = t;
    }
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        a.part_ml[((size_t)(h * G + g) * a.max_chunks + c) * 2 + 0] = m[g];
        a.part_ml[((size_t)(h * G + g) * a.max_chunks + c) * 2 + 1] = l[g];
    }
    // ---- last arriving workgroup of this kv-head merges the chunks ----
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) is_last = (atomicAdd(&a.counter[h], 1) == nch - 1);
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int i = threadIdx.x; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        const size_t base = (size_t)(h * G + g) * a.max_chunks;
        // plain loads: the acquire fence above invalidated this CU's L1
        const float *pml = a.part_ml + base * 2, *po = a.part + base * HD + d;
        float M = -INFINITY;
        for (int k = 0; k < nch; k++) M = fmaxf(M, pml[k * 2]);
        float L = 0.0f, acc = 0.0f;
        for (int k = 0; k < nch; k++) {
            const float w = expf(pml[k * 2] - M);
            L += pml[k * 2 + 1] * w; acc += po[(size_t)k * HD] * w;
        }
        a.ao[(size_t)(h * G + g) * HD + d] = acc / L;
    }
    if (threadIdx.x == 0) a.counter[h] = 0;
}

// ---- exact mode: pass 1, integer scores on the softmax grid + chunk max ----
template <int EPL, int G>
__global__ __launch_bounds__(256) void k_attn_exact_scores(AttnArgs a) {
    const int HD = EPL * 64, c = blockIdx.x, h = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int pos = a.st->pos;
    int cs, ce, nch;
    chunk_range(a, pos, c, cs, ce, nch);
    if (c >= nch) return;
    __shared__ int zmax[4][G];
    int32_t qi[G][EPL];
    #pragma unroll
    for (int g = 0; g < G; g++)
        #pragma unroll
        for (int e = 0; e < EPL; e++) qi[g][e] = (int32_t)rintf(a.qr[(size_t)(h * G + g) * HD + lane * EPL + e] * 65536.0f);
    const int32_t *K = (const int32_t *)(page_of(a.pages, a.ring_pages, cs) + (size_t)h * PAGE * HD);
    int mx[G];
    #pragma unroll
    for (int g = 0; g < G; g++) mx[g] = INT32_MIN;
    const int n = ce - cs;
    for (int j = wave; j < n; j += 4) {
        const int slot = (cs + j) % PAGE;
        int32_t kv[EPL];
        #pragma unroll
        for (int e = 0; e < EPL; e++) kv[e] = K[(size_t)slot * HD + lane * EPL + e];
        #pragma unroll
        for (int g = 0; g < G; g++) {
            int64_t ip = 0;
            #pragma unroll
            for (int e = 0; e < EPL; e++) ip += (int64_t)qi[g][e] * kv[e];
            ip = wsuml(ip);
            const float sc = (float)((double)ip / 4294967296.0) * a.ascale;
            const int32_t z = (int32_t)llround_d((double)sc * 16384.0);
            if (lane == 0) a.zscratch[(size_t)(h * G + g) * a.max_chunks * a.chunk + (size_t)c * a.chunk + j] = z;
            mx[g] = z > mx[g] ? z : mx[g];
        }
    }
    if (lane == 0) for (int g = 0; g < G; g++) zmax[wave][g] = mx[g];
    __syncthreads();
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        int t = zmax[0][g];
        for (int w = 1; w < 4; w++) t = zmax[w][g] > t ? zmax[w][g] : t;
        ((int32_t *)a.part_ml)[((size_t)(h * G + g) * a.max_chunks + c) * 4] = t;
    }
}

// ---- exact mode: pass 2, exp weights on the island grid, exact V-sum ----
template <int EPL, int G>
__global__ __launch_bounds__(256) void k_attn_exact_vsum(AttnArgs a) {
    const int HD = EPL * 64, c = blockIdx.x, h = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int pos = a.st->pos;
    int cs, ce, nch;
    chunk_range(a, pos, c, cs, ce, nch);
    if (c >= nch) return;
    __shared__ int64_t ew[G][PAGE];
    __shared__ int64_t ored[4][G][EPL * 64];
    __shared__ int is_last;
    int32_t *pml = (int32_t *)a.part_ml;
    int M[G];
    #pragma unroll
    for (int g = 0; g < G; g++) {
        int t = INT32_MIN;
        for (int k = lane; k < nch; k += 64) {
            const int v = pml[((size_t)(h * G + g) * a.max_chunks + k) * 4];
            t = v > t ? v : t;
        }
        #pragma unroll
        for (int o = 32; o > 0; o >>= 1) { const int u = __shfl_xor(t, o, 64); t = u > t ? u : t; }
        M[g] = t;
    }
    const int n = ce - cs;
    for (int i = threadIdx.x; i < G * n; i += 256) {
        const int g = i / n, j = i % n;
        const int64_t z = a.zscratch[(size_t)(h * G + g) * a.max_chunks * a.chunk + (size_t)c * a.chunk + j];
        ew[g][j] = exp_fixed(((z - (int64_t)M[g]) * ONE) >> 14) >> 7;
    }
    __syncthreads();
    const int32_t *V = (const int32_t *)(page_of(a.pages, a.ring_pages, cs) + (size_t)a.NKV * PAGE * HD + (size_t)h * PAGE * HD);
    int64_t o[G][EPL];
    #pragma unroll
    for (int g = 0; g < G; g++)
        #pragma unroll
        for (int e = 0; e < EPL; e++) o[g][e] = 0;
    for (int j = wave; j < n; j += 4) {
        const int slot = (cs + j) % PAGE;
        int32_t vv[EPL];
        #pragma unroll
        for (int e = 0; e < EPL; e++) vv[e] = V[(size_t)slot * HD + lane * EPL + e];
        #pragma unroll
        for (int g = 0; g < G; g++)
            #pragma unroll
            for (int e = 0; e < EPL; e++) o[g][e] += ew[g][j] * (int64_t)vv[e];
    }
    #pragma unroll
    for (int g = 0; g < G; g++)
        #pragma unroll
        for (int e = 0; e < EPL; e++) ored[wave][g][lane * EPL + e] = o[g][e];
    __syncthreads();
    int64_t *part = (int64_t *)a.part;
    for (int i = threadIdx.x; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        part[((size_t)(h * G + g) * a.max_chunks + c) * HD + d] = ored[0][g][d] + ored[1][g][d] + ored[2][g][d] + ored[3][g][d];
    }
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        int64_t S = 0;
        for (int j = 0; j < n; j++) S += ew[g][j];
        *(int64_t *)&pml[((size_t)(h * G + g) * a.max_chunks + c) * 4 + 2] = S;
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) is_last = (atomicAdd(&a.counter[h], 1) == nch - 1);
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int i = threadIdx.x; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        const size_t base = (size_t)(h * G + g) * a.max_chunks;
        i128 acc = 0; int64_t S = 0;
        for (int k = 0; k < nch; k++) {          // plain loads after the acquire fence
            acc += (i128)part[(base + k) * HD + d];
            S += *(const int64_t *)&pml[(base + k) * 4 + 2];
        }
        a.ao[(size_t)(h * G + g) * HD + d] = rne_div_to_float(acc, S, 16);
    }
    if (threadIdx.x == 0) a.counter[h] = 0;
}

template <int EPL, int G> static void attn_dispatch(const AttnArgs &a, int grid_chunks, hipStream_t s) {
    dim3 grid(grid_chunks, a.NKV);
    if (a.mode == FLOAT) hipLaunchKernelGGL((k_attn_float<EPL, G>), grid, dim3(256), 0, s, a);
    else {
        hipLaunchKernelGGL((k_attn_exact_scores<EPL, G>), grid, dim3(256), 0, s, a);
        hipLaunchKernelGGL((k_attn_exact_vsum<EPL, G>), grid, dim3(256), 0, s, a);
    }
}

void launch_attention(const AttnArgs &a, int grid_chunks, hipStream_t s) {
    const int G = a.NH / a.NKV;
    if (a.HD == 256 && G == 2) attn_dispatch<4, 2>(a, grid_chunks, s);
    else if (a.HD == 128 && G == 2) attn_dispatch<2, 2>(a, grid_chunks, s);
    else if (a.HD == 128 && G == 4) attn_dispatch<2, 4>(a, grid_chunks, s);
    else if (a.HD == 64 && G == 2) attn_dispatch<1, 2>(a, grid_chunks, s);
    else if (a.HD == 256 && G == 4) attn_dispatch<4, 4>(a, grid_chunks, s);
    else if (a.HD == 64 && G == 4) attn_dispatch<1, 4>(a, grid_chunks, s);
}

// ------------------------------------------------------------------ embedding
__global__ __launch_bounds__(256) void k_embed(DevW w, const DState *st, const int *tokbuf, float *x, float scale) {
    const int tok = st->drive == DRIVE_STREAM ? tokbuf[st->pos] : st->tok, E = w.cols;
    const uint8_t *rc = w.codes + (size_t)tok * ((E + 1) / 2);
    const uint16_t *bs = w.bs + (size_t)tok * w.nblk;
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
void launch_embed(const DevW &embd, const DState *st, const int *tokbuf, float *x, float scale, hipStream_t s) {
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, s, embd, st, tokbuf, x, scale);
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
        pv[blockIdx.x] = v; pi[blockIdx.x] = idx;
        __threadfence();
        is_last = atomicAdd(counter, 1) == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (!is_last || threadIdx.x != 0) return;
    __threadfence();
    float bv = -INFINITY; int bi = 0x7FFFFFFF;
    for (int b = 0; b < (int)gridDim.x; b++) amax_merge(bv, bi, pv[b], pi[b]);
    if (bi == 0x7FFFFFFF) bi = 0;
    st->tok = bi;
    if (gen_log) gen_log[st->pos] = bi;
    if (st->drive == DRIVE_GREEDY) st->pos = st->pos + 1;
    *counter = 0;
}
int argmax_blocks(int V) { int b = (V + 2047) / 2048; return b < 1 ? 1 : (b > 256 ? 256 : b); }
void launch_argmax(const float *logits, int V, float *pval, int *pidx, int *counter, DState *st,
                   int *gen_log, int nblocks, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax, dim3(nblocks), dim3(256), 0, s, logits, V, pval, pidx, counter, st, gen_log);
}

}  // namespace kvd
