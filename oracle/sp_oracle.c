/* sp_oracle.c -- TEST INFRASTRUCTURE ONLY (the checker; see sp_oracle.h).
 *
 * Float mode is a line-by-line restatement of the reference decode so that it is
 * bit-identical to it when compiled with the same flags (gcc -O2, SSE2, no FMA
 * contraction, glibc libm):
 *   orc_rmsnorm      <- core/forward_kernels/forward_kernels.c:17-22 (and :24-29)
 *   orc_rope_neox    <- core/forward_kernels/forward_kernels.c:31-41
 *   orc_attn_head    <- core/forward_kernels/forward_kernels.c:59-81
 *                       (Qwen3's inline copy, core/session/sp_session.c:327-347, is
 *                        the same arithmetic with win = -1)
 *   orc_q4b_gemv     <- core/forward_dispatch/forward_dispatch.c:69-85 (Q4B branch)
 *   embed row        <- core/frobenius/frobenius_lift.c:116-125
 *   f16 -> f32       <- core/weight_dtype/weight_dtype.c:9-28
 *   step_qwen3       <- core/session/sp_session.c:274-363 (kv_step)
 *   step_gemma3      <- core/session/sp_session.c:380-464 (kv_step_gemma3)
 *   rewind / clone   <- core/session/sp_session.c:773-824
 * Exact islands restate core/exact_islands/exact_islands.c:21-124.
 *
 * Exact mode (build-defined; the reference has no integer decode) replaces every
 * reduction and transcendental with integer arithmetic:
 *   RMSNorm        island (no eps), per vector and per Q/K head
 *   GEMV           activations to a per-vector power-of-two grid (max |xq| < 2^22,
 *                  round-half-even), int32 block dots, f16 scale = M*2^e applied
 *                  exactly into an int128 row accumulator, one RNE conversion
 *   RoPE           integer frequency table base^(-2i/d) in Q60, p*F mod 2*pi,
 *                  62-step CORDIC (Volder 1959) for cos/sin in Q62, RNE to float,
 *                  float rotation without contraction
 *   attention      qi = rne(q*2^16), ki = rne(k*2^16), exact int64 dot,
 *                  score = (float)((double)ip/2^32)*ascale (decode.c:141-152 form),
 *                  softmax island exp weights e (Q30), V-sum over e>>8 (Q22) and
 *                  vq = clamp(rne(v*2^16), +-(2^23-1)): every product < 2^45, so the
 *                  sum fits int64 for contexts below 2^18; one RNE division
 *   SwiGLU         silu via the island exp (sigmoid in Q30); GeGLU = GELU island
 * KV cache in exact mode holds ki and vq as int32 (same 4 bytes per element). */
#include "sp_oracle.h"
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

typedef __int128 i128;
typedef unsigned __int128 u128;

/* Threads for the row-parallel loops (GEMV rows, attention heads): each row or
 * head is computed exactly as in the scalar order, so results do not depend
 * on the count.  1 = the scalar oracle. */
static int g_threads = 1;
void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int orc_threads(void) { return g_threads; }

/* ======================= minimal .sp-model reader ======================= */
typedef struct { char name[80]; uint32_t dtype, n_dims; uint64_t dims[8]; uint64_t off, size;
                 uint32_t bs, bc; uint8_t dig[32]; uint64_t hash; uint8_t pad[40]; } orc_entry;

typedef struct { const uint8_t *codes; const uint16_t *bs; int rows, cols; } orc_w;

typedef struct {
    orc_w q, k, v, o, gate, up, down;
    const float *attn_norm, *q_norm, *k_norm, *ffn_norm, *post_attn, *post_ffw;
} orc_layer;

struct orc_model {
    uint8_t *map; size_t len;
    uint32_t arch, V, E, NL, NH, NKV, HD, FF, SW, max_ctx;
    float base, eps;
    orc_w embd, out;
    const float *out_norm;
    orc_layer *L;
};

static const orc_entry *find_entry(const uint8_t *map, const char *name) {
    uint32_t n; memcpy(&n, map + 316, 4);
    for (uint32_t i = 0; i < n; i++) {
        const orc_entry *e = (const orc_entry *)(map + 512 + (size_t)i * 256);
        if (strncmp(e->name, name, 80) == 0) return e;
    }
    return NULL;
}
static const void *entry_data(const orc_model *m, const orc_entry *e) {
    uint64_t doff; memcpy(&doff, m->map + 328, 8);
    return m->map + doff + e->off;
}
static int get_w(orc_model *m, const char *name, orc_w *w) {
    const orc_entry *e = find_entry(m->map, name);
    if (!e || e->dtype != 13u) return 1;                 /* OK_Q4B only */
    char sn[100]; snprintf(sn, sizeof sn, "%s.bscale", name);
    const orc_entry *s = find_entry(m->map, sn);
    if (!s || s->dtype != 14u) return 1;
    w->cols = (int)e->dims[0]; w->rows = (int)e->dims[1];
    w->codes = (const uint8_t *)entry_data(m, e); w->bs = (const uint16_t *)entry_data(m, s);
    return 0;
}
static const float *get_norm(orc_model *m, const char *name) {
    const orc_entry *e = find_entry(m->map, name);
    return (e && e->dtype == 1u) ? (const float *)entry_data(m, e) : NULL;
}

orc_model *orc_model_load(const char *path) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) return NULL;
    struct stat st; fstat(fd, &st);
    uint8_t *map = (uint8_t *)mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return NULL;
    orc_model *m = (orc_model *)calloc(1, sizeof *m);
    m->map = map; m->len = (size_t)st.st_size;
    const uint8_t *a = map + 24;                          /* arch_struct = sp_arch_info */
    uint32_t u[9]; memcpy(u, a, 36);
    m->arch = u[0]; m->V = u[1]; m->E = u[2]; m->NL = u[3]; m->NH = u[4]; m->NKV = u[5];
    m->HD = u[6]; m->max_ctx = u[7]; m->SW = u[8];
    memcpy(&m->base, a + 36, 4);
    memcpy(&m->FF, a + 44, 4); memcpy(&m->eps, a + 48, 4);
    if (m->eps == 0.0f) m->eps = 1e-6f;
    int bad = get_w(m, "token_embd.weight", &m->embd);
    if (find_entry(map, "output.weight")) bad |= get_w(m, "output.weight", &m->out);
    else m->out = m->embd;
    if (!m->FF) { const orc_entry *g = find_entry(map, "blk.0.ffn_gate.weight"); if (g) m->FF = (uint32_t)g->dims[1]; }
    m->out_norm = get_norm(m, "output_norm.weight");
    m->L = (orc_layer *)calloc(m->NL, sizeof(orc_layer));
    char nm[96];
    for (uint32_t l = 0; l < m->NL && !bad; l++) {
        orc_layer *y = &m->L[l];
#define W(f, s) do { snprintf(nm, sizeof nm, "blk.%u." s ".weight", l); bad |= get_w(m, nm, &y->f); } while (0)
#define N(f, s) do { snprintf(nm, sizeof nm, "blk.%u." s ".weight", l); y->f = get_norm(m, nm); } while (0)
        W(q, "attn_q"); W(k, "attn_k"); W(v, "attn_v"); W(o, "attn_output");
        W(gate, "ffn_gate"); W(up, "ffn_up"); W(down, "ffn_down");
        N(attn_norm, "attn_norm"); N(q_norm, "attn_q_norm"); N(k_norm, "attn_k_norm");
        N(ffn_norm, "ffn_norm"); N(post_attn, "post_attention_norm"); N(post_ffw, "post_ffw_norm");
#undef W
#undef N
    }
    if (bad || !m->out_norm) { orc_model_free(m); return NULL; }
    return m;
}
void orc_model_free(orc_model *m) {
    if (!m) return;
    munmap(m->map, m->len); free(m->L); free(m);
}
void orc_model_dims(const orc_model *m, uint32_t o[9]) {
    o[0] = m->arch; o[1] = m->V; o[2] = m->E; o[3] = m->NL; o[4] = m->NH; o[5] = m->NKV;
    o[6] = m->HD; o[7] = m->FF; o[8] = m->SW;
}

/* ======================= float-mode kernels ======================= */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, f;
    if (exp == 0) {
        if (man == 0) f = sign;
        else {
            exp = 127u - 15u + 1u;
            while ((man & 0x400u) == 0) { man <<= 1; exp--; }
            man &= 0x3FFu;
            f = sign | (exp << 23) | (man << 13);
        }
    } else if (exp == 0x1Fu) f = sign | 0x7F800000u | (man << 13);
    else f = sign | ((exp - 15u + 127u) << 23) | (man << 13);
    float o; memcpy(&o, &f, 4); return o;
}

void orc_rmsnorm(const float *x, const float *w, int n, float eps, float *out) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    float scale = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}
static void rmsnorm_head(float *v, const float *w, int d, float eps) {
    double ss = 0.0;
    for (int i = 0; i < d; i++) ss += (double)v[i] * v[i];
    float scale = 1.0f / sqrtf((float)(ss / d) + eps);
    for (int i = 0; i < d; i++) v[i] = v[i] * scale * w[i];
}

void orc_rope_neox(float *v, int d, int p, float base) {
    int half = d / 2;
    for (int i = 0; i < half; i++) {
        float freq = powf(base, -2.0f * (float)i / (float)d);
        float theta = (float)p * freq;
        float c = cosf(theta), s = sinf(theta);
        float a = v[i], b = v[i + half];
        v[i] = a * c - b * s;
        v[i + half] = a * s + b * c;
    }
}

void orc_attn_head(const float *qh, const float *KC, const float *VC, int pos, int KVD,
                   int kvh, int HD, float ascale, int win, float *sc, float *out) {
    int s0 = (win >= 0 && pos - win + 1 > 0) ? pos - win + 1 : 0;
    float maxs = -INFINITY;
    for (int s = s0; s <= pos; s++) {
        const float *kh = KC + (size_t)s * KVD + (size_t)kvh * HD;
        float acc = 0.0f;
        for (int i = 0; i < HD; i++) acc += qh[i] * kh[i];
        float d = acc * ascale;
        sc[s] = d;
        if (d > maxs) maxs = d;
    }
    float sum = 0.0f;
    for (int s = s0; s <= pos; s++) { sc[s] = expf(sc[s] - maxs); sum += sc[s]; }
    float inv = 1.0f / sum;
    for (int i = 0; i < HD; i++) out[i] = 0.0f;
    for (int s = s0; s <= pos; s++) {
        float w = sc[s] * inv;
        const float *vh = VC + (size_t)s * KVD + (size_t)kvh * HD;
        for (int i = 0; i < HD; i++) out[i] += w * vh[i];
    }
}

static inline int nib(const uint8_t *row, int i) {
    uint8_t b = (i & 1) ? (uint8_t)(row[i >> 1] >> 4) : (uint8_t)(row[i >> 1] & 0xF);
    return (b & 8) ? (int)b - 16 : (int)b;
}

int orc_q4b_gemv(const uint8_t *codes, const uint16_t *bs, int rows, int cols,
                 const float *x, float *y) {
    const size_t rb = (size_t)(cols + 1) / 2, nb = (size_t)(cols + 31) / 32;
    #pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && rows >= 64)
    for (int j = 0; j < rows; j++) {
        const uint8_t *rc = codes + (size_t)j * rb;
        const uint16_t *b = bs + (size_t)j * nb;
        float facc = 0.0f;
        for (int blk = 0; blk * 32 < cols; blk++) {
            int i0 = blk * 32, i1 = i0 + 32 < cols ? i0 + 32 : cols;
            float acc = 0.0f;
            for (int i = i0; i < i1; i++) acc += (float)nib(rc, i) * x[i];
            facc += acc * orc_f16_to_f32(b[blk]);
        }
        y[j] = facc;
    }
    return 0;
}
static void gemv(const orc_w *w, const float *x, float *y) {
    orc_q4b_gemv(w->codes, w->bs, w->rows, w->cols, x, y);
}
static void embed_row(const orc_w *w, int tok, float *dst) {
    const uint8_t *rc = w->codes + (size_t)tok * (size_t)((w->cols + 1) / 2);
    const uint16_t *b = w->bs + (size_t)tok * (size_t)((w->cols + 31) / 32);
    for (int i = 0; i < w->cols; i++) dst[i] = (float)nib(rc, i) * orc_f16_to_f32(b[i >> 5]);
}

static float gelu_tanh(float x) {
    const float k = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}

/* ======================= exact islands (reference arithmetic) ======================= */
#define FB  30
#define ONE (1LL << FB)
static const int64_t LOG2E = 1549082005LL;
static const int64_t EXPC[7] = {1073741824LL, 744261118LL, 257941248LL, 59597083LL,
                                10327387LL, 1431680LL, 165394LL};
static int64_t exp2_frac(int64_t r) {
    int64_t acc = EXPC[6];
    for (int k = 5; k >= 0; k--) acc = ((acc * r) >> FB) + EXPC[k];
    return acc;
}
static int64_t exp_fixed(int64_t d) {
    int64_t g = (int64_t)(-(((i128)d * LOG2E) >> FB));
    int64_t n = g >> FB, r = g - (n << FB);
    if (n >= 32) return 0;
    if (r) return exp2_frac(ONE - r) >> (n + 1);
    return ONE >> n;
}
static uint64_t isqrt_u64(uint64_t v) {
    uint64_t x = 0, b = 1ULL << 62;
    while (b > v) b >>= 2;
    while (b) {
        if (v >= x + b) { v -= x + b; x = (x >> 1) + b; } else x >>= 1;
        b >>= 2;
    }
    return x;
}
void orc_rmsnorm_exact(const float *x, const float *w, int n, float *out) {
    enum { Q = 16, IB = 20, Qw = 16 };
    int64_t sumsq = 0;
    for (int i = 0; i < n; i++) { int64_t xi = (int64_t)llround((double)x[i] * (double)(1 << Q)); sumsq += xi * xi; }
    if (sumsq == 0) { for (int i = 0; i < n; i++) out[i] = 0.0f; return; }
    i128 num = (i128)n << (2 * (Q + IB));
    uint64_t q = (uint64_t)(num / (i128)sumsq);
    int64_t inv = (int64_t)isqrt_u64(q);
    const double denom = (double)(1ULL << (Q + IB + Qw));
    for (int i = 0; i < n; i++) {
        int64_t xi = (int64_t)llround((double)x[i] * (double)(1 << Q));
        int64_t wi = (int64_t)llround((double)w[i] * (double)(1 << Qw));
        i128 yi = (i128)xi * inv * wi;
        out[i] = (float)((double)(int64_t)yi / denom);
    }
}
void orc_softmax_exact(const float *z, int m, double *p) {
    enum { ZB = 14 };
    int64_t mx = INT64_MIN;
    for (int i = 0; i < m; i++) { int64_t zi = (int64_t)llround((double)z[i] * (double)(1 << ZB)); if (zi > mx) mx = zi; }
    int64_t S = 0;
    for (int i = 0; i < m; i++) {
        int64_t zi = (int64_t)llround((double)z[i] * (double)(1 << ZB));
        int64_t d = ((zi - mx) * ONE) >> ZB;
        p[i] = (double)exp_fixed(d);
        S += (int64_t)p[i];
    }
    for (int i = 0; i < m; i++) p[i] /= (double)S;
}
static const int64_t GK = 856722024LL, GA = 48012366LL;
static int64_t tanh_fixed(int64_t t) {
    int s = (t >= 0) ? 1 : -1;
    int64_t a = (t >= 0) ? t : -t;
    int64_t e2 = exp_fixed(-(2 * a));
    int64_t num = (2 * e2) << FB;
    return (int64_t)s * (ONE - num / (ONE + e2));
}
void orc_gelu_exact(const float *x, int n, float *out) {
    enum { ZB = 16 };
    for (int i = 0; i < n; i++) {
        int64_t xq = (int64_t)llround((double)x[i] * (double)(1 << ZB));
        int64_t X = (xq * ONE) >> ZB;
        i128 X2 = ((i128)X * X) >> FB;
        int64_t x3 = (int64_t)((X2 * X) >> FB);
        i128 inner = ((i128)GK * (X + (int64_t)(((i128)GA * x3) >> FB))) >> FB;
        int64_t t = tanh_fixed((int64_t)inner);
        int64_t g = (int64_t)(((i128)(X >> 1) * (ONE + t)) >> FB);
        out[i] = (float)((double)g / (double)ONE);
    }
}

/* ======================= build-defined exact primitives ======================= */
/* SiLU on the GELU island's grid: X = floor(rne_away(x*2^16) * 2^30 / 2^16),
 * sigma(X) in Q30 via exp_fixed of -|X|, silu = X*sigma >> 30. */
void orc_silu_exact(const float *x, int n, float *out) {
    for (int i = 0; i < n; i++) {
        int64_t xq = (int64_t)llround((double)x[i] * 65536.0);
        int64_t X = (xq * ONE) >> 16;
        int64_t e = exp_fixed(X >= 0 ? -X : X);                 /* e^-|X| in Q30 */
        int64_t sg = X >= 0 ? (int64_t)(((i128)ONE << FB) / (ONE + e))
                            : (int64_t)(((i128)e << FB) / (ONE + e));
        int64_t g = (int64_t)(((i128)X * sg) >> FB);
        out[i] = (float)((double)g / (double)ONE);
    }
}

/* RNE of (mag * 2^k) to float, mag > 0 unsigned 128-bit; handles subnormal and
 * overflow.  The single rounding primitive every exact-mode float result uses. */
static float u128_scaled_to_float(u128 mag, int k) {
    if (!mag) return 0.0f;
    int msb = 127; while (!((mag >> msb) & 1u)) msb--;
    int e = msb + k;                                   /* value in [2^e, 2^(e+1)) */
    int keep = 24;                                     /* significant bits kept */
    if (e < -126) keep = 24 - (-126 - e);              /* subnormal: fewer bits */
    if (keep <= 0) {                                   /* below half the smallest subnormal? */
        if (keep == 0) {                               /* value in [2^-150, 2^-149): round */
            u128 half = (u128)1 << msb;               /* value == 2^e exactly iff mag is a power of two */
            int tie = (mag == half);
            return tie ? 0.0f : 0x1.0p-149f;          /* tie rounds to even (zero) */
        }
        return 0.0f;
    }
    int drop = msb + 1 - keep;
    u128 q;
    if (drop > 0) {
        q = mag >> drop;
        u128 rem = mag & (((u128)1 << drop) - 1u), half = (u128)1 << (drop - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
    } else {
        q = mag << (-drop);
    }
    /* q has keep or keep+1 bits; value = q * 2^(k + drop) */
    int ex = k + drop;
    if (q >> keep) { /* rounding carried into a new bit: still exact via ldexp */ }
    float f = ldexpf((float)(uint32_t)q, ex);         /* q < 2^25: exact in float; ldexp exact or inf */
    return f;
}
static float i128_scaled_to_float(i128 v, int k) {
    if (v >= 0) return u128_scaled_to_float((u128)v, k);
    return -u128_scaled_to_float((u128)(-v), k);
}
/* RNE of num / (den * 2^k), den > 0: widen the numerator until the integer
 * quotient has >= 27 bits, fold the remainder into a sticky bit, round once. */
static int bitlen128(u128 v) { int b = 0; while (v) { v >>= 1; b++; } return b; }
static float i128_div_to_float(i128 num, int64_t den, int k) {
    if (!num) return 0.0f;
    int neg = num < 0;
    u128 n = neg ? (u128)(-num) : (u128)num, d = (u128)den;
    int sh = 28 + bitlen128(d) - bitlen128(n);
    if (sh < 0) sh = 0;
    n <<= sh;
    u128 q = n / d, r = n % d;
    q = (q << 1) | (r ? 1u : 0u);
    float f = u128_scaled_to_float(q, -(k + sh + 1));
    return neg ? -f : f;
}

/* activation grid: sh such that max|x| * 2^sh < 2^22 */
static int act_shift(const float *x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; i++) { float a = fabsf(x[i]); if (a > m) m = a; }
    if (m == 0.0f) return 1 << 20;                      /* all-zero marker */
    int e; frexpf(m, &e);                               /* m < 2^e */
    return 22 - e;
}
static void f16_parts(uint16_t h, int64_t *M, int *e) {
    int E5 = (h >> 10) & 31, mant = h & 1023;
    int64_t mm = E5 ? (int64_t)(1024 + mant) : (int64_t)mant;
    *e = E5 ? E5 - 25 : -24;
    *M = (h & 0x8000u) ? -mm : mm;
}
int orc_q4b_gemv_exact(const uint8_t *codes, const uint16_t *bs, int rows, int cols,
                       const float *x, float *y) {
    const size_t rb = (size_t)(cols + 1) / 2, nb = (size_t)(cols + 31) / 32;
    const int sh = act_shift(x, cols);
    if (sh == (1 << 20)) { for (int j = 0; j < rows; j++) y[j] = 0.0f; return 0; }
    int32_t *xq = (int32_t *)malloc((size_t)cols * sizeof(int32_t));
    for (int i = 0; i < cols; i++) xq[i] = (int32_t)rint(ldexp((double)x[i], sh));
    #pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && rows >= 64)
    for (int j = 0; j < rows; j++) {
        const uint8_t *rc = codes + (size_t)j * rb;
        const uint16_t *b = bs + (size_t)j * nb;
        i128 acc = 0;
        for (int blk = 0; blk * 32 < cols; blk++) {
            int i0 = blk * 32, i1 = i0 + 32 < cols ? i0 + 32 : cols;
            int32_t a = 0;
            for (int i = i0; i < i1; i++) a += nib(rc, i) * xq[i];
            int64_t M; int e; f16_parts(b[blk], &M, &e);
            /* (d * M) * 2^(e + 24): shifted as the unsigned image (a signed left
             * shift of a negative value is undefined in C; the bits are the same) */
            acc += (i128)((u128)(i128)((int64_t)a * M) << (e + 24));
        }
        y[j] = i128_scaled_to_float(acc, -24 - sh);
    }
    free(xq);
    return 0;
}

/* ---- integer transcendental constants for RoPE ---- */
/* isqrt of an unsigned 128-bit value */
static u128 isqrt_u128(u128 v) {
    u128 x = 0, b = (u128)1 << 126;
    while (b > v) b >>= 2;
    while (b) {
        if (v >= x + b) { v -= x + b; x = (x >> 1) + b; } else x >>= 1;
        b >>= 2;
    }
    return x;
}
/* round(2*pi * 2^60) and round(pi/2 * 2^60), from the decimal expansion of pi */
#define TWO_PI_Q60  ((int64_t)7244019458077122842LL)
#define HALF_PI_Q60 ((int64_t)1811004864519280711LL)
static int64_t ATAN_Q60[64];     /* atan(2^-i) */
static int64_t KINV_Q62;         /* prod 1/sqrt(1+2^-2i), i = 0..61 */
static int64_t EXP2NEG_Q62[64];  /* 2^(-2^-j), j = 1..62 */
static int cordic_ready;
static void cordic_init(void) {
    /* atan(t) for t = 2^-i by the alternating series, in Q120 then rounded to Q60;
     * atan(1) = pi/4 = HALF_PI/2. */
    ATAN_Q60[0] = HALF_PI_Q60 / 2;
    for (int i = 1; i < 64; i++) {
        i128 sum = 0; int sgn = 1;
        for (int k = 0; ; k++) {
            int pw = i * (2 * k + 1);                 /* t^(2k+1) = 2^-pw */
            if (pw >= 120) break;
            i128 term = ((i128)1 << (120 - pw)) / (2 * k + 1);
            sum += sgn > 0 ? term : -term; sgn = -sgn;
        }
        ATAN_Q60[i] = (int64_t)((sum + ((i128)1 << 59)) >> 60);
    }
    /* K^-1 = prod_i 1/sqrt(1 + 4^-i): each factor as floor(2^124 / isqrt((1+4^-i) 2^124)) >> 0 in Q62 */
    u128 k = (u128)1 << 62;
    for (int i = 0; i < 62; i++) {
        u128 r = isqrt_u128(((u128)1 << 124) + ((u128)1 << (124 - 2 * i)));   /* sqrt(1+4^-i) in Q62 */
        u128 f = ((u128)1 << 124) / r;                                         /* 1/sqrt in Q62 */
        k = (k * f) >> 62;
    }
    KINV_Q62 = (int64_t)k;
    /* 2^(-2^-j): repeated square roots of 1/2 in Q62 */
    u128 c = (u128)1 << 61;                           /* 2^-1 */
    for (int j = 1; j < 64; j++) {
        c = isqrt_u128(c << 62);                      /* sqrt in Q62 */
        EXP2NEG_Q62[j] = (int64_t)c;
    }
    cordic_ready = 1;
}

/* cos/sin of theta (Q60, any value in [0, 2*pi)) in Q62 via quadrant fold + CORDIC */
static void cordic_q62(int64_t th, int64_t *co, int64_t *si) {
    if (!cordic_ready) cordic_init();
    int quad = 0;
    while (th >= HALF_PI_Q60 && quad < 3) { th -= HALF_PI_Q60; quad++; }
    int64_t x = KINV_Q62, y = 0, z = th;              /* z in Q60 */
    for (int i = 0; i < 62; i++) {
        int64_t xs = x >> i, ys = y >> i;
        if (z >= 0) { x -= ys; y += xs; z -= ATAN_Q60[i]; }
        else        { x += ys; y -= xs; z += ATAN_Q60[i]; }
    }
    switch (quad) {
        case 0: *co = x;  *si = y;  break;
        case 1: *co = -y; *si = x;  break;
        case 2: *co = -x; *si = -y; break;
        default: *co = y; *si = -x; break;
    }
}
void orc_cordic_sincos(int64_t theta_q60, int32_t *cos_q30, int32_t *sin_q30) {
    int64_t c, s; cordic_q62(theta_q60, &c, &s);
    *cos_q30 = (int32_t)(c >> 32); *sin_q30 = (int32_t)(s >> 32);
}

/* log2 of a positive float in Q62 by repeated squaring (one bit per square) */
static i128 log2_q62(float v) {
    uint32_t bits; memcpy(&bits, &v, 4);
    int e = (int)((bits >> 23) & 255u) - 127;
    uint64_t m = (uint64_t)((bits & 0x7FFFFFu) | 0x800000u);   /* normal floats only */
    u128 y = (u128)m << (62 - 23);                    /* mantissa in [1,2) as Q62 */
    i128 frac = 0;
    for (int b = 61; b >= 0; b--) {
        y = (y * y) >> 62;
        if (y >= ((u128)2 << 62)) { y >>= 1; frac |= (i128)1 << b; }
    }
    return (i128)((u128)(i128)e << 62) + frac;      /* e < 0 for v < 1: shifted unsigned */
}
/* base^(-2i/d) in Q60: t = (2i/d)*log2(base) = n + r, result = 2^-r >> n with
 * 2^-r = prod over the set bits j of r of 2^(-2^-j). */
int64_t orc_rope_freq_q60(float base, int i, int d) {
    if (!cordic_ready) cordic_init();
    if (i == 0) return (int64_t)1 << 60;
    i128 t = (log2_q62(base) * (i128)(2 * i)) / (i128)d;   /* Q62, >= 0 for base > 1 */
    if (t < 0) t = 0;
    int64_t n = (int64_t)(t >> 62);
    uint64_t r = (uint64_t)(t & (((i128)1 << 62) - 1));
    u128 acc = (u128)1 << 62;
    for (int j = 1; j <= 62; j++)
        if ((r >> (62 - j)) & 1u) acc = (acc * (u128)EXP2NEG_Q62[j]) >> 62;
    if (n >= 62) return 0;
    return (int64_t)((acc >> 2) >> n);                /* Q62 -> Q60 */
}

void orc_rope_exact(float *v, int d, int p, float base) {
    const int half = d / 2;
    for (int i = 0; i < half; i++) {
        const int64_t F = orc_rope_freq_q60(base, i, d);
        const i128 th = (i128)p * F;
        const int64_t r = (int64_t)(th % (i128)TWO_PI_Q60);
        int64_t c, s; cordic_q62(r, &c, &s);
        const float cf = i128_scaled_to_float(c, -62), sf = i128_scaled_to_float(s, -62);
        const float a = v[i], b = v[i + half];
        const float ac = a * cf, bs = b * sf, as = a * sf, bc = b * cf;
        v[i] = ac - bs;
        v[i + half] = as + bc;
    }
}


/* ======================= Spinor-63 KV block codec =======================
 * Restates core/vht2/vht2.c:31-104 (CRC-8, VHT2 canonical projection and int8
 * quantization), core/vht2/mobius_reorder.c:16-55 (the affine permutation,
 * A = 17 mod 55) and core/vht2/spinor_block.c:59-149 (63-byte assembly and the
 * balanced multi-block split).  Byte image: [0..3] scale float32 LE, [4] exponent
 * (0), [5] basis (0 = canonical), [6] reserved (0), [7..61] body with
 * body[17 i mod 55] = coeff[i], [62] CRC-8 of bytes 0..61. */
#define SPN_BODY 55
#define SPN_MOBIUS_A 17

uint8_t orc_crc8(const uint8_t *d, int n) {
    /* CRC-8/SMBus: polynomial x^8 + x^2 + x + 1 (0x07), MSB first, init 0 */
    unsigned r = 0;
    for (int i = 0; i < n; i++) {
        r ^= d[i];
        for (int b = 0; b < 8; b++) r = (r & 0x80u) ? ((r << 1) ^ 0x07u) & 0xFFu : (r << 1) & 0xFFu;
    }
    return (uint8_t)r;
}
int orc_spinor_blocks_for(int k) { return k <= SPN_BODY ? 1 : (k + SPN_BODY - 1) / SPN_BODY; }

/* round half away from zero as the reference writes it (x + 0.5 rounded in float first) */
static int32_t spn_round(float x) { return (int32_t)(x >= 0.0f ? floorf(x + 0.5f) : ceilf(x - 0.5f)); }

void orc_spinor_encode(const float *vec, int k, uint8_t blk[63]) {
    const int lim = k < 0 ? 0 : (k < SPN_BODY ? k : SPN_BODY);
    float mx = 0.0f;
    for (int i = 0; i < lim; i++) if (fabsf(vec[i]) > mx) mx = fabsf(vec[i]);
    const float scale = mx > 0.0f ? mx : 1.0f;
    memset(blk, 0, 63);
    uint32_t sb; memcpy(&sb, &scale, 4);
    for (int j = 0; j < 4; j++) blk[j] = (uint8_t)(sb >> (8 * j));
    for (int i = 0; i < lim; i++) {
        int32_t c = spn_round((vec[i] / scale) * 127.0f);
        c = c > 127 ? 127 : (c < -127 ? -127 : c);
        blk[7 + (SPN_MOBIUS_A * i) % SPN_BODY] = (uint8_t)(int8_t)c;
    }
    blk[62] = orc_crc8(blk, 62);
}
int orc_spinor_decode(const uint8_t blk[63], float *vec, int k) {
    if (orc_crc8(blk, 62) != blk[62]) return 1;
    const uint32_t sb = (uint32_t)blk[0] | (uint32_t)blk[1] << 8 | (uint32_t)blk[2] << 16 | (uint32_t)blk[3] << 24;
    float scale; memcpy(&scale, &sb, 4);
    const float mul = scale * ldexpf(1.0f, (int)(int8_t)blk[4]) / 127.0f;
    const int lim = k < 0 ? 0 : (k < SPN_BODY ? k : SPN_BODY);
    for (int i = 0; i < lim; i++) vec[i] = (float)(int8_t)blk[7 + (SPN_MOBIUS_A * i) % SPN_BODY] * mul;
    for (int i = SPN_BODY; i < k; i++) vec[i] = 0.0f;
    return 0;
}
/* k coordinates in nblk contiguous chunks of k/nblk, the first k % nblk one longer */
void orc_spinor_encode_vec(const float *vec, int k, uint8_t *blocks) {
    const int nb = orc_spinor_blocks_for(k), base = k / nb, extra = k % nb;
    for (int b = 0, off = 0; b < nb; b++) {
        const int len = base + (b < extra);
        orc_spinor_encode(vec + off, len, blocks + 63 * b);
        off += len;
    }
}
int orc_spinor_decode_vec(const uint8_t *blocks, int k, float *vec) {
    const int nb = orc_spinor_blocks_for(k), base = k / nb, extra = k % nb;
    int rc = 0;
    for (int b = 0, off = 0; b < nb; b++) {
        const int len = base + (b < extra);
        rc |= orc_spinor_decode(blocks + 63 * b, vec + off, len);
        off += len;
    }
    return rc;
}
static void spinor_roundtrip(float *v, int k) {
    uint8_t blk[63 * 16];                 /* k <= 880 */
    orc_spinor_encode_vec(v, k, blk);
    (void)orc_spinor_decode_vec(blk, k, v);
}

/* ======================= ARM recall router =======================
 * Restates core/arm/arm.c: the frozen +-1 projection (SplitMix64 from the seed
 * of include/sp/arm.h:49, :17-27), the sequential float projection (:31-45),
 * the descending median-of-three quickselect (:49-76) and the selection
 * sinks u top-(B-W-sink) u recent-W (:110-160), with the sidecar layout
 * projk[((L*P + s)*NKV + kvh)*r + p] of arm.h:60-67. */
#define ORC_ARM_SEED 0x5350524F4A2BULL
typedef struct { float s; int i; } orc_sidx;
static uint64_t arm_splitmix(uint64_t *st) {
    uint64_t z = (*st += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
void orc_arm_build_R(signed char *R, int r, int hd) {
    uint64_t st = ORC_ARM_SEED;
    for (int i = 0; i < r * hd; i++) R[i] = (arm_splitmix(&st) & 1) ? 1 : -1;
}
void orc_arm_project(const signed char *R, int r, int hd, const float *vec, float *proj) {
    for (int p = 0; p < r; p++) {
        float a = 0.0f;
        for (int d = 0; d < hd; d++) a += (float)R[(size_t)p * hd + d] * vec[d];
        proj[p] = a;
    }
}
static void sidx_swap(orc_sidx *a, int i, int j) { orc_sidx t = a[i]; a[i] = a[j]; a[j] = t; }
static int qsel_partition(orc_sidx *a, int lo, int hi) {
    const int mid = lo + (hi - lo) / 2;
    if (a[mid].s > a[lo].s) sidx_swap(a, lo, mid);
    if (a[hi].s > a[lo].s) sidx_swap(a, lo, hi);
    if (a[hi].s > a[mid].s) sidx_swap(a, mid, hi);
    const float pivot = a[mid].s;
    sidx_swap(a, mid, hi);
    int store = lo;
    for (int j = lo; j < hi; j++) if (a[j].s > pivot) { sidx_swap(a, j, store); store++; }
    sidx_swap(a, store, hi);
    return store;
}
static void qsel_topk(orc_sidx *a, int n, int k) {
    if (k <= 0 || k >= n) return;
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int p = qsel_partition(a, lo, hi);
        if (p == k) break;
        else if (p < k) lo = p + 1;
        else hi = p - 1;
    }
}
/* one head's recall set into ri (returns its size): [0, pos] when B <= 0 or
 * the context is within budget, else sinks u top-(B-W-sink) u recent-W;
 * pk: this layer's sidecar rows for kv head kvh, stride nkv*r floats */
int orc_arm_select(const signed char *R, int r, int hd, const float *qh, const float *pk, int nkv,
                   int B, int W0, int sink0, int pos, void *cand_v, int *ri) {
    orc_sidx *cand = (orc_sidx *)cand_v;
    if (B <= 0 || pos + 1 <= B) { for (int s = 0; s <= pos; s++) ri[s] = s; return pos + 1; }
    float pq[64];
    orc_arm_project(R, r, hd, qh, pq);
    int W = W0 > pos + 1 ? pos + 1 : W0;
    int sink = sink0 > pos + 1 ? pos + 1 : sink0;
    int cand_hi = pos + 1 - W;
    if (cand_hi < sink) cand_hi = sink;
    if (cand_hi > pos + 1) cand_hi = pos + 1;
    int topk = B - W - sink; if (topk < 0) topk = 0;
    if (topk > cand_hi - sink) topk = cand_hi - sink;
    int nc = 0;
    for (int s = sink; s < cand_hi; s++) {
        const float *k = pk + (size_t)s * nkv * r;
        float a = 0.0f;
        for (int p = 0; p < r; p++) a += pq[p] * k[p];
        cand[nc].s = a; cand[nc].i = s; nc++;
    }
    if (topk > nc) topk = nc;
    qsel_topk(cand, nc, topk);
    /* Ties at the k-th score: the quickselect keeps whichever equal candidates
     * its partitions leave in front, an artefact of its order.  The rule here
     * (and on the device) keeps the lowest positions among the candidates equal
     * to the k-th score; without such a tie the set is the quickselect's.
     * (-0.0 == +0.0, as in the reference's comparisons.)  Parity unpinned
     * against the reference for exact ties at the k-th score. */
    if (topk > 0 && topk < nc) {
        float th = cand[0].s;
        for (int t = 1; t < topk; t++) if (cand[t].s < th) th = cand[t].s;
        int tied_out = 0;
        for (int t = topk; t < nc; t++) if (cand[t].s == th) { tied_out = 1; break; }
        if (tied_out) {
            int above = 0;                 /* selected strictly above th, kept in place */
            for (int t = 0; t < topk; t++) if (cand[t].s > th) sidx_swap(cand, t, above++);
            /* the remaining slots: candidates equal to th, lowest positions first */
            for (int t = above; t < topk; t++) {
                int best = -1;
                for (int u = t; u < nc; u++)
                    if (cand[u].s == th && (best < 0 || cand[u].i < cand[best].i)) best = u;
                sidx_swap(cand, t, best);
            }
        }
    }
    int m = 0;
    for (int s2 = 0; s2 < sink; s2++) ri[m++] = s2;
    for (int t = 0; t < topk; t++) ri[m++] = cand[t].i;
    for (int s2 = cand_hi; s2 <= pos; s2++) ri[m++] = s2;
    return m;
}

/* float attention of one head over the positions ri[0, mm) in that order
 * (core/forward/decode.c:755-790: scores, max, exp-sum and V-sum in ri order) */
static void attn_head_list(const float *qh, const float *KC, const float *VC, const int *ri, int mm, int KVD,
                           int kvh, int HD, float ascale, float *sc, float *out) {
    float maxs = -INFINITY;
    for (int jj = 0; jj < mm; jj++) {
        const float *kh = KC + (size_t)ri[jj] * KVD + (size_t)kvh * HD;
        float acc = 0.0f;
        for (int i = 0; i < HD; i++) acc += qh[i] * kh[i];
        const float d = acc * ascale;
        sc[jj] = d;
        if (d > maxs) maxs = d;
    }
    float sum = 0.0f;
    for (int jj = 0; jj < mm; jj++) { sc[jj] = expf(sc[jj] - maxs); sum += sc[jj]; }
    const float inv = 1.0f / sum;
    for (int i = 0; i < HD; i++) out[i] = 0.0f;
    for (int jj = 0; jj < mm; jj++) {
        const float w = sc[jj] * inv;
        const float *vh = VC + (size_t)ri[jj] * KVD + (size_t)kvh * HD;
        for (int i = 0; i < HD; i++) out[i] += w * vh[i];
    }
}

/* ======================= session + steps ======================= */
struct orc_sess {
    orc_model *m;
    int mode, P, pos, kv_filled;
    uint32_t kv_flags;                /* ORC_KV_SPINOR / ORC_KV_SPINOR_REF: K/V pass the Spinor codec */
    int kv_forced;                    /* steps keep the K/V rows resident at pos (set by orc_kv_set) */
    int vclamp;                       /* exact mode: V heads stored with a clamped element */
    /* ARM recall (orc_set_recall): budget B, window W, sinks, projection rows r;
     * R [r][HD] frozen +-1 projection, projk [NL][P][NKV][r] sidecar, per-head
     * selection scratch ri / cand [NH][P] */
    int rec_B, rec_W, rec_sink, rec_r;
    int rec_dense;                    /* orc_set_recall_dense: effective budget 0 (identity lists) */
    int rec_kvsel;                    /* orc_set_recall_kvsel: one selection per kv head (SP_RECALL_KVSEL) */
    int rec_mm[256];                  /* KVSEL: each kv head's set size this step */
    float *rec_qg;                    /* KVSEL: the group-centroid query [HD] */
    signed char *rec_R;
    float *projk;
    int *rec_ri;
    void *rec_cand;
    float *kc, *vc;                   /* [NL][P][KVD]; int32 payload in exact mode */
    float *x, *nx, *q, *kn, *vn, *ao, *ap, *gg, *up, *dn, *sc;
    double *pd;
};

orc_sess *orc_sess_new(orc_model *m, int max_ctx, int mode) { return orc_sess_new_kv(m, max_ctx, mode, 0u); }
orc_sess *orc_sess_new_kv(orc_model *m, int max_ctx, int mode, uint32_t kv_flags) {
    if (!m || max_ctx <= 0) return NULL;
    orc_sess *s = (orc_sess *)calloc(1, sizeof *s);
    s->m = m; s->mode = mode; s->P = max_ctx; s->kv_flags = kv_flags;
    const size_t KVD = (size_t)m->NKV * m->HD, QD = (size_t)m->NH * m->HD;
    const size_t kv = (size_t)m->NL * (size_t)max_ctx * KVD;
    s->kc = (float *)malloc(kv * sizeof(float)); s->vc = (float *)malloc(kv * sizeof(float));
    s->x = (float *)malloc(m->E * sizeof(float)); s->nx = (float *)malloc(m->E * sizeof(float));
    s->q = (float *)malloc(QD * sizeof(float)); s->kn = (float *)malloc(KVD * sizeof(float));
    s->vn = (float *)malloc(KVD * sizeof(float)); s->ao = (float *)malloc(QD * sizeof(float));
    s->ap = (float *)malloc(m->E * sizeof(float)); s->gg = (float *)malloc(m->FF * sizeof(float));
    s->up = (float *)malloc(m->FF * sizeof(float)); s->dn = (float *)malloc(m->E * sizeof(float));
    s->sc = (float *)malloc((size_t)m->NH * (size_t)max_ctx * sizeof(float));   /* one score row per q head */
    s->pd = (double *)malloc((size_t)max_ctx * sizeof(double));
    if (!s->kc || !s->vc || !s->sc || !s->pd) { orc_sess_free(s); return NULL; }
    return s;
}
void orc_sess_free(orc_sess *s) {
    if (!s) return;
    free(s->kc); free(s->vc); free(s->x); free(s->nx); free(s->q); free(s->kn); free(s->vn);
    free(s->ao); free(s->ap); free(s->gg); free(s->up); free(s->dn); free(s->sc); free(s->pd);
    free(s->rec_R); free(s->projk); free(s->rec_ri); free(s->rec_cand); free(s->rec_qg); free(s);
}
int orc_set_recall(orc_sess *s, int B, int W, int sink, int r) {
    if (!s || B < 0 || W < 0 || sink < 0 || r < 1 || r > 64) return 1;
    free(s->rec_R); free(s->projk); free(s->rec_ri); free(s->rec_cand); free(s->rec_qg);
    s->rec_R = NULL; s->projk = NULL; s->rec_ri = NULL; s->rec_cand = NULL; s->rec_qg = NULL;
    s->rec_B = B; s->rec_W = W; s->rec_sink = sink; s->rec_r = r;
    if (!B) return 0;
    const orc_model *m = s->m;
    s->rec_R = (signed char *)malloc((size_t)r * m->HD);
    s->projk = (float *)calloc((size_t)m->NL * s->P * m->NKV * r, sizeof(float));
    s->rec_ri = (int *)malloc((size_t)m->NH * s->P * sizeof(int));
    s->rec_cand = malloc((size_t)m->NH * s->P * sizeof(orc_sidx));
    s->rec_qg = (float *)malloc((size_t)m->HD * sizeof(float));
    if (!s->rec_R || !s->projk || !s->rec_ri || !s->rec_cand || !s->rec_qg) return 1;
    orc_arm_build_R(s->rec_R, r, (int)m->HD);
    return 0;
}
void orc_set_recall_dense(orc_sess *s, int on) { s->rec_dense = on ? 1 : 0; }
/* SP_RECALL_KVSEL (core/forward/decode.c:53-63, :600-629, :738-757): the
 * group leader selects once per kv head with the group-centroid query
 * qg = ((0 + q_0) + q_1) + ... (float, in head order) and every q head of the
 * group attends over that shared set with its own q. */
int orc_set_recall_kvsel(orc_sess *s, int on) {
    if (on && s->m->NKV > 256) return 1;
    s->rec_kvsel = on ? 1 : 0;
    return 0;
}
/* the KVSEL lists of one layer at pos: list kvh at rec_ri + kvh * P */
static void kvsel_select(orc_sess *s, int L, const float *q, int pos, float *qg) {
    const orc_model *m = s->m;
    const int HD = (int)m->HD, NKV = (int)m->NKV, group = (int)(m->NH / m->NKV), P = s->P;
    for (int kvh = 0; kvh < NKV; kvh++) {
        for (int i = 0; i < HD; i++) qg[i] = 0.0f;
        for (int g2 = 0; g2 < group; g2++) {
            const float *qx = q + (size_t)(kvh * group + g2) * HD;
            for (int i = 0; i < HD; i++) qg[i] += qx[i];
        }
        s->rec_mm[kvh] = orc_arm_select(s->rec_R, s->rec_r, HD, qg, s->projk + ((size_t)L * P * NKV + kvh) * s->rec_r,
                                        NKV, s->rec_dense ? 0 : s->rec_B, s->rec_W, s->rec_sink, pos,
                                        (orc_sidx *)s->rec_cand + (size_t)kvh * P, s->rec_ri + (size_t)kvh * P);
    }
}
int orc_recall_sidecar_set(orc_sess *s, int layer, int p0, int n, const float *in) {
    if (!s || !s->projk || layer < 0 || layer >= (int)s->m->NL || p0 < 0 || n < 0 || p0 + n > s->P) return 1;
    const size_t row = (size_t)s->m->NKV * s->rec_r;
    memcpy(s->projk + ((size_t)layer * s->P + p0) * row, in, (size_t)n * row * sizeof(float));
    return 0;
}
int orc_recall_sidecar(const orc_sess *s, int layer, int p0, int n, float *out) {
    if (!s || !s->projk || layer < 0 || layer >= (int)s->m->NL || p0 < 0 || n < 0 || p0 + n > s->P) return 1;
    const size_t row = (size_t)s->m->NKV * s->rec_r;
    memcpy(out, s->projk + ((size_t)layer * s->P + p0) * row, (size_t)n * row * sizeof(float));
    return 0;
}
int orc_pos(const orc_sess *s) { return s->pos; }
void orc_set_kv_forced(orc_sess *s, int on) { s->kv_forced = on ? 1 : 0; }
int orc_set_pos(orc_sess *s, int pos) {
    if (pos < 0 || pos > s->P) return 1;
    s->pos = pos; s->kv_filled = pos; return 0;
}
int orc_rewind(orc_sess *s, int n) {
    if (n < 0 || n > s->pos) return 1;
    s->pos -= n;
    if (s->kv_filled > s->pos) s->kv_filled = s->pos;
    return 0;
}
orc_sess *orc_clone(const orc_sess *s) {
    orc_sess *c = orc_sess_new_kv(s->m, s->P, s->mode, s->kv_flags);
    if (!c) return NULL;
    const size_t kv = (size_t)s->m->NL * (size_t)s->P * s->m->NKV * s->m->HD;
    memcpy(c->kc, s->kc, kv * sizeof(float)); memcpy(c->vc, s->vc, kv * sizeof(float));
    c->pos = s->pos; c->kv_filled = s->kv_filled;
    if (s->rec_B > 0) {
        if (orc_set_recall(c, s->rec_B, s->rec_W, s->rec_sink, s->rec_r)) { orc_sess_free(c); return NULL; }
        memcpy(c->projk, s->projk, (size_t)s->m->NL * s->P * s->m->NKV * s->rec_r * sizeof(float));
    }
    c->rec_dense = s->rec_dense;
    c->rec_kvsel = s->rec_kvsel;
    return c;
}
int orc_kv_get(const orc_sess *s, int layer, int p0, int n, float *k, float *v) {
    const size_t KVD = (size_t)s->m->NKV * s->m->HD;
    if (layer < 0 || layer >= (int)s->m->NL || p0 < 0 || n < 0 || p0 + n > s->P) return 1;
    const size_t off = ((size_t)layer * s->P + p0) * KVD;
    memcpy(k, s->kc + off, (size_t)n * KVD * sizeof(float));
    memcpy(v, s->vc + off, (size_t)n * KVD * sizeof(float));
    return 0;
}
int orc_kv_set(orc_sess *s, int layer, int p0, int n, const float *k, const float *v) {
    const size_t KVD = (size_t)s->m->NKV * s->m->HD;
    if (layer < 0 || layer >= (int)s->m->NL || p0 < 0 || n < 0 || p0 + n > s->P) return 1;
    const size_t off = ((size_t)layer * s->P + p0) * KVD;
    memcpy(s->kc + off, k, (size_t)n * KVD * sizeof(float));
    memcpy(s->vc + off, v, (size_t)n * KVD * sizeof(float));
    return 0;
}

/* exact-mode attention for one q-head over [s0, pos] -- or, with a position
 * list ri[0, mm), over those positions (recall); K/V slabs hold int32.  Every
 * sum is an integer, so the list's order does not matter. */
static void attn_head_exact_sel(const float *qh, const int32_t *KC, const int32_t *VC, int pos, int KVD,
                                int kvh, int HD, float ascale, int win, const int *ri, int mm, float *out) {
    const int s0 = (win >= 0 && pos - win + 1 > 0) ? pos - win + 1 : 0;
    const int n = ri ? mm : pos + 1 - s0;
    int32_t qi[1024];
    for (int i = 0; i < HD; i++) qi[i] = (int32_t)rintf(qh[i] * 65536.0f);
    int64_t mx = INT64_MIN;
    int64_t *zi = (int64_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(int64_t));
    for (int j = 0; j < n; j++) {
        const int s = ri ? ri[j] : s0 + j;
        const int32_t *kh = KC + (size_t)s * KVD + (size_t)kvh * HD;
        int64_t ip = 0;
        for (int i = 0; i < HD; i++) ip += (int64_t)qi[i] * kh[i];
        const float scv = (float)((double)ip / 4294967296.0) * ascale;
        zi[j] = (int64_t)llround((double)scv * 16384.0);
        if (zi[j] > mx) mx = zi[j];
    }
    int64_t S = 0;
    i128 acc[1024];
    for (int i = 0; i < HD; i++) acc[i] = 0;
    for (int j = 0; j < n; j++) {
        const int s = ri ? ri[j] : s0 + j;
        int64_t e = exp_fixed(((zi[j] - mx) * ONE) >> 14) >> 8;
        S += e;
        const int32_t *vh = VC + (size_t)s * KVD + (size_t)kvh * HD;
        for (int i = 0; i < HD; i++) acc[i] += (i128)((int64_t)e * vh[i]);
    }
    for (int i = 0; i < HD; i++) out[i] = i128_div_to_float(acc[i], S, 16);
    free(zi);
}
static void attn_head_exact(const float *qh, const int32_t *KC, const int32_t *VC, int pos, int KVD,
                            int kvh, int HD, float ascale, int win, float *sc, float *out) {
    (void)sc;
    attn_head_exact_sel(qh, KC, VC, pos, KVD, kvh, HD, ascale, win, NULL, 0, out);
}

static int32_t vq_of(float v, int *clamped) {
    float r = rintf(v * 65536.0f);
    if (r > 8388607.0f) { r = 8388607.0f; *clamped = 1; }
    if (r < -8388607.0f) { r = -8388607.0f; *clamped = 1; }
    return (int32_t)r;
}
int32_t orc_vq_of(float v, int *clamped) { int c = 0; int32_t q = vq_of(v, &c); if (clamped) *clamped = c; return q; }
void orc_attn_head_exact(const float *qh, const int32_t *KC, const int32_t *VC, int pos, int KVD, int kvh,
                         int HD, float ascale, int win, float *out) {
    float *sc = (float *)malloc((size_t)(pos + 1) * sizeof(float));
    attn_head_exact(qh, KC, VC, pos, KVD, kvh, HD, ascale, win, sc, out);
    free(sc);
}
float orc_i128_div_to_float(int64_t num_hi, uint64_t num_lo, int64_t den, int k) {
    const i128 num = (i128)(((u128)(uint64_t)num_hi << 64) | num_lo);
    return i128_div_to_float(num, den, k);
}
int orc_v_clamps(const orc_sess *s) { return s->vclamp; }

static int step_any(orc_sess *s, int32_t tok, int pos, float *logits) {
    orc_model *m = s->m;
    const int gemma = (m->arch == 3u), ex = (s->mode == ORC_EXACT);
    const int E = (int)m->E, FF = (int)m->FF, HD = (int)m->HD, NH = (int)m->NH, NKV = (int)m->NKV;
    const int KVD = NKV * HD, group = NH / NKV, P = s->P;
    const float eps = m->eps, ascale = 1.0f / sqrtf((float)HD);
    float *x = s->x, *nx = s->nx, *q = s->q, *kn = s->kn, *vn = s->vn, *ao = s->ao, *ap = s->ap,
          *gg = s->gg, *up = s->up, *dn = s->dn, *sc = s->sc;
    if (tok < 0 || (uint32_t)tok >= m->V) return 1;
#define GEMV(w, in, out) (ex ? (void)orc_q4b_gemv_exact((w)->codes, (w)->bs, (w)->rows, (w)->cols, (in), (out)) \
                             : gemv((w), (in), (out)))
#define NORM(in, w, n, out) (ex ? orc_rmsnorm_exact((in), (w), (n), (out)) : orc_rmsnorm((in), (w), (n), eps, (out)))
    embed_row(&m->embd, tok, x);
    if (gemma) { const float es = sqrtf((float)E); for (int i = 0; i < E; i++) x[i] *= es; }
    for (uint32_t L = 0; L < m->NL; L++) {
        const orc_layer *ly = &m->L[L];
        const int global = gemma ? ((L % 6) == 5) : 1;
        const float rbase = (gemma && !global) ? 10000.0f : m->base;
        const int win = (gemma && !global) ? (int)m->SW : -1;
        NORM(x, ly->attn_norm, E, nx);
        GEMV(&ly->q, nx, q); GEMV(&ly->k, nx, kn); GEMV(&ly->v, nx, vn);
        for (int h = 0; h < NH; h++) {
            float *qh = q + (size_t)h * HD;
            if (ex) { orc_rmsnorm_exact(qh, ly->q_norm, HD, qh); orc_rope_exact(qh, HD, pos, rbase); }
            else { rmsnorm_head(qh, ly->q_norm, HD, eps); orc_rope_neox(qh, HD, pos, rbase); }
        }
        for (int h = 0; h < NKV; h++) {
            float *kh = kn + (size_t)h * HD;
            if (ex) { orc_rmsnorm_exact(kh, ly->k_norm, HD, kh); orc_rope_exact(kh, HD, pos, rbase); }
            else { rmsnorm_head(kh, ly->k_norm, HD, eps); orc_rope_neox(kh, HD, pos, rbase); }
        }
        if (s->rec_B > 0 && !s->kv_forced)            /* recall sidecar of the new position (decode.c:493-503) */
            for (int h = 0; h < NKV; h++)
                orc_arm_project(s->rec_R, s->rec_r, HD, kn + (size_t)h * HD,
                                s->projk + (((size_t)L * P + pos) * NKV + h) * (size_t)s->rec_r);
        if (s->kv_forced) { /* the caller's rows at pos stand */ }
        else if (s->kv_flags & (ORC_KV_SPINOR | ORC_KV_SPINOR_REF))
            /* sp_session.c:298-320: the block cache (mode 1) and the in-place
             * round trip (mode 2) hand the attention the same decoded values */
            for (int h = 0; h < 2 * NKV; h++) spinor_roundtrip((h < NKV ? kn : vn) + (size_t)(h % NKV) * HD, HD);
        float *kcl = s->kc + (size_t)L * P * KVD, *vcl = s->vc + (size_t)L * P * KVD;
        if (ex) {
            int32_t *kd = (int32_t *)(kcl + (size_t)pos * KVD), *vd = (int32_t *)(vcl + (size_t)pos * KVD);
            if (!s->kv_forced)
                for (int h = 0; h < NKV; h++) {
                    int cl = 0;
                    for (int i = h * HD; i < (h + 1) * HD; i++) { kd[i] = (int32_t)rintf(kn[i] * 65536.0f); vd[i] = vq_of(vn[i], &cl); }
                    s->vclamp += cl;
                }
            const int kvsel = s->rec_B > 0 && win < 0 && s->rec_kvsel;
            if (kvsel) kvsel_select(s, L, q, pos, s->rec_qg);
            #pragma omp parallel for schedule(static, 1) num_threads(g_threads) if (g_threads > 1 && pos >= 256)
            for (int h = 0; h < NH; h++) {
                if (s->rec_B > 0 && win < 0) {           /* recall: the head's selected positions */
                    int *ri = s->rec_ri + (size_t)(kvsel ? h / group : h) * P;
                    const int mm = kvsel ? s->rec_mm[h / group]
                                         : orc_arm_select(s->rec_R, s->rec_r, HD, q + (size_t)h * HD,
                                                  s->projk + ((size_t)L * P * NKV + h / group) * s->rec_r, NKV,
                                                  s->rec_dense ? 0 : s->rec_B, s->rec_W, s->rec_sink, pos,
                                                  (orc_sidx *)s->rec_cand + (size_t)h * P, ri);
                    attn_head_exact_sel(q + (size_t)h * HD, (const int32_t *)kcl, (const int32_t *)vcl, pos, KVD,
                                        h / group, HD, ascale, -1, ri, mm, ao + (size_t)h * HD);
                } else {
                    attn_head_exact(q + (size_t)h * HD, (const int32_t *)kcl, (const int32_t *)vcl, pos, KVD,
                                    h / group, HD, ascale, win, sc + (size_t)h * P, ao + (size_t)h * HD);
                }
            }
        } else {
            if (!s->kv_forced) {
                memcpy(kcl + (size_t)pos * KVD, kn, (size_t)KVD * sizeof(float));
                memcpy(vcl + (size_t)pos * KVD, vn, (size_t)KVD * sizeof(float));
            }
            const int kvsel = s->rec_B > 0 && win < 0 && s->rec_kvsel;
            if (kvsel) kvsel_select(s, L, q, pos, s->rec_qg);
            #pragma omp parallel for schedule(static, 1) num_threads(g_threads) if (g_threads > 1 && pos >= 256)
            for (int h = 0; h < NH; h++) {
                if (s->rec_B > 0 && win < 0) {           /* recall: decode.c:740-790 */
                    int *ri = s->rec_ri + (size_t)(kvsel ? h / group : h) * P;
                    const int mm = kvsel ? s->rec_mm[h / group]
                                         : orc_arm_select(s->rec_R, s->rec_r, HD, q + (size_t)h * HD,
                                                  s->projk + ((size_t)L * P * NKV + h / group) * s->rec_r, NKV,
                                                  s->rec_dense ? 0 : s->rec_B, s->rec_W, s->rec_sink, pos,
                                                  (orc_sidx *)s->rec_cand + (size_t)h * P, ri);
                    attn_head_list(q + (size_t)h * HD, kcl, vcl, ri, mm, KVD, h / group, HD, ascale,
                                   sc + (size_t)h * P, ao + (size_t)h * HD);
                } else {
                    orc_attn_head(q + (size_t)h * HD, kcl, vcl, pos, KVD, h / group, HD, ascale, win, sc + (size_t)h * P,
                                  ao + (size_t)h * HD);
                }
            }
        }
        GEMV(&ly->o, ao, ap);
        if (gemma) { NORM(ap, ly->post_attn, E, nx); for (int i = 0; i < E; i++) x[i] += nx[i]; }
        else { for (int i = 0; i < E; i++) x[i] += ap[i]; }
        NORM(x, ly->ffn_norm, E, nx);
        GEMV(&ly->gate, nx, gg); GEMV(&ly->up, nx, up);
        if (gemma) {
            if (ex) { orc_gelu_exact(gg, FF, gg); for (int i = 0; i < FF; i++) gg[i] = gg[i] * up[i]; }
            else for (int i = 0; i < FF; i++) gg[i] = gelu_tanh(gg[i]) * up[i];
        } else {
            if (ex) { orc_silu_exact(gg, FF, gg); for (int i = 0; i < FF; i++) gg[i] = gg[i] * up[i]; }
            else for (int i = 0; i < FF; i++) { float gv = gg[i]; gg[i] = gv / (1.0f + expf(-gv)) * up[i]; }
        }
        GEMV(&ly->down, gg, dn);
        if (gemma) { NORM(dn, ly->post_ffw, E, nx); for (int i = 0; i < E; i++) x[i] += nx[i]; }
        else { for (int i = 0; i < E; i++) x[i] += dn[i]; }
    }
    if (logits) {
        NORM(x, m->out_norm, E, nx);
        GEMV(&m->out, nx, logits);
    }
#undef GEMV
#undef NORM
    return 0;
}

/* sp_decode_step semantics (sp_session.c:748-769): lazily backfill K/V for
 * [kv_filled, pos), then step the new token at pos. */
int orc_step(orc_sess *s, int32_t tok, float *logits) {
    if (s->pos >= s->P) return 1;
    int p = s->pos;
    if (step_any(s, tok, p, logits)) return 1;
    s->kv_filled = p + 1;
    s->pos = p + 1;
    return 0;
}
