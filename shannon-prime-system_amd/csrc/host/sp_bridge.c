/* sp_bridge.c -- .sp-model handle -> qwen3_model (the representation the
 * section-6b open() receives), plus the named packed-tensor arena behind it.
 *
 * Reproduces the observable result of core/session/sp_model_bridge.c:114-171
 * (packed builders, norm copies) and :173-485 (qwen3 / gemma3 bridges):
 *  - every matmul weight and token_embd becomes an arena entry keyed by its
 *    GGUF name, aliasing the mapped codes (and .scale / .bscale sibling);
 *    OK_Q4B rows get row_prec 4, row_scale NULL, bs_nblk = ceil(cols/32);
 *  - norm vectors are copied to owned f32 and found again by pointer identity
 *    (sp_as_f32, core/forward_dispatch/forward_dispatch.c:182-188);
 *  - n_ff falls back to blk.0.ffn_gate's out-dim, rms_eps to 1e-6;
 *  - output.weight present => untied head, else output == token_embd.
 * One allocation bundle per model; qwen3_free releases it. */
#include "sp_model_abi.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct sp_arena { sp_arena_tensor *t; int n; int precision; };

const sp_arena_tensor *sp_arena_find(const sp_arena *a, const char *name) {
    if (!a || !name) return NULL;
    for (int i = 0; i < a->n; i++)
        if (strcmp(a->t[i].name, name) == 0) return &a->t[i];
    return NULL;
}

static void packed_free(sp_frob_packed_tensor *p) {
    free(p->row_prec); free(p->row_off);
    if (!(p->alias_mask & 1u)) free(p->codes);
    if (!(p->alias_mask & 2u)) free(p->row_scale);
    memset(p, 0, sizeof *p);
}

sp_arena *sp_arena_from_packed(const sp_arena_tensor *ts, int n, int precision) {
    if (!ts || n < 0 || (precision != 4 && precision != 8)) return NULL;
    sp_arena *a = (sp_arena *)calloc(1, sizeof *a);
    if (!a) return NULL;
    a->t = (sp_arena_tensor *)calloc((size_t)(n > 0 ? n : 1), sizeof(sp_arena_tensor));
    if (!a->t) { free(a); return NULL; }
    memcpy(a->t, ts, (size_t)n * sizeof *ts);
    a->n = n; a->precision = precision;
    return a;
}

void sp_arena_free(sp_arena *a) {
    if (!a) return;
    for (int i = 0; i < a->n; i++) packed_free(&a->t[i].pt);
    free(a->t); free(a);
}

/* frobenius_lift.c:193-219: Q8 row = code*scale/127; OK_Q4B row = code*f16(block
 * scale); per-row Q4 = code*scale/7.  Nibble: low = even column, sign-extended. */
int sp_frob_packed_dequant_row(const sp_frob_packed_tensor *t, int r, float *dst) {
    if (!t || !dst || r < 0 || r >= t->rows) return 1;
    const uint8_t *c = t->codes + t->row_off[r];
    if (t->row_prec[r] == 8u) {
        const float step = t->row_scale[r] / 127.0f;
        for (int i = 0; i < t->cols; i++) dst[i] = (float)(int8_t)c[i] * step;
        return 0;
    }
    for (int i = 0; i < t->cols; i++) {
        int nib = (c[i >> 1] >> ((i & 1) * 4)) & 15;
        int q = nib >= 8 ? nib - 16 : nib;
        dst[i] = t->bscale ? (float)q * sp_f16_to_f32(t->bscale[(size_t)r * (size_t)t->bs_nblk + (size_t)(i >> 5)])
                           : (float)q * (t->row_scale[r] / 7.0f);
    }
    return 0;
}

/* ---- the per-model allocation bundle ---- */
typedef struct {
    qwen3_model   qm;            /* first member: qwen3_free casts back */
    gguf_tensor  *synth;   int n_synth, cap_synth;
    qwen3_layer  *layers;
    const gguf_tensor **nsrc; float **nbuf; int n_norm, cap_norm;
    sp_arena_tensor *ents; int n_ent, cap_ent;
} model_bundle;

const float *sp_as_f32(const qwen3_model *m, const gguf_tensor *t) {
    if (!m || !t) return NULL;
    for (int i = 0; i < m->n_norm; i++) if (m->norm_src[i] == t) return m->norm_buf[i];
    return NULL;
}

void qwen3_free(qwen3_model *qm) {
    if (!qm) return;
    model_bundle *b = (model_bundle *)qm;
    sp_arena_free(qm->arena);
    if (b->ents) { for (int i = 0; i < b->n_ent; i++) packed_free(&b->ents[i].pt); free(b->ents); }
    for (int i = 0; i < b->n_norm; i++) free(b->nbuf[i]);
    free(b->nsrc); free(b->nbuf); free(b->synth); free(b->layers); free(b);
}

static gguf_tensor *synth_for(model_bundle *b, const sp_model *sm, const char *name) {
    gguf_tensor *g = &b->synth[b->n_synth++];
    snprintf(g->name, sizeof g->name, "%s", name);
    const sp_tensor_entry *e = sp_model_find_tensor(sm, name);
    if (e) {
        g->n_dims = e->n_dims;
        for (uint32_t d = 0; d < e->n_dims && d < GGUF_MAX_DIMS; d++) g->dims[d] = e->dims[d];
    }
    return g;
}

/* Packed view of one matmul weight, aliasing the mapping (sp_model_bridge.c:39-157). */
static int add_packed(model_bundle *b, const sp_model *sm, const char *name) {
    const sp_tensor_entry *e = sp_model_find_tensor(sm, name);
    if (!e || e->n_dims < 2) return 1;
    const uint64_t cols = e->dims[0], rows = e->dims[1] * (e->n_dims >= 3 ? e->dims[2] : 1u);
    if (!rows || !cols) return 1;
    const uint8_t *codes = (const uint8_t *)sp_model_tensor_data(sm, e);
    if (!codes) return 1;
    sp_frob_packed_tensor *p = &b->ents[b->n_ent].pt;
    memset(&b->ents[b->n_ent], 0, sizeof b->ents[b->n_ent]);
    snprintf(b->ents[b->n_ent].name, sizeof b->ents[b->n_ent].name, "%s", name);
    uint8_t prec; uint64_t row_bytes;
    char sib[96];
    if (e->dtype_id == (uint32_t)SP_DT_OK_Q4B) {
        const uint64_t nblk = (cols + 31u) / 32u;
        row_bytes = (cols + 1u) / 2u; prec = 4u;
        if (e->size_bytes != rows * row_bytes) return 1;
        snprintf(sib, sizeof sib, "%s.bscale", name);
        const sp_tensor_entry *se = sp_model_find_tensor(sm, sib);
        if (!se || se->dtype_id != (uint32_t)SP_DT_BLOCK_SCALE_FP16 || se->size_bytes != rows * nblk * 2u) return 1;
        p->bscale = (const uint16_t *)sp_model_tensor_data(sm, se);
        if (!p->bscale) return 1;
        p->bs_nblk = (int)nblk;
        p->alias_mask = 7u;
    } else if (e->dtype_id == (uint32_t)SP_DT_OK_Q4 || e->dtype_id == (uint32_t)SP_DT_OK_Q8) {
        prec = e->dtype_id == (uint32_t)SP_DT_OK_Q8 ? 8u : 4u;
        row_bytes = prec == 8u ? cols : (cols + 1u) / 2u;
        if (e->size_bytes != rows * row_bytes) return 1;
        snprintf(sib, sizeof sib, "%s.scale", name);
        const sp_tensor_entry *se = sp_model_find_tensor(sm, sib);
        if (!se || se->dtype_id != (uint32_t)SP_DT_FROBENIUS_SCALE_FP32 ||
            se->dims[0] != rows || se->size_bytes != rows * 4u) return 1;
        p->row_scale = (float *)(uintptr_t)sp_model_tensor_data(sm, se);
        if (!p->row_scale) return 1;
        p->alias_mask = 3u;
    } else {
        return 1;
    }
    p->rows = (int)rows; p->cols = (int)cols;
    p->codes = (uint8_t *)(uintptr_t)codes;
    p->codes_bytes = (size_t)(rows * row_bytes);
    p->row_prec = (uint8_t *)malloc((size_t)rows);
    p->row_off = (size_t *)malloc((size_t)rows * sizeof(size_t));
    if (!p->row_prec || !p->row_off) { packed_free(p); return 1; }
    for (uint64_t r = 0; r < rows; r++) { p->row_prec[r] = prec; p->row_off[r] = (size_t)(r * row_bytes); }
    b->n_ent++;
    return 0;
}

/* Owned f32 copy of a norm vector of exactly n elements (a shorter tensor would
 * let every consumer of the copy read past its end). */
static int add_norm(model_bundle *b, const sp_model *sm, const gguf_tensor *key, uint64_t n) {
    const sp_tensor_entry *e = sp_model_find_tensor(sm, key->name);
    if (!e || e->dtype_id != (uint32_t)SP_DT_F32 || !n || e->size_bytes != 4u * n) return 1;
    const void *src = sp_model_tensor_data(sm, e);
    float *dst = src ? (float *)malloc((size_t)e->size_bytes) : NULL;
    if (!dst) return 1;
    memcpy(dst, src, (size_t)e->size_bytes);
    b->nsrc[b->n_norm] = key; b->nbuf[b->n_norm] = dst; b->n_norm++;
    return 0;
}

static qwen3_model *bridge(const sp_model *sm, uint32_t want_arch, sp_arch_t arch, const char *who) {
    char err[160];
    sp_arch_info ai;
    if (!sm || sp_model_arch(sm, &ai) != SP_OK) { snprintf(err, sizeof err, "%s: null handle", who); sp_set_error(err); return NULL; }
    if (ai.arch_id != want_arch) { snprintf(err, sizeof err, "%s: wrong architecture id %u", who, ai.arch_id); sp_set_error(err); return NULL; }
    const uint32_t NL = ai.n_layers;
    if (!NL) { snprintf(err, sizeof err, "%s: zero layers", who); sp_set_error(err); return NULL; }
    const int sandwich = (arch == SP_ARCH_GEMMA3);
    uint32_t n_ff = ai.n_ff;
    if (!n_ff) {
        const sp_tensor_entry *fg = sp_model_find_tensor(sm, "blk.0.ffn_gate.weight");
        if (!fg || fg->n_dims < 2) { snprintf(err, sizeof err, "%s: n_ff unknown", who); sp_set_error(err); return NULL; }
        n_ff = (uint32_t)fg->dims[1];
    }
    const int untied = sp_model_find_tensor(sm, "output.weight") != NULL;

    model_bundle *b = (model_bundle *)calloc(1, sizeof *b);
    const int per_layer_norms = sandwich ? 6 : 4;
    if (b) {
        b->cap_synth = 3 + 13 * (int)NL;
        b->cap_norm = 1 + per_layer_norms * (int)NL;
        b->cap_ent = 2 + 7 * (int)NL;
        b->synth = (gguf_tensor *)calloc((size_t)b->cap_synth, sizeof(gguf_tensor));
        b->layers = (qwen3_layer *)calloc(NL, sizeof(qwen3_layer));
        b->nsrc = (const gguf_tensor **)calloc((size_t)b->cap_norm, sizeof(*b->nsrc));
        b->nbuf = (float **)calloc((size_t)b->cap_norm, sizeof(*b->nbuf));
        b->ents = (sp_arena_tensor *)calloc((size_t)b->cap_ent, sizeof(sp_arena_tensor));
    }
    if (!b || !b->synth || !b->layers || !b->nsrc || !b->nbuf || !b->ents) {
        snprintf(err, sizeof err, "%s: out of memory", who); sp_set_error(err);
        if (b) qwen3_free(&b->qm);
        return NULL;
    }
    qwen3_model *qm = &b->qm;
    char nm[96];
#define FAIL(what) do { snprintf(err, sizeof err, "%s: bad %s", who, (what)); sp_set_error(err); qwen3_free(qm); return NULL; } while (0)
    qm->token_embd = synth_for(b, sm, "token_embd.weight");
    if (add_packed(b, sm, "token_embd.weight")) FAIL("weight token_embd.weight");
    qm->output = qm->token_embd;
    if (untied) {
        qm->output = synth_for(b, sm, "output.weight");
        if (add_packed(b, sm, "output.weight")) FAIL("weight output.weight");
    }
    for (uint32_t L = 0; L < NL; L++) {
        qwen3_layer *ly = &b->layers[L];
        static const char *mm[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
        const gguf_tensor **mslot[7] = {&ly->attn_q, &ly->attn_k, &ly->attn_v, &ly->attn_output,
                                        &ly->ffn_gate, &ly->ffn_up, &ly->ffn_down};
        for (int k = 0; k < 7; k++) {
            snprintf(nm, sizeof nm, "blk.%u.%s.weight", L, mm[k]);
            *mslot[k] = synth_for(b, sm, nm);
            if (add_packed(b, sm, nm)) FAIL(nm);
        }
        const char *nn[6] = {"attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm",
                             "post_attention_norm", "post_ffw_norm"};
        const gguf_tensor **nslot[6] = {&ly->attn_norm, &ly->attn_q_norm, &ly->attn_k_norm,
                                        &ly->ffn_norm, &ly->post_attn_norm, &ly->post_ffw_norm};
        for (int k = 0; k < per_layer_norms; k++) {
            snprintf(nm, sizeof nm, "blk.%u.%s.weight", L, nn[k]);
            const gguf_tensor *g = synth_for(b, sm, nm);
            *nslot[k] = g;
            if (add_norm(b, sm, g, (k == 1 || k == 2) ? ai.head_dim : ai.hidden_dim)) FAIL(nm);
        }
    }
    qm->output_norm = synth_for(b, sm, "output_norm.weight");
    if (add_norm(b, sm, qm->output_norm, ai.hidden_dim)) FAIL("output_norm.weight");
#undef FAIL
    int prec = (b->n_ent > 0 && b->ents[0].pt.row_prec[0] == 4u) ? 4 : 8;
    qm->arena = sp_arena_from_packed(b->ents, b->n_ent, prec);
    if (!qm->arena) { sp_set_error("bridge: arena adoption failed"); qwen3_free(qm); return NULL; }
    free(b->ents); b->ents = NULL; b->n_ent = 0;    /* arena owns the packed buffers now */

    qwen3_config *c = &qm->cfg;
    c->arch = arch; c->n_layers = NL; c->n_embd = ai.hidden_dim; c->n_ff = n_ff;
    c->n_head = ai.n_heads; c->n_head_kv = ai.n_kv_heads; c->head_dim = ai.head_dim;
    c->n_vocab = ai.vocab_size; c->context_length = ai.max_context;
    c->sliding_window = ai.swa_window; c->rope_freq_base = ai.rope_freq_base;
    c->rms_eps = ai.rms_eps != 0.0f ? ai.rms_eps : 1e-6f;
    c->has_qk_norm = sandwich ? 1 : (ai.has_qk_norm ? 1 : 0);
    c->tied_embedding = untied ? 0 : 1;
    qm->gguf = NULL; qm->layers = b->layers; qm->synth_tensors = b->synth;
    qm->released = 1; qm->norm_src = b->nsrc; qm->norm_buf = b->nbuf; qm->n_norm = b->n_norm;
    return qm;
}

qwen3_model *sp_model_to_qwen3(const sp_model *m) {
    return bridge(m, (uint32_t)SP_ARCH_ID_QWEN3, SP_ARCH_QWEN3, "sp_model_to_qwen3");
}
qwen3_model *sp_model_to_gemma3(const sp_model *m) {
    return bridge(m, (uint32_t)SP_ARCH_ID_GEMMA3, SP_ARCH_GEMMA3, "sp_model_to_gemma3");
}
