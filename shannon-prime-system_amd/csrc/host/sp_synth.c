/* sp_synth.c -- OK_Q4B producer: the block quantizer and a seeded random-init
 * .sp-model writer.  The reference tree consumes OK_Q4B
 * (core/session/sp_model_bridge.c:114-148, core/frobenius/frobenius_lift.c:200-209,
 * core/forward_dispatch/forward_dispatch.c:69-85) but ships no producer.
 *
 * Weight generator (one stream over all matmul weights, in file order below):
 *   out_k   = splitmix64 output k of state `seed`      (k = 0,1,2,...)
 *   u1      = ((out_{2j} >> 11) + 1) * 2^-53  in (0,1]
 *   u2      =  (out_{2j+1} >> 11)    * 2^-53  in [0,1)
 *   r       = sqrt(-2 ln u1);  element 2j = 0.02 r cos(2 pi u2), 2j+1 = 0.02 r sin(2 pi u2)
 *   (double arithmetic, rounded once to float)
 * Element order: token_embd, [output], then per layer attn_q, attn_k, attn_v,
 * attn_output, ffn_gate, ffn_up, ffn_down; each row-major [rows][cols].
 * Norm vectors are 1.0.  File layout follows the frozen format: 512-byte header
 * (CRC-32 over [0,360)), xxh64-sorted 256-byte table, 65536-aligned data region,
 * 64-aligned tensors, tokenizer SHA-256 in the header. */
#include "sp_model_abi.h"
#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

static inline uint64_t sm64_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static inline uint64_t sm64_out(uint64_t seed, uint64_t k) {
    return sm64_mix(seed + (k + 1u) * 0x9E3779B97F4A7C15ull);
}
/* element e of the stream */
static float synth_normal(uint64_t seed, uint64_t e) {
    const uint64_t j = e >> 1;
    const double u1 = ((double)(sm64_out(seed, 2u * j) >> 11) + 1.0) * 0x1.0p-53;
    const double u2 = (double)(sm64_out(seed, 2u * j + 1u) >> 11) * 0x1.0p-53;
    const double r = sqrt(-2.0 * log(u1)), a = 6.283185307179586476925 * u2;
    return (float)(0.02 * r * ((e & 1u) ? sin(a) : cos(a)));
}

static float round_half_away(float x) { return x >= 0.0f ? floorf(x + 0.5f) : ceilf(x - 0.5f); }

void sp_q4b_quantize_row(const float *w, int cols, uint8_t *codes, uint16_t *bscale) {
    memset(codes, 0, (size_t)(cols + 1) / 2);
    for (int b0 = 0, bi = 0; b0 < cols; b0 += 32, bi++) {
        const int b1 = b0 + 32 < cols ? b0 + 32 : cols;
        float amax = 0.0f;
        for (int i = b0; i < b1; i++) { float a = fabsf(w[i]); if (a > amax) amax = a; }
        const uint16_t h = sp_f32_to_f16(amax / 7.0f);
        const float step = sp_f16_to_f32(h);
        bscale[bi] = h;
        for (int i = b0; i < b1; i++) {
            float q = step > 0.0f ? round_half_away(w[i] / step) : 0.0f;
            if (q > 7.0f) q = 7.0f;
            if (q < -7.0f) q = -7.0f;
            codes[i >> 1] |= (uint8_t)(((int)q & 15) << ((i & 1) * 4));
        }
    }
}

/* ---- tensor plan ---- */
typedef struct {
    char     name[80];
    uint32_t dtype, n_dims;
    uint64_t dims[2];
    uint64_t size, offset, hash;
    uint32_t block_size;
    int      kind;          /* 0 = q4b codes, 1 = bscale, 2 = f32 ones */
    int      weight;        /* index of the matmul weight this entry belongs to */
    uint64_t rows, cols, elem0;   /* matmul geometry + first stream element */
} plan_t;

typedef struct {
    const sp_synth_spec *sp;
    plan_t  *P; int np;
    uint8_t *data;            /* mapped data region */
    int      w;               /* weight currently generated */
    int      codes_i, scale_i;
    uint64_t spread_rows;     /* rows of the current weight with spread block scales */
    uint64_t row_next;        /* work cursor */
    int      digest_next;
    pthread_mutex_t mu;
} gen_ctx;

static void *gen_rows(void *arg) {
    gen_ctx *g = (gen_ctx *)arg;
    const plan_t *pc = &g->P[g->codes_i], *ps = &g->P[g->scale_i];
    const uint64_t cols = pc->cols, rb = (cols + 1u) / 2u, nb = (cols + 31u) / 32u;
    float *row = (float *)malloc((size_t)cols * sizeof(float));
    if (!row) return (void *)1;
    for (;;) {
        pthread_mutex_lock(&g->mu);
        uint64_t r0 = g->row_next, r1 = r0 + 64u < pc->rows ? r0 + 64u : pc->rows;
        g->row_next = r1;
        pthread_mutex_unlock(&g->mu);
        if (r0 >= pc->rows) break;
        for (uint64_t r = r0; r < r1; r++) {
            const uint64_t e0 = pc->elem0 + r * cols;
            if (!(e0 & 1u) && !(cols & 1u)) {          /* whole Box-Muller pairs: one log/sincos each */
                for (uint64_t c = 0; c < cols; c += 2) {
                    const uint64_t j = (e0 + c) >> 1;
                    const double u1 = ((double)(sm64_out(g->sp->seed, 2u * j) >> 11) + 1.0) * 0x1.0p-53;
                    const double u2 = (double)(sm64_out(g->sp->seed, 2u * j + 1u) >> 11) * 0x1.0p-53;
                    const double rr = sqrt(-2.0 * log(u1)), a = 6.283185307179586476925 * u2;
                    row[c] = (float)(0.02 * rr * cos(a));
                    row[c + 1] = (float)(0.02 * rr * sin(a));
                }
            } else {
                for (uint64_t c = 0; c < cols; c++) row[c] = synth_normal(g->sp->seed, e0 + c);
            }
            if (r < g->spread_rows)                    /* odd blocks x 2^13, even blocks x 2^-7 */
                for (uint64_t c = 0; c < cols; c++) row[c] = ldexpf(row[c], ((c / 32u) & 1u) ? 13 : -7);
            sp_q4b_quantize_row(row, (int)cols, g->data + pc->offset + r * rb,
                                (uint16_t *)(g->data + ps->offset) + r * nb);
        }
    }
    free(row);
    return NULL;
}

typedef struct { gen_ctx *g; uint8_t (*dig)[32]; } dig_arg;
static void *gen_digests(void *arg) {
    dig_arg *d = (dig_arg *)arg;
    for (;;) {
        pthread_mutex_lock(&d->g->mu);
        int i = d->g->digest_next++;
        pthread_mutex_unlock(&d->g->mu);
        if (i >= d->g->np) break;
        sp_blake3_256(d->g->data + d->g->P[i].offset, (size_t)d->g->P[i].size, d->dig[i]);
    }
    return NULL;
}

static int cmp_plan(const void *a, const void *b) {
    uint64_t x = ((const plan_t *)a)->hash, y = ((const plan_t *)b)->hash;
    return x < y ? -1 : x > y;
}

static void run_threads(void *(*fn)(void *), void *arg, int n) {
    pthread_t th[256];
    int started = 0;
    for (int i = 0; i < n && i < 256; i++)
        if (pthread_create(&th[i], NULL, fn, arg) == 0) started++;
    if (!started) fn(arg);
    for (int i = 0; i < started; i++) pthread_join(th[i], NULL);
}

sp_status sp_write_synthetic_q4b(const sp_synth_spec *sp, const char *model_path,
                                 const char *tok_path, int n_threads) {
    if (!sp || !model_path || !tok_path) { sp_set_error("sp_write_synthetic_q4b: null arg"); return SP_EBADARG; }
    if ((sp->arch_id != SP_ARCH_ID_QWEN3 && sp->arch_id != SP_ARCH_ID_GEMMA3) || !sp->n_layers ||
        !sp->hidden || !sp->n_heads || !sp->n_kv_heads || !sp->head_dim || !sp->n_ff || !sp->vocab) {
        sp_set_error("sp_write_synthetic_q4b: bad spec"); return SP_EBADARG;
    }
    if (n_threads <= 0) { long c = sysconf(_SC_NPROCESSORS_ONLN); n_threads = c > 0 ? (int)c : 1; }
    if (n_threads > 64) n_threads = 64;
    const int gemma = sp->arch_id == SP_ARCH_ID_GEMMA3;
    const uint32_t E = sp->hidden, QD = sp->n_heads * sp->head_dim, KVD = sp->n_kv_heads * sp->head_dim;

    /* ---- build the plan in generation order ---- */
    const int n_w = 1 + (sp->untied ? 1 : 0) + 7 * (int)sp->n_layers;
    const int n_n = 1 + (int)sp->n_layers * (gemma ? 6 : 4);
    const int np = 2 * n_w + n_n;
    plan_t *P = (plan_t *)calloc((size_t)np, sizeof(plan_t));
    if (!P) { sp_set_error("sp_write_synthetic_q4b: OOM"); return SP_ENOMEM; }
    int k = 0, wi = 0;
    uint64_t elem = 0;
#define ADDW(nm, R, C) do { \
        plan_t *a = &P[k++], *s = &P[k++]; \
        snprintf(a->name, sizeof a->name, "%s", (nm)); \
        a->dtype = SP_DT_OK_Q4B; a->n_dims = 2; a->dims[0] = (C); a->dims[1] = (R); \
        a->rows = (R); a->cols = (C); a->size = (uint64_t)(R) * (((C) + 1u) / 2u); \
        a->block_size = 1; a->kind = 0; a->weight = wi; a->elem0 = elem; \
        snprintf(s->name, sizeof s->name, "%s.bscale", (nm)); \
        s->dtype = SP_DT_BLOCK_SCALE_FP16; s->n_dims = 2; s->dims[0] = ((C) + 31u) / 32u; s->dims[1] = (R); \
        s->size = (uint64_t)(R) * (((C) + 31u) / 32u) * 2u; s->block_size = 2; s->kind = 1; s->weight = wi; \
        elem += (uint64_t)(R) * (C); wi++; } while (0)
#define ADDN(nm, N) do { plan_t *a = &P[k++]; snprintf(a->name, sizeof a->name, "%s", (nm)); \
        a->dtype = SP_DT_F32; a->n_dims = 1; a->dims[0] = (N); a->size = (uint64_t)(N) * 4u; \
        a->block_size = 4; a->kind = 2; a->weight = -1; } while (0)
    char nm[80];
    ADDW("token_embd.weight", sp->vocab, E);
    if (sp->untied) ADDW("output.weight", sp->vocab, E);
    for (uint32_t L = 0; L < sp->n_layers; L++) {
        snprintf(nm, sizeof nm, "blk.%u.attn_q.weight", L);      ADDW(nm, QD, E);
        snprintf(nm, sizeof nm, "blk.%u.attn_k.weight", L);      ADDW(nm, KVD, E);
        snprintf(nm, sizeof nm, "blk.%u.attn_v.weight", L);      ADDW(nm, KVD, E);
        snprintf(nm, sizeof nm, "blk.%u.attn_output.weight", L); ADDW(nm, E, QD);
        snprintf(nm, sizeof nm, "blk.%u.ffn_gate.weight", L);    ADDW(nm, sp->n_ff, E);
        snprintf(nm, sizeof nm, "blk.%u.ffn_up.weight", L);      ADDW(nm, sp->n_ff, E);
        snprintf(nm, sizeof nm, "blk.%u.ffn_down.weight", L);    ADDW(nm, E, sp->n_ff);
        snprintf(nm, sizeof nm, "blk.%u.attn_norm.weight", L);   ADDN(nm, E);
        snprintf(nm, sizeof nm, "blk.%u.attn_q_norm.weight", L); ADDN(nm, sp->head_dim);
        snprintf(nm, sizeof nm, "blk.%u.attn_k_norm.weight", L); ADDN(nm, sp->head_dim);
        snprintf(nm, sizeof nm, "blk.%u.ffn_norm.weight", L);    ADDN(nm, E);
        if (gemma) {
            snprintf(nm, sizeof nm, "blk.%u.post_attention_norm.weight", L); ADDN(nm, E);
            snprintf(nm, sizeof nm, "blk.%u.post_ffw_norm.weight", L);       ADDN(nm, E);
        }
    }
    ADDN("output_norm.weight", E);
#undef ADDW
#undef ADDN
    for (int i = 0; i < np; i++) P[i].hash = sp_xxh64(P[i].name, strlen(P[i].name), 0);
    /* weights are generated in plan order; keep that order in a side index */
    int *gen_order = (int *)malloc((size_t)np * sizeof(int));
    qsort(P, (size_t)np, sizeof(plan_t), cmp_plan);
    if (!gen_order) { free(P); sp_set_error("sp_write_synthetic_q4b: OOM"); return SP_ENOMEM; }
    const uint64_t table_off = SP_HEADER_SIZE;
    const uint64_t data_off = (table_off + (uint64_t)np * SP_TENSOR_ENTRY_SIZE + SP_DATA_REGION_ALIGN - 1u)
                              & ~(uint64_t)(SP_DATA_REGION_ALIGN - 1u);
    uint64_t cur = 0;
    for (int i = 0; i < np; i++) {
        cur = (cur + SP_TENSOR_ALIGN - 1u) & ~(uint64_t)(SP_TENSOR_ALIGN - 1u);
        P[i].offset = cur; cur += P[i].size;
    }
    const uint64_t file_size = data_off + ((cur + SP_TENSOR_ALIGN - 1u) & ~(uint64_t)(SP_TENSOR_ALIGN - 1u));

    /* ---- tokenizer: 128-byte header + 64-byte blob ---- */
    uint8_t tk[SP_TOK_HEADER_SIZE + 64];
    memset(tk, 0, sizeof tk);
    {
        sp_tok_header th; memset(&th, 0, sizeof th);
        th.magic = SP_TOK_MAGIC; th.version_major = SP_MODEL_VER_MAJOR; th.version_minor = SP_MODEL_VER_MINOR;
        th.header_size = SP_TOK_HEADER_SIZE; th.type_id = SP_TOK_BPE_GPT2; th.vocab_size = sp->vocab;
        th.bos_token = 1u; th.eos_token = 2u; th.pad_token = 0u; th.unk_token = 3u;
        th.blob_offset = SP_TOK_HEADER_SIZE; th.blob_size = 64u;
        memcpy(tk, &th, sizeof th);
        for (int i = 0; i < 64; i++) tk[SP_TOK_HEADER_SIZE + i] = (uint8_t)i;
        uint32_t c = sp_crc32(tk, SP_TOK_CRC_COVER);
        memcpy(tk + SP_TOK_CRC_COVER, &c, 4);
    }
    FILE *tf = fopen(tok_path, "wb");
    if (!tf || fwrite(tk, 1, sizeof tk, tf) != sizeof tk) {
        if (tf) fclose(tf);
        free(P); free(gen_order); sp_set_error("sp_write_synthetic_q4b: cannot write tokenizer"); return SP_EIO;
    }
    fclose(tf);

    /* ---- model file, generated in place through a shared mapping ---- */
    int fd = open(model_path, O_RDWR | O_CREAT | O_TRUNC, 0644);
    if (fd < 0 || ftruncate(fd, (off_t)file_size) != 0) {
        if (fd >= 0) close(fd);
        free(P); free(gen_order); sp_set_error("sp_write_synthetic_q4b: cannot create model file"); return SP_EIO;
    }
    uint8_t *map = (uint8_t *)mmap(NULL, (size_t)file_size, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    if (map == MAP_FAILED) {
        close(fd); free(P); free(gen_order); sp_set_error("sp_write_synthetic_q4b: mmap failed"); return SP_EIO;
    }
    gen_ctx g; memset(&g, 0, sizeof g);
    g.sp = sp; g.P = P; g.np = np; g.data = map + data_off;
    pthread_mutex_init(&g.mu, NULL);
    for (int i = 0; i < np; i++)
        if (P[i].kind == 2) { float *f = (float *)(g.data + P[i].offset); for (uint64_t j = 0; j < P[i].dims[0]; j++) f[j] = 1.0f; }
    static const char *const kinds[9] = {"token_embd.", "output.", ".attn_q.", ".attn_k.", ".attn_v.",
                                         ".attn_output.", ".ffn_gate.", ".ffn_up.", ".ffn_down."};
    for (int w = 0; w < n_w; w++) {
        g.codes_i = g.scale_i = -1;
        for (int i = 0; i < np; i++) if (P[i].weight == w) { if (P[i].kind == 0) g.codes_i = i; else g.scale_i = i; }
        const char *wn = P[g.codes_i].name;
        int kind = 0;                       /* the first two are prefixes ("attn_output." holds "output.") */
        while (kind < 9 && !(kind < 2 ? strncmp(wn, kinds[kind], strlen(kinds[kind])) == 0 : strstr(wn, kinds[kind]) != NULL)) kind++;
        g.spread_rows = (!sp->spread_mask || (kind < 9 && (sp->spread_mask >> kind) & 1u)) ? sp->spread_rows : 0;
        g.row_next = 0;
        run_threads(gen_rows, &g, n_threads);
    }
    uint8_t (*dig)[32] = (uint8_t (*)[32])calloc((size_t)np, 32);
    if (dig) { dig_arg da = {&g, dig}; g.digest_next = 0; run_threads(gen_digests, &da, n_threads); }

    for (int i = 0; i < np; i++) {
        sp_tensor_entry e; memset(&e, 0, sizeof e);
        snprintf(e.name, sizeof e.name, "%s", P[i].name);
        e.dtype_id = P[i].dtype; e.n_dims = P[i].n_dims;
        e.dims[0] = P[i].dims[0]; e.dims[1] = P[i].dims[1];
        e.offset_in_data = P[i].offset; e.size_bytes = P[i].size;
        e.block_size = P[i].block_size;
        e.block_count = (uint32_t)(P[i].size / P[i].block_size);
        if (dig) memcpy(e.blake3, dig[i], 32);
        e.name_hash = P[i].hash;
        memcpy(map + table_off + (uint64_t)i * SP_TENSOR_ENTRY_SIZE, &e, sizeof e);
    }
    sp_arch_info ai; memset(&ai, 0, sizeof ai);
    ai.arch_id = sp->arch_id; ai.vocab_size = sp->vocab; ai.hidden_dim = E; ai.n_layers = sp->n_layers;
    ai.n_heads = sp->n_heads; ai.n_kv_heads = sp->n_kv_heads; ai.head_dim = sp->head_dim;
    ai.max_context = sp->max_context; ai.swa_window = sp->swa_window; ai.rope_freq_base = sp->rope_base;
    ai.ffn_variant = (uint8_t)gemma; ai.norm_variant = (uint8_t)gemma;
    ai.tied_embeddings = (uint8_t)(sp->untied ? 0 : 1); ai.has_qk_norm = 1;
    ai.n_ff = sp->n_ff; ai.rms_eps = sp->rms_eps;
    sp_model_header h; memset(&h, 0, sizeof h);
    h.magic = SP_MODEL_MAGIC; h.version_major = SP_MODEL_VER_MAJOR; h.version_minor = SP_MODEL_VER_MINOR;
    h.header_size = SP_HEADER_SIZE; h.arch_id = sp->arch_id;
    h.arch_struct_size = (uint32_t)sizeof ai; h.arch_struct_capacity = 256u;
    memcpy(h.arch_struct, &ai, sizeof ai);
    sp_sha256(tk, sizeof tk, h.tokenizer_hash);
    h.vocab_size = sp->vocab; h.tensor_count = (uint32_t)np;
    h.tensor_table_offset = table_off; h.tensor_data_offset = data_off; h.file_size = file_size;
    h.created_unix_seconds = 1700000000ull;
    memcpy(map, &h, sizeof h);
    uint32_t crc = sp_crc32(map, SP_HEADER_CRC_COVER);
    memcpy(map + SP_HEADER_CRC_COVER, &crc, 4);

    int rc = munmap(map, (size_t)file_size);
    rc |= close(fd);
    pthread_mutex_destroy(&g.mu);
    free(dig); free(P); free(gen_order);
    if (rc) { sp_set_error("sp_write_synthetic_q4b: write-back failed"); return SP_EIO; }
    return SP_OK;
}
