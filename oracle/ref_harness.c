/* ref_harness.c -- TEST INFRASTRUCTURE: a thin driver linked into
 * oracle/_ref/libspref.so (the compiled reference) so tests can run the
 * reference's own session decode on a given .sp-model.  Calls only the
 * reference's public API (include/sp/sp_l1.h, sp_model.h, qwen3_fixture.h). */
#include "sp/sp_l1.h"
#include "sp/sp_model.h"
#include "sp/sp_hash.h"
#include "sp/model.h"
#include "qwen3_fixture.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int argmax_lowest(const float *v, int n) {
    int a = 0;
    for (int j = 1; j < n; j++) if (v[j] > v[a]) a = j;
    return a;
}

/* prefill `prompt`, then n_gen decode steps; step k feeds forced[k] when forced
 * is non-NULL, else the greedy argmax of the previous logits.  Writes the
 * prefill logits (V), every decode step's logits (n_gen x V) and the fed tokens. */
int refh_decode_flags(const char *spm, const char *spt, const int32_t *prompt, int n_prompt,
                      int n_gen, const int32_t *forced, float *prefill_logits, float *logits,
                      int32_t *fed, uint32_t flags);
int refh_decode(const char *spm, const char *spt, const int32_t *prompt, int n_prompt,
                int n_gen, const int32_t *forced, float *prefill_logits, float *logits,
                int32_t *fed) {
    return refh_decode_flags(spm, spt, prompt, n_prompt, n_gen, forced, prefill_logits, logits, fed, 0u);
}
/* the same with sp_session_config.flags (SP_KV_SPINOR / SP_KV_SPINOR_REF) */
int refh_decode_flags(const char *spm, const char *spt, const int32_t *prompt, int n_prompt,
                      int n_gen, const int32_t *forced, float *prefill_logits, float *logits,
                      int32_t *fed, uint32_t flags) {
    sp_model *m = NULL;
    if (sp_model_load(spm, spt, &m) != SP_OK) return -1;
    sp_arch_info ai; sp_model_arch(m, &ai);
    const int V = (int)ai.vocab_size;
    sp_session_config cfg; memset(&cfg, 0, sizeof cfg);
    cfg.deterministic = 1; cfg.max_context = (size_t)(n_prompt + n_gen + 1);
    cfg.flags = flags;
    sp_session *s = NULL;
    int rc = -2;
    if (sp_session_create(m, &cfg, NULL, &s) != SP_OK) goto out;
    rc = -3;
    if (sp_prefill_chunk(s, prompt, (size_t)n_prompt, prefill_logits, (size_t)V) != SP_OK) goto out;
    int t = argmax_lowest(prefill_logits, V);
    for (int k = 0; k < n_gen; k++) {
        if (forced) t = forced[k];
        fed[k] = t;
        rc = -4 - k;
        if (sp_decode_step(s, t, logits + (size_t)k * V, (size_t)V) != SP_OK) goto out;
        t = argmax_lowest(logits + (size_t)k * V, V);
    }
    rc = 0;
out:
    if (s) sp_session_destroy(s);
    sp_model_unload(m);
    return rc;
}

/* the reference's own qwen3 session fixture: SHA-256 of the .sp-model bytes */
int refh_qwen3_fixture_sha(uint8_t out[32], size_t *len) {
    uint8_t *mb = NULL, *tb = NULL;
    sp_qwen3_fixture_info info;
    if (sp_qwen3_fixture_build(&mb, &tb, &info)) return 1;
    sp_sha256(mb, info.model_len, out);
    *len = info.model_len;
    free(mb); free(tb);
    return 0;
}

/* SP_RECALL_KVSEL for the recall calls below (0: off, the default) */
static int g_refh_kvsel = 0;
void refh_set_kvsel(int on) { g_refh_kvsel = on ? 1 : 0; }

/* The reference's decode-path perplexity (core/forward/decode.c
 * qwen3_ppl_decode) on a Qwen3 .sp-model with the ARM recall knobs
 * SP_RECALL_B / _W / _SINK / _R set for the call (B = 0: recall off); the
 * other knobs are cleared.  Returns 0 and *ppl on success. */
int refh_ppl_recall(const char *spm, const char *spt, const int32_t *toks, int n, int n_warm,
                    int B, int W, int sink, int r, double *ppl) {
    static const char *off[] = {"SP_RING2", "SP_RING2_DISK", "SP_RECALL_DECODE_ONLY", "SP_RECALL_FUSE", "SP_NTT_KV",
                                "SP_RECALL_BITS", "SP_RECALL_KVSEL", "SP_REPLAY", "SP_ENGINE_NTT_ATTN",
                                "SP_KV_SPINOR", "SP_KV_SPINOR_REF"};
    for (size_t i = 0; i < sizeof off / sizeof off[0]; i++) unsetenv(off[i]);
    char b[32];
    snprintf(b, sizeof b, "%d", B); setenv("SP_RECALL_B", b, 1);
    snprintf(b, sizeof b, "%d", W); setenv("SP_RECALL_W", b, 1);
    snprintf(b, sizeof b, "%d", sink); setenv("SP_RECALL_SINK", b, 1);
    snprintf(b, sizeof b, "%d", r); setenv("SP_RECALL_R", b, 1);
    if (g_refh_kvsel) setenv("SP_RECALL_KVSEL", "1", 1);
    sp_model *m = NULL;
    if (sp_model_load(spm, spt, &m) != SP_OK) return -1;
    struct qwen3_model *qm = sp_model_to_qwen3(m);
    int rc = -2;
    if (qm) {
        int32_t *t = (int32_t *)malloc((size_t)n * sizeof(int32_t));
        memcpy(t, toks, (size_t)n * sizeof(int32_t));
        rc = qwen3_ppl_decode(qm, t, n, n_warm, ppl, NULL) ? -3 : 0;
        free(t);
        qwen3_free(qm);
    }
    sp_model_unload(m);
    unsetenv("SP_RECALL_B"); unsetenv("SP_RECALL_KVSEL");
    return rc;
}

/* qwen3_generate_kv (decode.c:909-912) greedy over n_gen tokens after the
 * prompt with the ARM recall knobs; decode_only sets SP_RECALL_DECODE_ONLY=1
 * (dense prompt, the router at the generated positions).  seq: n_prompt +
 * n_gen ints, the prompt in front; returns the number generated or < 0. */
int refh_generate_recall(const char *spm, const char *spt, int32_t *seq, int n_prompt, int n_gen,
                         int B, int W, int sink, int r, int decode_only) {
    static const char *off[] = {"SP_RING2", "SP_RING2_DISK", "SP_RECALL_DECODE_ONLY", "SP_RECALL_FUSE", "SP_NTT_KV",
                                "SP_RECALL_BITS", "SP_RECALL_KVSEL", "SP_REPLAY", "SP_ENGINE_NTT_ATTN",
                                "SP_KV_SPINOR", "SP_KV_SPINOR_REF"};
    for (size_t i = 0; i < sizeof off / sizeof off[0]; i++) unsetenv(off[i]);
    char b[32];
    snprintf(b, sizeof b, "%d", B); setenv("SP_RECALL_B", b, 1);
    snprintf(b, sizeof b, "%d", W); setenv("SP_RECALL_W", b, 1);
    snprintf(b, sizeof b, "%d", sink); setenv("SP_RECALL_SINK", b, 1);
    snprintf(b, sizeof b, "%d", r); setenv("SP_RECALL_R", b, 1);
    if (decode_only) setenv("SP_RECALL_DECODE_ONLY", "1", 1);
    if (g_refh_kvsel) setenv("SP_RECALL_KVSEL", "1", 1);
    sp_model *m = NULL;
    if (sp_model_load(spm, spt, &m) != SP_OK) return -1;
    struct qwen3_model *qm = sp_model_to_qwen3(m);
    int rc = -2;
    if (qm) {
        rc = qwen3_generate_kv(qm, seq, n_prompt, n_gen, -1);
        qwen3_free(qm);
    }
    sp_model_unload(m);
    unsetenv("SP_RECALL_B"); unsetenv("SP_RECALL_DECODE_ONLY"); unsetenv("SP_RECALL_KVSEL");
    return rc;
}
