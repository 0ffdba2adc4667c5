/* sp_session.c -- the L1 session verbs over a persistent-KV decode backend.
 *
 * Same argument checks, status codes, error strings and state-commit points as
 * core/session/sp_session.c (create :78-130, position :143-147, prefill
 * :154-212, decode :725-770, clone :773-816, rewind :818-824, section-6b
 * registration :909-925), with the decode itself always done by the registered
 * section-6b backend.  This library carries no host decode: an unregistered
 * session returns SP_EUNSUPPORTED from prefill/decode.  The reference's own L1
 * keeps its host path for such sessions; the dispatch table (sp_hipkv_dispatch)
 * is the drop-in and also runs under that L1 with a registrant that follows the
 * sp_l1.h:386-402 contract.
 *
 * Default routing is the reference's (sp_l1.h:396-399): sp_decode_step calls
 * dt->decode_step and nothing else calls the table -- the registrant drives
 * dt->prefill and dt->rewind itself, sp_session_rewind only moves the host
 * position and sp_session_clone leaves the clone unregistered (:792-799).
 *
 * Lifecycle routing, opt-in per session (spx_session_route_kv_lifecycle, set
 * by sp_hipkv_attach; the frozen header is unchanged):
 *  - sp_prefill_chunk: dt->prefill over tokens[0..n-2] then dt->decode_step on
 *    tokens[n-1] for the last-position logits (no O(n^2) re-forward);
 *  - sp_session_rewind: also calls dt->rewind;
 *  - sp_session_clone: when the backend registered a fork (spx_register_fork),
 *    the clone gets a copy-on-write fork of the parent's device KV, owns it and
 *    inherits the routing; otherwise it is left unregistered. */
#include "sp_l1_abi.h"
#include "sp_model_abi.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define CTX_FALLBACK 4096u

/* fork hook: a backend that supports copy-on-write forks registers it here
 * against its dispatch table (sp_hipkv does so when its library loads). */
static const sp_kvdecode_dispatch_fn *g_fork_dt[8];
static spx_fork_fn g_fork_fn[8];
void spx_register_fork(const sp_kvdecode_dispatch_fn *dt, spx_fork_fn fn) {
    for (int i = 0; i < 8; i++)
        if (!g_fork_dt[i] || g_fork_dt[i] == dt) { g_fork_dt[i] = dt; g_fork_fn[i] = fn; return; }
}
static spx_fork_fn fork_for(const sp_kvdecode_dispatch_fn *dt) {
    for (int i = 0; i < 8; i++) if (dt && g_fork_dt[i] == dt) return g_fork_fn[i];
    return NULL;
}

/* batch hook: a backend that decodes many handles in one pass registers it */
static const sp_kvdecode_dispatch_fn *g_batch_dt[8];
static spx_batch_fn g_batch_fn[8];
void spx_register_batch(const sp_kvdecode_dispatch_fn *dt, spx_batch_fn fn) {
    for (int i = 0; i < 8; i++)
        if (!g_batch_dt[i] || g_batch_dt[i] == dt) { g_batch_dt[i] = dt; g_batch_fn[i] = fn; return; }
}
static spx_batch_fn batch_for(const sp_kvdecode_dispatch_fn *dt) {
    for (int i = 0; i < 8; i++) if (dt && g_batch_dt[i] == dt) return g_batch_fn[i];
    return NULL;
}

struct sp_session {
    const sp_model     *model;
    qwen3_model        *qm;         /* borrowed from the model handle */
    sp_session_config   cfg;
    volatile int       *cancel;
    int32_t            *hist;
    size_t              hist_cap, pos;
    uint32_t            n_vocab, precision;
    sp_kvdecode_handle *kv_h;
    const sp_kvdecode_dispatch_fn *kv_dt;
    int                 kv_owned;   /* close kv_h on destroy / re-registration */
    int                 kv_route;   /* lifecycle routing: prefill / rewind / clone reach the table */
};

static int cancelled(const sp_session *s) { return s->cancel && *s->cancel; }

sp_status sp_session_create(const sp_model *m, const sp_session_config *cfg,
                            volatile int *cancel_flag, sp_session **out) {
    if (!m || !out) { sp_set_error("sp_session_create: null arg"); return SP_EBADARG; }
    *out = NULL;
    sp_arch_info ai;
    sp_model_arch(m, &ai);
    qwen3_model *qm = sp_model_borrow_qm(m);
    if (!qm) {                                   /* built once, hoisted into the model */
        if (ai.arch_id == (uint32_t)SP_ARCH_ID_GEMMA3) qm = sp_model_to_gemma3(m);
        else if (ai.arch_id == (uint32_t)SP_ARCH_ID_QWEN3) qm = sp_model_to_qwen3(m);
        else { sp_set_error("sp_session_create: architecture not served by this library"); return SP_EBADARCH; }
        if (!qm) return SP_EBADFORMAT;
        sp_model_store_qm((sp_model *)m, qm, qwen3_free);
    }
    sp_session *s = (sp_session *)calloc(1, sizeof *s);
    if (!s) { sp_set_error("sp_session_create: OOM"); return SP_ENOMEM; }
    s->model = m; s->qm = qm; s->cancel = cancel_flag; s->n_vocab = qm->cfg.n_vocab;
    if (cfg) s->cfg = *cfg;
    const uint32_t ovr = cfg ? cfg->precision_override : 0u;
    s->precision = ovr ? ovr : (ai.preferred_precision ? ai.preferred_precision : (uint32_t)SP_PRECISION_F32);
    size_t cap = s->cfg.max_context;
    if (!cap) cap = qm->cfg.context_length;
    if (!cap) cap = CTX_FALLBACK;
    s->hist_cap = cap;
    s->hist = (int32_t *)malloc(cap * sizeof(int32_t));
    if (!s->hist) { free(s); sp_set_error("sp_session_create: OOM (history)"); return SP_ENOMEM; }
    *out = s;
    return SP_OK;
}

static void drop_backend(sp_session *s) {
    if (s->kv_owned && s->kv_dt && s->kv_dt->close) s->kv_dt->close(s->kv_h);
    s->kv_h = NULL; s->kv_dt = NULL; s->kv_owned = 0; s->kv_route = 0;
}

void sp_session_destroy(sp_session *s) {
    if (!s) return;
    drop_backend(s);
    free(s->hist);
    free(s);
}

sp_status sp_session_position(const sp_session *s, size_t *pos_out) {
    if (!s || !pos_out) { sp_set_error("sp_session_position: null arg"); return SP_EBADARG; }
    *pos_out = s->pos;
    return SP_OK;
}

uint32_t sp_session_precision(const sp_session *s) {
    return s ? s->precision : (uint32_t)SP_PRECISION_UNSPECIFIED;
}

static int backend_ready(const sp_session *s, const char *who) {
    if (s->kv_dt && s->kv_dt->decode_step) return 1;
    char msg[200];
    snprintf(msg, sizeof msg, "%s: no kvdecode backend registered (this library has no host decode; "
             "attach the HIP backend with sp_hipkv_attach)", who);
    sp_set_error(msg);
    return 0;
}

sp_status sp_prefill_chunk(sp_session *s, const int32_t *tokens, size_t n_tokens,
                           float *logits_last, size_t logits_capacity) {
    if (!s || !tokens || !logits_last) { sp_set_error("sp_prefill_chunk: null arg"); return SP_EBADARG; }
    if (n_tokens == 0) { sp_set_error("sp_prefill_chunk: n_tokens == 0"); return SP_EBADARG; }
    if (logits_capacity < s->n_vocab) { sp_set_error("sp_prefill_chunk: logits_capacity < vocab_size"); return SP_EBADARG; }
    if (n_tokens > s->hist_cap - s->pos) { sp_set_error("sp_prefill_chunk: context full"); return SP_ECONTEXT_FULL; }
    if (cancelled(s)) return SP_ECANCEL;
    if (!backend_ready(s, "sp_prefill_chunk")) return SP_EUNSUPPORTED;
    if (!s->kv_route) {
        /* the reference prefills on the host (a full forward); under the
         * sp_l1.h contract the registrant feeds dt->prefill itself */
        sp_set_error("sp_prefill_chunk: this library has no host prefill; drive dt->prefill from the "
                     "registrant or enable lifecycle routing (spx_session_route_kv_lifecycle / sp_hipkv_attach)");
        return SP_EUNSUPPORTED;
    }
    if (n_tokens - 1u > (size_t)0x7FFFFFFF) { sp_set_error("sp_prefill_chunk: chunk too large"); return SP_EBADARG; }

    memcpy(s->hist + s->pos, tokens, n_tokens * sizeof(int32_t));
    int rc = 0;
    if (n_tokens > 1) {
        if (s->kv_dt->prefill) {
            rc = s->kv_dt->prefill(s->kv_h, tokens, (int)(n_tokens - 1u));
        } else {                            /* table without prefill: step through */
            for (size_t i = 0; i + 1 < n_tokens && !rc; i++)
                rc = s->kv_dt->decode_step(s->kv_h, tokens[i], logits_last);
        }
    }
    int done_prefix = !rc;
    if (!rc) rc = s->kv_dt->decode_step(s->kv_h, tokens[n_tokens - 1u], logits_last);
    if (rc) {
        /* keep the backend's position in step with the session's */
        if (done_prefix && n_tokens > 1 && s->kv_dt->prefill && s->kv_dt->rewind)
            (void)s->kv_dt->rewind(s->kv_h, (int)(n_tokens - 1u));
        const char *prev = sp_last_error();
        if (!prev || !prev[0]) sp_set_error("sp_prefill_chunk: kvdecode backend failed");
        return SP_EBADSTATE;
    }
    s->pos += n_tokens;                     /* commit only after success */
    return SP_OK;
}

sp_status sp_decode_step(sp_session *s, int32_t token, float *logits, size_t logits_capacity) {
    if (!s || !logits) { sp_set_error("sp_decode_step: null arg"); return SP_EBADARG; }
    if (logits_capacity < s->n_vocab) { sp_set_error("sp_decode_step: logits_capacity < vocab_size"); return SP_EBADARG; }
    if (s->pos >= s->hist_cap) { sp_set_error("sp_decode_step: context full"); return SP_ECONTEXT_FULL; }
    if (cancelled(s)) return SP_ECANCEL;
    if (!backend_ready(s, "sp_decode_step")) return SP_EUNSUPPORTED;
    s->hist[s->pos] = token;
    if (s->kv_dt->decode_step(s->kv_h, token, logits)) {
        sp_set_error("sp_decode_step: kvdecode backend step failed");
        return SP_EBADSTATE;
    }
    s->pos++;
    return SP_OK;
}

sp_status spx_decode_batch(sp_session *const *ss, size_t n, const int32_t *tokens, float *logits,
                           size_t logits_capacity, int32_t *next_tokens) {
    if (!ss || !tokens || n == 0) { sp_set_error("spx_decode_batch: null arg"); return SP_EBADARG; }
    if (n > 0x7FFFFFFF) { sp_set_error("spx_decode_batch: too many sessions"); return SP_EBADARG; }
    const sp_kvdecode_dispatch_fn *dt = ss[0] ? ss[0]->kv_dt : NULL;
    for (size_t i = 0; i < n; i++) {            /* every guard before any decode */
        sp_session *s = ss[i];
        if (!s) { sp_set_error("spx_decode_batch: null session"); return SP_EBADARG; }
        if (logits && logits_capacity / n < s->n_vocab) {
            sp_set_error("spx_decode_batch: logits_capacity < n * vocab_size"); return SP_EBADARG;
        }
        if (s->pos >= s->hist_cap) { sp_set_error("spx_decode_batch: context full"); return SP_ECONTEXT_FULL; }
        if (cancelled(s)) return SP_ECANCEL;
        if (!backend_ready(s, "spx_decode_batch")) return SP_EUNSUPPORTED;
        if (s->kv_dt != dt || s->model != ss[0]->model) {
            sp_set_error("spx_decode_batch: sessions use different models or backends"); return SP_EBADARG;
        }
        for (size_t j = 0; j < i; j++)
            if (ss[j] == s) { sp_set_error("spx_decode_batch: a session appears twice"); return SP_EBADARG; }
    }
    const uint32_t V = ss[0]->n_vocab;
    spx_batch_fn fn = batch_for(dt);
    int rc = 0;
    if (fn) {
        sp_kvdecode_handle **hs = (sp_kvdecode_handle **)malloc(n * sizeof *hs);
        if (!hs) { sp_set_error("spx_decode_batch: out of memory"); return SP_ENOMEM; }
        for (size_t i = 0; i < n; i++) hs[i] = ss[i]->kv_h;
        rc = fn(hs, (int)n, tokens, logits, next_tokens);
        free(hs);
    } else {                                    /* no batch hook: one step each */
        float *row = logits ? NULL : (float *)malloc((size_t)V * sizeof(float));
        if (!logits && !row) { sp_set_error("spx_decode_batch: out of memory"); return SP_ENOMEM; }
        for (size_t i = 0; i < n && !rc; i++) {
            float *lg = logits ? logits + i * V : row;
            rc = dt->decode_step(ss[i]->kv_h, tokens[i], lg);
            if (!rc && next_tokens) {
                uint32_t best = 0;
                for (uint32_t k = 1; k < V; k++) if (lg[k] > lg[best]) best = k;
                next_tokens[i] = (int32_t)best;
            }
        }
        free(row);
    }
    /* commit what the backend advanced (all of them on success) */
    for (size_t i = 0; i < n; i++) {
        sp_session *s = ss[i];
        if (rc && (!dt->position || dt->position(s->kv_h) != (int)s->pos + 1)) continue;
        s->hist[s->pos] = tokens[i];
        s->pos++;
    }
    if (rc) {
        const char *prev = sp_last_error();
        if (!prev || !prev[0]) sp_set_error("spx_decode_batch: kvdecode backend batch step failed");
        return SP_EBADSTATE;
    }
    return SP_OK;
}

sp_status sp_session_clone(const sp_session *s, volatile int *cancel_flag, sp_session **out) {
    if (!s || !out) { sp_set_error("sp_session_clone: null arg"); return SP_EBADARG; }
    *out = NULL;
    sp_status st = sp_session_create(s->model, &s->cfg, cancel_flag, out);
    if (st != SP_OK) return st;
    sp_session *c = *out;
    memcpy(c->hist, s->hist, s->pos * sizeof(int32_t));
    c->pos = s->pos;
    spx_fork_fn fk = s->kv_route ? fork_for(s->kv_dt) : NULL;
    if (fk && s->kv_h) {
        sp_kvdecode_handle *child = NULL;
        if (fk(s->kv_h, &child) || !child) {
            sp_session_destroy(c); *out = NULL;
            const char *prev = sp_last_error();
            if (!prev || !prev[0]) sp_set_error("sp_session_clone: backend fork failed");
            return SP_EBACKEND_OOM;
        }
        c->kv_h = child; c->kv_dt = s->kv_dt; c->kv_owned = 1; c->kv_route = 1;
    }
    return SP_OK;
}

sp_status sp_session_rewind(sp_session *s, size_t n_tokens) {
    if (!s) { sp_set_error("sp_session_rewind: null handle"); return SP_EBADARG; }
    if (n_tokens > s->pos) { sp_set_error("sp_session_rewind: n_tokens > position"); return SP_EBADARG; }
    if (s->kv_route && s->kv_dt && s->kv_dt->rewind && n_tokens) {
        if (n_tokens > (size_t)0x7FFFFFFF || s->kv_dt->rewind(s->kv_h, (int)n_tokens)) {
            const char *prev = sp_last_error();
            if (!prev || !prev[0]) sp_set_error("sp_session_rewind: kvdecode backend rewind failed");
            return SP_EBADSTATE;
        }
    }
    s->pos -= n_tokens;
    return SP_OK;
}

sp_status sp_session_register_kvdecode_backend(sp_session *s, sp_kvdecode_handle *handle,
                                               const sp_kvdecode_dispatch_fn *dt) {
    if (!s) { sp_set_error("sp_session_register_kvdecode_backend: null session"); return SP_EBADARG; }
    /* an owned backend that is replaced or unregistered is closed here */
    if (s->kv_owned && (s->kv_h != handle || !dt)) drop_backend(s);
    if (s->kv_dt != dt || s->kv_h != handle) s->kv_route = 0;   /* a new registration starts on default routing */
    /* both fields are stored as given, as the reference does (sp_session.c:913-914):
     * a NULL dt unregisters (sp_decode_step no longer routes) while the handle
     * readback still returns the handle passed */
    s->kv_h = handle; s->kv_dt = dt;
    if (!dt) { s->kv_owned = 0; s->kv_route = 0; }
    return SP_OK;
}

sp_status spx_session_own_kvdecode(sp_session *s, int owned) {
    if (!s) { sp_set_error("spx_session_own_kvdecode: null session"); return SP_EBADARG; }
    s->kv_owned = (owned && s->kv_dt) ? 1 : 0;
    return SP_OK;
}

sp_status spx_session_route_kv_lifecycle(sp_session *s, int on) {
    if (!s) { sp_set_error("spx_session_route_kv_lifecycle: null session"); return SP_EBADARG; }
    if (on && !s->kv_dt) { sp_set_error("spx_session_route_kv_lifecycle: no kvdecode backend registered"); return SP_EBADSTATE; }
    s->kv_route = on ? 1 : 0;
    return SP_OK;
}

uint32_t spx_session_flags(const sp_session *s) { return s ? s->cfg.flags : 0u; }
sp_kvdecode_handle *sp_session_kvdecode_backend_handle(const sp_session *s) { return s ? s->kv_h : NULL; }
const sp_kvdecode_dispatch_fn *sp_session_kvdecode_backend_dt(const sp_session *s) { return s ? s->kv_dt : NULL; }
const void *sp_session_qwen3_model(const sp_session *s) { return s ? (const void *)s->qm : NULL; }
