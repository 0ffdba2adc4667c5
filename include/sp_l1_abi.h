/* sp_l1_abi.h -- the frozen Layer-1 C ABI surface this library implements,
 * restated from its documented byte layouts (same field order, widths and
 * status values, so an L2 binding compiled against the original header links
 * against this library unchanged).
 *
 * Replaces:
 *   include/sp/sp_status.h:19-60   (status codes, sp_last_error)
 *   include/sp/sp_error.h          (sp_set_error, backend-facing producer half)
 *   include/sp/sp_l1.h:55-206      (arch info, session config, session verbs)
 *   include/sp/sp_l1.h:381-427     (the section-6b persistent-KV decode table)
 *
 * Only the session/decode half of the ABI is declared here; the section-5
 * (NTT compute) and section-6 (full-forward) hooks are outside the decode path
 * and are not provided.
 */
#ifndef SPKV_L1_ABI_H
#define SPKV_L1_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: include/sp/sp_status.h:19-56 (values are wire-frozen) ---- */
typedef enum {
    SP_OK = 0,
    SP_ENOMEM = -1, SP_ECANCEL = -2, SP_EBADARG = -3, SP_EBADSTATE = -4,
    SP_EUNSUPPORTED = -5, SP_EIO = -6,
    SP_EBADFORMAT = -10, SP_EBADARCH = -11, SP_ETOKENIZER_HASH = -12, SP_EVOCAB = -13,
    SP_ESPINOR_BADBLOCK = -20, SP_EVHT2_DOMAIN = -21, SP_EMOBIUS_PERM = -22,
    SP_EOK_NORM = -23, SP_EFROBENIUS_QUANT = -24, SP_ENTT_OVERFLOW = -25,
    SP_ERING_DEGREE = -26,
    SP_ESIEVE_FULL = -30, SP_EARM_BANK_FULL = -31, SP_EDOMINANCE_CYCLE = -32,
    SP_ECONTEXT_FULL = -33,
    SP_ECUDA = -40, SP_EVULKAN = -41, SP_EHVX = -42, SP_EBACKEND_OOM = -43
} sp_status;

/* Thread-local detail string of the last failing call (include/sp/sp_status.h:60,
 * core/io_format/sp_error.c:50-63: 512-byte buffer, truncating copy). */
const char *sp_last_error(void);
void        sp_set_error(const char *msg);

/* ---- working precision: include/sp/sp_l1.h:59-65 ---- */
enum sp_precision {
    SP_PRECISION_UNSPECIFIED = 0, SP_PRECISION_F32 = 1,
    SP_PRECISION_FP16 = 2, SP_PRECISION_QF32 = 3
};

/* ---- arch info: include/sp/sp_l1.h:78-148 (192 bytes on LP64) ----
 * Stored verbatim in the .sp-model header's 256-byte arch_struct. */
typedef struct {
    uint32_t arch_id, vocab_size, hidden_dim, n_layers, n_heads, n_kv_heads,
             head_dim, max_context, swa_window;
    float    rope_freq_base;
    uint8_t  ffn_variant, norm_variant, tied_embeddings, has_qk_norm;
    uint32_t n_ff;
    float    rms_eps;
    uint32_t preferred_precision;
    /* Gemma4 tail (zero on the architectures this decode path serves) */
    uint32_t g4_hd_swa, g4_nh_swa, g4_nkv_swa;
    float    g4_rope_base_swa;
    uint32_t g4_n_embd_per_layer, g4_n_kv_from_start;
    float    g4_logit_softcap;
    uint32_t g4_swa_period;
    /* qwen35moe tail */
    uint32_t q36_full_attn_interval, q36_n_expert, q36_n_expert_used,
             q36_n_ff_exp, q36_n_ff_shexp;
    float    q36_expert_weights_scale;
    uint32_t q36_gdn_conv_k, q36_gdn_state, q36_gdn_n_k_heads,
             q36_gdn_n_v_heads, q36_gdn_inner;
    int32_t  q36_rope_sections[4];
    uint32_t q36_rope_dim;
    float    q36_rope_base;
    uint32_t q36_nextn_predict_layers;
    /* diffusion-gemma tail */
    uint32_t dg_canvas_length, dg_eb_max_steps;
    float    dg_eb_t_min, dg_eb_t_max, dg_eb_entropy_bound,
             dg_eb_stability_threshold, dg_eb_confidence_threshold;
    uint32_t dg_shift_logits;
} sp_arch_info;

/* ---- session config: include/sp/sp_l1.h:154-169 (32 bytes on LP64) ---- */
#define SP_KV_SPINOR     (1u << 0)
#define SP_KV_SPINOR_REF (1u << 1)
typedef struct {
    size_t   max_context;        /* 0 = arch default */
    int      deterministic;
    uint32_t arm_bank_kb;
    uint32_t sieve_capacity;
    uint32_t flags;
    uint32_t precision_override; /* override > arch preference > F32 */
} sp_session_config;

typedef struct sp_session sp_session;
struct sp_model;

/* ---- session verbs: include/sp/sp_l1.h:152-206 ---- */
sp_status sp_model_arch(const struct sp_model *m, sp_arch_info *out);
sp_status sp_session_create(const struct sp_model *m, const sp_session_config *cfg,
                            volatile int *cancel_flag, sp_session **out_session);
void      sp_session_destroy(sp_session *s);
uint32_t  sp_session_precision(const sp_session *s);
sp_status sp_prefill_chunk(sp_session *s, const int32_t *tokens, size_t n_tokens,
                           float *logits_last, size_t logits_capacity);
sp_status sp_decode_step(sp_session *s, int32_t token, float *logits,
                         size_t logits_capacity);
sp_status sp_session_clone(const sp_session *s, volatile int *cancel_flag, sp_session **out);
sp_status sp_session_rewind(sp_session *s, size_t n_tokens);
sp_status sp_session_position(const sp_session *s, size_t *pos_out);
const void *sp_session_qwen3_model(const sp_session *s);   /* sp_l1.h:354 */

/* ---- section 6b: persistent-KV decode dispatch (include/sp/sp_l1.h:384-427) ----
 * 48 bytes on LP64.  Each function returns 0 on success, non-zero on error with
 * the detail in sp_last_error(). */
typedef struct sp_kvdecode_handle sp_kvdecode_handle;
typedef struct sp_kvdecode_dispatch_fn {
    int  (*open)       (const void *qm_opaque, int pmax, sp_kvdecode_handle **out);
    int  (*prefill)    (sp_kvdecode_handle *h, const int32_t *tokens, int n_tok);
    int  (*decode_step)(sp_kvdecode_handle *h, int32_t token, float *logits);
    int  (*rewind)     (sp_kvdecode_handle *h, int n);
    int  (*position)   (const sp_kvdecode_handle *h);
    void (*close)      (sp_kvdecode_handle *h);
} sp_kvdecode_dispatch_fn;

sp_status sp_session_register_kvdecode_backend(sp_session *s, sp_kvdecode_handle *handle,
                                               const sp_kvdecode_dispatch_fn *dt);
sp_kvdecode_handle            *sp_session_kvdecode_backend_handle(const sp_session *s);
const sp_kvdecode_dispatch_fn *sp_session_kvdecode_backend_dt(const sp_session *s);

/* ---- this library's session-side extension (no counterpart in sp_l1.h) ----
 * Marks the registered kvdecode handle as owned by the session: it is closed by
 * sp_session_destroy and on re-registration.  Used for handles the session
 * creates itself (the fork made by sp_session_clone) and by sp_hipkv_attach. */
sp_status spx_session_own_kvdecode(sp_session *s, int owned);
/* Lifecycle routing of a registered section-6b table (default off, which is the
 * reference's contract, sp_l1.h:396-399: only sp_decode_step reaches the table).
 * On: sp_prefill_chunk runs dt->prefill plus one dt->decode_step for the last
 * position's logits, sp_session_rewind also calls dt->rewind, and
 * sp_session_clone forks the backend (spx_register_fork) into the clone, which
 * inherits the routing.  Registering another table or handle turns it off.
 * SP_EBADSTATE without a registered table.  sp_hipkv_attach turns it on. */
sp_status spx_session_route_kv_lifecycle(sp_session *s, int on);
/* The session's sp_session_config.flags (SP_KV_SPINOR, SP_KV_SPINOR_REF), for a
 * backend that stores the session's K/V itself.  0 for NULL. */
uint32_t spx_session_flags(const sp_session *s);

/* A backend that can fork its resident cache copy-on-write registers the fork
 * against its dispatch table; sp_session_clone then forks instead of dropping
 * the registration.  No counterpart in sp_l1.h (the table has no fork row). */
typedef int (*spx_fork_fn)(const sp_kvdecode_handle *parent, sp_kvdecode_handle **child);
void spx_register_fork(const sp_kvdecode_dispatch_fn *dt, spx_fork_fn fn);

/* A backend that decodes many handles in one batched step registers it against
 * its dispatch table (sp_hipkv registers sp_hipkv_decode_batch).  No counterpart
 * in sp_l1.h. */
typedef int (*spx_batch_fn)(sp_kvdecode_handle *const *hs, int n, const int32_t *tokens, float *logits,
                            int32_t *next_tokens);
void spx_register_batch(const sp_kvdecode_dispatch_fn *dt, spx_batch_fn fn);

/* sp_decode_step for n sessions at once: session i takes tokens[i] at its own
 * position; logits (NULL allowed) receives n rows of vocab_size floats
 * (logits_capacity >= n * vocab_size); next_tokens (NULL allowed) the greedy
 * token of each row (lowest index on ties).  Same guards and status codes as
 * sp_decode_step, checked for every session before any decodes; the sessions
 * must be distinct and registered on one dispatch table.  With a registered
 * batch hook the backend decodes them in one pass, otherwise one
 * decode_step each.  Every session that advanced is committed (pos + 1, token
 * in its history) even when a later one fails (SP_EBADSTATE).  No counterpart
 * in sp_l1.h: the many-sessions-per-step entry of the batched configuration. */
sp_status spx_decode_batch(sp_session *const *ss, size_t n, const int32_t *tokens, float *logits,
                           size_t logits_capacity, int32_t *next_tokens);

#if defined(__STDC_VERSION__) && __STDC_VERSION__ >= 201112L && !defined(__cplusplus)
_Static_assert(sizeof(sp_arch_info) == 192, "sp_arch_info is 192 bytes");
_Static_assert(sizeof(sp_session_config) == 32, "sp_session_config is 32 bytes");
_Static_assert(sizeof(sp_kvdecode_dispatch_fn) == 48, "sp_kvdecode_dispatch_fn is 48 bytes");
#endif

#ifdef __cplusplus
}
#endif
#endif /* SPKV_L1_ABI_H */
