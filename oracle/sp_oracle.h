/* sp_oracle.h -- TEST INFRASTRUCTURE ONLY.  A scalar CPU restatement of the
 * reference's session-resident KV decode, used as the checker by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.  Nothing in the
 * product library links, loads or calls this code.
 *
 * Float mode restates core/session/sp_session.c kv_step (:274-363) and
 * kv_step_gemma3 (:380-464) with the OK_Q4B arena matmul
 * (core/forward_dispatch/forward_dispatch.c:59-98) and the scalar kernels
 * (core/forward_kernels/forward_kernels.c:11-81), in the same operation order,
 * so that it is bit-identical to the compiled reference on the same inputs.
 *
 * Exact mode is the build-defined integer decode (islands restated from
 * core/exact_islands/exact_islands.c:21-124 plus the integer GEMV, CORDIC RoPE
 * and integer attention specified in oracle/sp_oracle.c). */
#ifndef SP_ORACLE_H
#define SP_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_model orc_model;
typedef struct orc_sess  orc_sess;

enum { ORC_FLOAT = 0, ORC_EXACT = 1 };

/* threads of the row-parallel loops (GEMV rows, attention heads); results are
 * the same for every count (each row keeps its scalar order); default 1 */
void orc_set_threads(int n);
int  orc_threads(void);

orc_model *orc_model_load(const char *spm_path);
void       orc_model_free(orc_model *m);
/* arch_id, vocab, hidden, n_layers, n_heads, n_kv_heads, head_dim, n_ff, swa */
void       orc_model_dims(const orc_model *m, uint32_t out[9]);

orc_sess *orc_sess_new(orc_model *m, int max_ctx, int mode);
/* kv_flags as sp_session_config.flags (include/sp/sp_l1.h:156-157): either bit
 * passes every stored K/V head through the Spinor-63 codec */
enum { ORC_KV_SPINOR = 1u << 0, ORC_KV_SPINOR_REF = 1u << 1 };
orc_sess *orc_sess_new_kv(orc_model *m, int max_ctx, int mode, uint32_t kv_flags);
void      orc_sess_free(orc_sess *s);
/* one token at the session position (kv_step semantics); logits may be NULL */
int       orc_step(orc_sess *s, int32_t tok, float *logits);
int       orc_rewind(orc_sess *s, int n);
int       orc_pos(const orc_sess *s);
orc_sess *orc_clone(const orc_sess *s);
/* K/V rows of one layer for positions [p0, p0+n): KVD floats per position */
int       orc_kv_get(const orc_sess *s, int layer, int p0, int n, float *k, float *v);
int       orc_kv_set(orc_sess *s, int layer, int p0, int n, const float *k, const float *v);
int       orc_set_pos(orc_sess *s, int pos);
/* on: steps leave the K/V rows at their position as orc_kv_set wrote them (the
 * attention then reads caller-given rows: a float-mode check of a lossy K/V
 * codec against the codes another implementation chose) */
void      orc_set_kv_forced(orc_sess *s, int on);

/* ---- unit kernels (float mode: reference order) ---- */
float orc_f16_to_f32(uint16_t h);
void  orc_rmsnorm(const float *x, const float *w, int n, float eps, float *out);
void  orc_rope_neox(float *v, int d, int p, float base);
void  orc_attn_head(const float *qh, const float *KC, const float *VC, int pos, int KVD,
                    int kvh, int HD, float ascale, int win, float *sc, float *out);
int   orc_q4b_gemv(const uint8_t *codes, const uint16_t *bscale, int rows, int cols,
                   const float *x, float *y);
/* ---- Spinor-63 KV block codec (core/vht2/, include/sp/spinor_block.h) ---- */
uint8_t orc_crc8(const uint8_t *d, int n);
int   orc_spinor_blocks_for(int k);
void  orc_spinor_encode(const float *vec, int k, uint8_t blk[63]);
int   orc_spinor_decode(const uint8_t blk[63], float *vec, int k);
void  orc_spinor_encode_vec(const float *vec, int k, uint8_t *blocks);
int   orc_spinor_decode_vec(const uint8_t *blocks, int k, float *vec);
/* ---- exact islands (reference arithmetic) ---- */
void  orc_rmsnorm_exact(const float *x, const float *w, int n, float *out);
void  orc_softmax_exact(const float *z, int m, double *p);
void  orc_gelu_exact(const float *x, int n, float *out);
/* ---- build-defined exact primitives ---- */
void  orc_cordic_sincos(int64_t theta_q60, int32_t *cos_q30, int32_t *sin_q30);
void  orc_rope_exact(float *v, int d, int p, float base);
int   orc_q4b_gemv_exact(const uint8_t *codes, const uint16_t *bscale, int rows, int cols,
                         const float *x, float *y);
void  orc_silu_exact(const float *x, int n, float *out);
int64_t orc_rope_freq_q60(float base, int i, int d);
/* exact-mode attention of one q head over [s0, pos] (int32 K/V slabs, KVD per
 * position): qi = rne(q 2^16), int64 dots, the island softmax on the 2^14
 * grid, Q22 weights, int128 V-sum, one RNE division per output */
void  orc_attn_head_exact(const float *qh, const int32_t *KC, const int32_t *VC, int pos, int KVD, int kvh,
                          int HD, float ascale, int win, float *out);
/* RNE(num / (den * 2^k)) for a 128-bit num = num_hi * 2^64 + num_lo, den > 0 */
float orc_i128_div_to_float(int64_t num_hi, uint64_t num_lo, int64_t den, int k);
/* exact-mode V code clamp(rne(v 2^16), +-(2^23-1)); *clamped = 1 when clamped */
int32_t orc_vq_of(float v, int *clamped);
/* ---- ARM recall router (core/arm/arm.c, include/sp/arm.h) ---- */
/* R[r*hd] = +-1 from the frozen SplitMix64 seed */
void  orc_arm_build_R(signed char *R, int r, int hd);
/* proj[p] = sum_d R[p,d] * vec[d], sequential float */
void  orc_arm_project(const signed char *R, int r, int hd, const float *vec, float *proj);
/* one head's recall set (sp_arm_select semantics): pk = the layer's sidecar for
 * kv head kvh (stride nkv*r floats per position), cand = (pos+1) {float, int}
 * scratch; returns the set size, ri in the reference's order */
int   orc_arm_select(const signed char *R, int r, int hd, const float *qh, const float *pk, int nkv,
                     int B, int W, int sink, int pos, void *cand, int *ri);
/* Recall decode (core/forward/decode.c:740-790 with SP_RECALL_B/W/SINK/R):
 * every full-attention layer attends each q head's recall set; the K
 * projection sidecar is kept per position.  B = 0 switches it off.  Before the
 * first token. */
int   orc_set_recall(orc_sess *s, int B, int W, int sink, int r);
/* Dense recall steps (SP_RECALL_DECODE_ONLY=1 during the prompt, decode.c:561:
 * the effective budget is 0, so each q head attends every position through the
 * identity list) while on; the sidecar is still written.  Off by default. */
void  orc_set_recall_dense(orc_sess *s, int on);
int   orc_set_recall_kvsel(orc_sess *s, int on);     /* SP_RECALL_KVSEL */
/* sidecar rows [p0, p0+n) of a layer: NKV*r floats per position */
int   orc_recall_sidecar(const orc_sess *s, int layer, int p0, int n, float *out);
/* overwrite sidecar rows [p0, p0+n) of a layer (a state loaded from elsewhere) */
int   orc_recall_sidecar_set(orc_sess *s, int layer, int p0, int n, const float *in);
/* V heads this session stored with a clamped element (exact mode) */
int   orc_v_clamps(const orc_sess *s);

#ifdef __cplusplus
}
#endif
#endif
