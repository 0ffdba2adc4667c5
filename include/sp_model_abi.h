/* sp_model_abi.h -- the .sp-model on-disk format and the in-memory model
 * representation that the section-6b `open(qm_opaque, ...)` receives, restated
 * from their frozen byte layouts.
 *
 * Replaces:
 *   include/sp/sp_model.h:28-195     (format constants, dtype/arch enums, the
 *                                    512/256/128-byte structs, loader + bridge API)
 *   include/sp/gguf.h:44-52          (gguf_tensor: the name/dims carrier)
 *   include/sp/model.h:24-182        (qwen3_config / qwen3_layer / qwen3_model)
 *   include/sp/frobenius_lift.h:160-173, 196 (packed tensor layout v2, OK_Q4B)
 *   include/sp/arena.h:31-65         (named packed-tensor set)
 *   include/sp/forward_dispatch.h:44 (sp_as_f32)
 *   include/sp/weight_dtype.h        (sp_f16_to_f32 / sp_f32_to_f16)
 *   include/sp/sp_hash.h:31-51       (CRC-32, SHA-256, XXH64, digest placeholder)
 *
 * Layouts are byte-identical to the originals (sizes asserted below); the code
 * behind them in this library is written fresh.
 */
#ifndef SPKV_MODEL_ABI_H
#define SPKV_MODEL_ABI_H

#include <stddef.h>
#include <stdint.h>
#include "sp_l1_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- format constants: include/sp/sp_model.h:29-40 ---- */
#define SP_MODEL_MAGIC        0x444D5053u  /* "SPMD" */
#define SP_TOK_MAGIC          0x4B545053u  /* "SPTK" */
#define SP_MODEL_VER_MAJOR    0u
#define SP_MODEL_VER_MINOR    1u
#define SP_HEADER_SIZE        512u
#define SP_TOK_HEADER_SIZE    128u
#define SP_TENSOR_ENTRY_SIZE  256u
#define SP_DATA_REGION_ALIGN  65536u
#define SP_TENSOR_ALIGN       64u
#define SP_HEADER_CRC_COVER   360u
#define SP_TOK_CRC_COVER      52u
#define SP_SPINOR_SENTINEL    0xA5u

/* dtype ids: include/sp/sp_model.h:43-57 */
typedef enum {
    SP_DT_F32 = 1, SP_DT_F16 = 2, SP_DT_BF16 = 3,
    SP_DT_OK_Q8 = 10, SP_DT_OK_Q4 = 11, SP_DT_FROBENIUS_SCALE_FP32 = 12,
    SP_DT_OK_Q4B = 13, SP_DT_BLOCK_SCALE_FP16 = 14,
    SP_DT_SPINOR63 = 20, SP_DT_RING_RESIDUE_CRT_30_30 = 30, SP_DT_OK_INTEGER = 31
} sp_dtype_id;

/* wire arch ids: include/sp/sp_model.h:60-70 */
typedef enum {
    SP_ARCH_ID_LLAMA3 = 1, SP_ARCH_ID_QWEN3 = 2, SP_ARCH_ID_GEMMA3 = 3,
    SP_ARCH_ID_DEEPSEEK_V4 = 4, SP_ARCH_ID_QWEN25 = 6, SP_ARCH_ID_GEMMA4 = 7,
    SP_ARCH_ID_QWEN36 = 8, SP_ARCH_ID_DIFFUSION_GEMMA = 9
} sp_arch_id;

/* tokenizer family: include/sp/sp_model.h:75-79 */
typedef enum {
    SP_TOK_SENTENCEPIECE = 0, SP_TOK_BPE_LLAMA3 = 1, SP_TOK_BPE_GPT2 = 2,
    SP_TOK_TIKTOKEN_O200K = 3, SP_TOK_GEMMA4_BPE = 4
} sp_tok_type_id;

#pragma pack(push, 1)
typedef struct {                       /* include/sp/sp_model.h:84-103 */
    uint32_t magic;
    uint16_t version_major, version_minor;
    uint32_t header_size, arch_id, arch_struct_size, arch_struct_capacity;
    uint8_t  arch_struct[256];
    uint8_t  tokenizer_hash[32];
    uint32_t vocab_size, tensor_count;
    uint64_t tensor_table_offset, tensor_data_offset, file_size,
             created_unix_seconds, transcoded_from;
    uint32_t header_crc32;
    uint8_t  reserved[148];
} sp_model_header;

typedef struct {                       /* include/sp/sp_model.h:106-118 */
    char     name[80];
    uint32_t dtype_id, n_dims;
    uint64_t dims[8];
    uint64_t offset_in_data, size_bytes;
    uint32_t block_size, block_count;
    uint8_t  blake3[32];
    uint64_t name_hash;
    uint8_t  reserved[40];
} sp_tensor_entry;

typedef struct {                       /* include/sp/sp_model.h:121-136 */
    uint32_t magic;
    uint16_t version_major, version_minor;
    uint32_t header_size, type_id, vocab_size, bos_token, eos_token, pad_token, unk_token;
    uint64_t blob_offset, blob_size;
    uint32_t header_crc32;
    uint8_t  reserved[72];
} sp_tok_header;
#pragma pack(pop)

typedef struct sp_model sp_model;

/* loader: include/sp/sp_model.h:150-169 */
sp_status sp_model_load(const char *sp_model_path, const char *sp_tokenizer_path, sp_model **out);
void      sp_model_unload(sp_model *m);
const sp_model_header *sp_model_get_header(const sp_model *m);
uint32_t               sp_model_tensor_count(const sp_model *m);
const sp_tensor_entry *sp_model_tensor_at(const sp_model *m, uint32_t i);
const sp_tensor_entry *sp_model_find_tensor(const sp_model *m, const char *name);
const void            *sp_model_tensor_data(const sp_model *m, const sp_tensor_entry *e);
const void            *sp_model_tokenizer_blob(const sp_model *m, uint64_t *size_out);

/* ---- in-memory model (what section-6b open() receives) ---- */
#define GGUF_NAME_MAX  256
#define GGUF_MAX_DIMS  4
typedef struct {                       /* include/sp/gguf.h:44-52, 328 bytes */
    char     name[GGUF_NAME_MAX];
    uint32_t n_dims;
    uint64_t dims[GGUF_MAX_DIMS];
    uint32_t type;
    uint64_t offset, n_elements, nbytes;
} gguf_tensor;

typedef enum { SP_ARCH_QWEN3 = 0, SP_ARCH_GEMMA3 = 1, SP_ARCH_QWEN25 = 2, SP_ARCH_GEMMA4 = 3,
               SP_ARCH_QWEN36 = 4, SP_ARCH_DIFFUSION_GEMMA = 5 } sp_arch_t;   /* model.h:24-26 */

typedef struct {                       /* include/sp/model.h:28-84, 164 bytes */
    sp_arch_t arch;
    uint32_t n_layers, n_embd, n_ff, n_head, n_head_kv, head_dim, n_vocab,
             context_length, sliding_window;
    float    rope_freq_base, rms_eps;
    int      has_qk_norm, tied_embedding;
    uint32_t g4_hd_swa, g4_nh_swa, g4_nkv_swa;
    float    g4_rope_base_swa;
    uint32_t g4_n_embd_per_layer, g4_n_kv_from_start;
    float    g4_logit_softcap;
    uint32_t g4_swa_period;
    uint32_t q36_full_attn_interval, q36_n_expert, q36_n_expert_used, q36_n_ff_exp,
             q36_n_ff_shexp;
    float    q36_expert_weights_scale;
    uint32_t q36_gdn_conv_k, q36_gdn_state, q36_gdn_n_k_heads, q36_gdn_n_v_heads,
             q36_gdn_inner;
    int32_t  q36_rope_sections[4];
    uint32_t q36_rope_dim;
    float    q36_rope_base;
    uint32_t q36_nextn_predict_layers;
    uint32_t dg_canvas_length;
} qwen3_config;

typedef struct {                       /* include/sp/model.h:86-146, 360 bytes */
    const gguf_tensor *attn_norm, *attn_q, *attn_k, *attn_v, *attn_output,
                      *attn_q_norm, *attn_k_norm, *post_attn_norm, *ffn_norm,
                      *ffn_gate, *ffn_up, *ffn_down, *post_ffw_norm,
                      *attn_q_bias, *attn_k_bias, *attn_v_bias;
    const gguf_tensor *per_layer_inp_gate, *per_layer_proj, *per_layer_post_norm, *out_scale;
    int q36_is_recurrent;
    const gguf_tensor *gdn_qkv, *gdn_gate, *gdn_conv1d, *gdn_dt_bias, *gdn_a,
                      *gdn_alpha, *gdn_beta, *gdn_norm, *gdn_out;
    const gguf_tensor *ffn_gate_inp, *ffn_gate_exps, *ffn_up_exps, *ffn_down_exps,
                      *ffn_gate_inp_shexp, *ffn_gate_shexp, *ffn_up_shexp, *ffn_down_shexp;
    const gguf_tensor *ffn_gate_up_exps, *ffn_gate_inp_scale, *ffn_down_exps_scale,
                      *enc_out_scale, *pre_ffw_norm_2, *post_ffw_norm_1, *post_ffw_norm_2;
} qwen3_layer;

struct sp_arena;
typedef struct qwen3_model {           /* include/sp/model.h:150-182, 320 bytes */
    void              *gguf;
    qwen3_config       cfg;
    const gguf_tensor *token_embd, *output_norm, *output;
    qwen3_layer       *layers;
    struct sp_arena   *arena;
    int                released;
    const gguf_tensor **norm_src;
    float             **norm_buf;
    int                n_norm;
    gguf_tensor        *synth_tensors;
    const gguf_tensor  *per_layer_token_embd, *per_layer_model_proj, *per_layer_proj_norm,
                       *rope_freqs;
    const gguf_tensor  *self_cond_pre_norm, *self_cond_gate, *self_cond_up, *self_cond_down;
} qwen3_model;

/* packed weight tensor, arena layout v2 (include/sp/frobenius_lift.h:160-173, 72 bytes).
 * OK_Q4B rows: row_prec 4, nibble codes (low nibble = even column, two's
 * complement), bscale[r*bs_nblk + c/32] is the f16 step of each 32-column block. */
#define SP_FROB_ARENA_LAYOUT_VERSION 2u
typedef struct {
    int      rows, cols;
    uint8_t *row_prec;
    float   *row_scale;
    size_t  *row_off;
    uint8_t *codes;
    size_t   codes_bytes;
    uint8_t  alias_mask;
    const uint16_t *bscale;
    int      bs_nblk;
} sp_frob_packed_tensor;

typedef struct {                       /* include/sp/arena.h:31-34, 328 bytes */
    char                  name[256];
    sp_frob_packed_tensor pt;
} sp_arena_tensor;
typedef struct sp_arena sp_arena;

const sp_arena_tensor *sp_arena_find(const sp_arena *a, const char *name);   /* arena.h:52 */
sp_arena *sp_arena_from_packed(const sp_arena_tensor *ts, int n, int precision);
void      sp_arena_free(sp_arena *a);
int       sp_frob_packed_dequant_row(const sp_frob_packed_tensor *t, int r, float *dst);
const float *sp_as_f32(const qwen3_model *m, const gguf_tensor *t);   /* forward_dispatch.h:44 */

/* bridge: include/sp/sp_model.h:180-195 */
qwen3_model *sp_model_to_qwen3(const sp_model *m);
qwen3_model *sp_model_to_gemma3(const sp_model *m);
void         sp_model_store_qm(sp_model *m, qwen3_model *qm, void (*free_fn)(qwen3_model *));
qwen3_model *sp_model_borrow_qm(const sp_model *m);
void         qwen3_free(qwen3_model *m);

/* f16 <-> f32 bit conversion (include/sp/weight_dtype.h) */
float    sp_f16_to_f32(uint16_t h);
uint16_t sp_f32_to_f16(float f);

/* hashes (include/sp/sp_hash.h:31-51) */
uint32_t sp_crc32(const void *data, size_t len);
void     sp_sha256(const void *data, size_t len, uint8_t out[32]);
uint64_t sp_xxh64(const void *data, size_t len, uint64_t seed);
void     sp_blake3_256(const void *data, size_t len, uint8_t out[32]);

/* ---- OK_Q4B producer (this library; the reference tree ships no producer) ----
 * Quantize one row of `cols` floats to OK_Q4B: per 32-column block,
 * s = max|w|/7 rounded to f16 (nearest-even), code = round-half-away(w / f16(s))
 * clamped to [-7,7], nibbles packed low-first.  `codes` receives ceil(cols/2)
 * bytes, `bscale` ceil(cols/32) f16 words. */
void sp_q4b_quantize_row(const float *w, int cols, uint8_t *codes, uint16_t *bscale);

/* Synthetic random-init OK_Q4B model writer.  Weights N(0, 0.02) from one
 * SplitMix64 stream (seed) through Box-Muller in double; every norm vector 1.0;
 * tied LM head unless `untied`.  The first `spread_rows` rows of the weight
 * matrices that `spread_mask` selects (bit 0 token_embd, 1 output, 2 attn_q,
 * 3 attn_k, 4 attn_v, 5 attn_output, 6 ffn_gate, 7 ffn_up, 8 ffn_down; 0: all)
 * have their odd blocks' weights scaled by 2^13 and their even blocks' by 2^-7
 * before quantization: block scales about 2^20 apart, rows whose exact
 * accumulation needs more than 64 bits; 0 rows leaves every row plain.
 * `n_threads` <= 0 picks the machine's count.  Writes `model_path` and its
 * paired `tok_path`.  SP_OK or an error code. */
typedef struct {
    uint32_t arch_id;          /* SP_ARCH_ID_QWEN3 or SP_ARCH_ID_GEMMA3 */
    uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, n_ff, vocab;
    uint32_t max_context, swa_window;
    float    rope_base, rms_eps;
    int      untied;
    uint64_t seed;
    uint32_t spread_rows, spread_mask;
} sp_synth_spec;
sp_status sp_write_synthetic_q4b(const sp_synth_spec *spec, const char *model_path,
                                 const char *tok_path, int n_threads);

#if defined(__STDC_VERSION__) && __STDC_VERSION__ >= 201112L && !defined(__cplusplus)
_Static_assert(sizeof(sp_model_header) == 512, "sp_model_header is 512 bytes");
_Static_assert(sizeof(sp_tensor_entry) == 256, "sp_tensor_entry is 256 bytes");
_Static_assert(sizeof(sp_tok_header) == 128, "sp_tok_header is 128 bytes");
_Static_assert(sizeof(gguf_tensor) == 328, "gguf_tensor is 328 bytes");
_Static_assert(sizeof(qwen3_config) == 164, "qwen3_config is 164 bytes");
_Static_assert(sizeof(qwen3_layer) == 360, "qwen3_layer is 360 bytes");
_Static_assert(sizeof(qwen3_model) == 320, "qwen3_model is 320 bytes");
_Static_assert(sizeof(sp_frob_packed_tensor) == 72, "sp_frob_packed_tensor is 72 bytes");
_Static_assert(sizeof(sp_arena_tensor) == 328, "sp_arena_tensor is 328 bytes");
#endif

#ifdef __cplusplus
}
#endif
#endif /* SPKV_MODEL_ABI_H */
