/* sp_hipkv.h -- C ABI of the MI355X (gfx950) persistent-KV decode backend.
 *
 * The drop-in is `sp_hipkv_dispatch`: a section-6b dispatch table that an L2
 * registrant hands to sp_session_register_kvdecode_backend
 * (include/sp/sp_l1.h:403-423).  Its six entry points are also exported by name.
 * All pointers are plain host pointers; logits are caller-allocated host memory
 * of vocab floats.  Every failing call returns non-zero and sets sp_last_error().
 */
#ifndef SP_HIPKV_H
#define SP_HIPKV_H
#include <stddef.h>
#include <stdint.h>
#include "sp_l1_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The section-6b table (replaces the engine's registered gemma4_kv_* table,
 * include/sp/sp_l1.h:381-402; layout sp_l1.h:403-410). */
extern const sp_kvdecode_dispatch_fn sp_hipkv_dispatch;

/* open: sp_l1.h:390 -- qm_opaque is the session's `const qwen3_model *`
 * (sp_session_qwen3_model, sp_l1.h:354); uploads the OK_Q4B arena to HBM once
 * per model and reserves page tables for pmax positions (dpos = 0). */
int  sp_hipkv_open(const void *qm_opaque, int pmax, sp_kvdecode_handle **out);
/* prefill: sp_l1.h:392 -- store K/V for n_tok tokens at dpos.., dpos += n_tok */
int  sp_hipkv_prefill(sp_kvdecode_handle *h, const int32_t *tokens, int n_tok);
/* decode_step: sp_l1.h:393-395 -- one token at dpos, logits[vocab] of the next
 * position into caller memory, dpos += 1 */
int  sp_hipkv_decode_step(sp_kvdecode_handle *h, int32_t token, float *logits);
/* decode_step that allocates nothing -- no counterpart in the reference; for
 * callers that cannot allocate device memory (tight serving loops, harnesses
 * that forbid hipMalloc).  Same result as sp_hipkv_decode_step (bit for bit),
 * with plain kernel launches (no graph instantiation) and the step's transient
 * device memory (GEMV split-K accumulators and counters, attention partials,
 * score grid, V-sum accumulators, vector statistics) in the library's static
 * 32 MiB device buffer instead of the handle's.  Fails, with nothing changed,
 * when the handle's model and pmax need more step scratch than that (e.g.
 * float mode at head_dim 256 beyond ~65k positions) or when the position needs
 * more KV pages (new, or copies of pages shared with a fork) than the pool has
 * free without growing.  Like sp_hipkv_decode_step it waits for the step and
 * copies the logits to the host, so it cannot be called under stream capture.
 * All calls on one GPU share the buffer; a per-device lock makes such calls
 * (from several threads, on several handles and streams) run one after
 * another, each finished before the next starts. */
int  sp_hipkv_decode_step_noalloc(sp_kvdecode_handle *h, int32_t token, float *logits);
/* rewind: sp_l1.h:396 -- O(1): dpos -= n (n <= dpos) */
int  sp_hipkv_rewind(sp_kvdecode_handle *h, int n);
/* position: sp_l1.h:397 -- dpos, -1 on NULL */
int  sp_hipkv_position(const sp_kvdecode_handle *h);
/* close: sp_l1.h:398 -- NULL-safe */
void sp_hipkv_close(sp_kvdecode_handle *h);

/* ---- backend knobs (the section-6c/6d pattern: backend symbols, not session verbs) ---- */
/* Exact-integer decode on/off (replaces gemma4_kv_byteexact_set, sp_l1.h:440-455):
 * 0 = float mode (reference float semantics, tolerance-equal), 1 = exact mode
 * (integer islands + CORDIC RoPE + integer attention/GEMV, bit-reproducible).
 * Changing the mode invalidates the resident cache (dpos must be 0). */
int  sp_hipkv_set_mode(sp_kvdecode_handle *h, int exact);
/* Sliding-window layers keep a ring of window + max_rewind positions (rounded up
 * to whole pages, plus one page) instead of a full table (the SWA W-ring knob,
 * sp_l1.h:466-479).  A rewind then fails when the new position would lie more
 * than the ring's slack (ring positions - window) behind the highest position
 * ever written, since the ring has overwritten part of that position's window.
 * Only before the first token (dpos == 0).  0 = full table (default). */
int  sp_hipkv_set_max_rewind(sp_kvdecode_handle *h, int max_rewind);
/* Pages the KV pool allocates (one hipMalloc) when it has no free page left:
 * 0 = about 1 GiB of pages, at least 16 (default).  Applies to the pool this
 * handle shares with its forks, from the next growth on; a mode, codec or
 * recall change before the first token keeps the setting.  A serving caller
 * that packs many sessions into HBM uses it to grow in smaller steps.  No
 * counterpart in the reference (its KV slab is one malloc per session,
 * core/session/sp_session.c:240-245). */
int  sp_hipkv_set_pool_growth(sp_kvdecode_handle *h, int pages);
/* Copy-on-write fork of the resident cache (no counterpart in sp_l1.h: the
 * table has no fork row; sp_session_clone uses it through spx_register_fork). */
int  sp_hipkv_fork(const sp_kvdecode_handle *parent, sp_kvdecode_handle **child);
/* K/V codec of the resident cache (sp_session_config.flags, sp_l1.h:156-157,
 * the reference's session KV codec at core/session/sp_session.c:298-323):
 * 0 = plain (f32, or the int32 grid in exact mode), 1 = Spinor-63: every stored
 * K/V head passes the VHT2 int8 block codec, and attention reads the decoded
 * values, which SP_KV_SPINOR and SP_KV_SPINOR_REF share.  Float mode keeps the
 * int8 codes and chunk multipliers in HBM (HD + 4 ceil(HD/55) bytes per row,
 * padded to 16, for 4 HD); exact mode keeps the decoded values' int32 grid.
 * Head dims 64, 128, 256.  Only before the first token (dpos == 0). */
int  sp_hipkv_set_kv_codec(sp_kvdecode_handle *h, int codec);
/* ARM recall router on the global-attention layers (replaces the reference's
 * SP_RECALL_B / SP_RECALL_W / SP_RECALL_SINK / SP_RECALL_R knobs with
 * SP_RECALL_DECODE_ONLY=1, core/forward/decode.c:85-98 and :561, router
 * core/arm/arm.c:17-160): every appended K head is projected on the frozen
 * +-1 matrix (r rows, seed of include/sp/arm.h:49) into a sidecar kept in the
 * KV pages; at each decode step each q head attends only over sinks u
 * top-(B-W-sink) by projected score u the recent W positions (all positions
 * while the context holds at most B).  Prefill attends densely and writes the
 * sidecar.  B = 0 switches recall off.  r in [1, 64]; head dims 64, 128, 256;
 * not with Spinor code rows in float mode.  Only before the first token
 * (dpos == 0).  Forks inherit it; batched decodes step such handles one by one. */
int  sp_hipkv_set_recall(sp_kvdecode_handle *h, int B, int W, int sink, int r);
/* SP_RECALL_KVSEL (core/forward/decode.c:53-63, :600-629, :738-757): route
 * and select once per kv head with the group-centroid query (the float sum of
 * the group's rotated q heads, in head order) instead of once per q head; the
 * group's q heads then attend over that shared set with their own q.  Off by
 * default (per-q-head selection).  Any time; forks inherit it. */
int  sp_hipkv_set_recall_kvsel(sp_kvdecode_handle *h, int on);
/* Ring-2 (SP_RING2 with the SP_RECALL_FUSE boundary, core/forward/decode.c:
 * 117-131, 233-237, 408-440, 518-556; include/sp/arm.h:196-256): with recall
 * on, before each decode step (and each device greedy run) the full-context
 * layers' pages that hold neither a sink position nor a position of the recall
 * window move to pinned host memory (the Ring-2 store), so HBM keeps the
 * Ring-1 set (sinks + W-window, by 64-position page) plus the page being
 * written; the recalled rows of spilled pages are read over the bus, the same
 * bytes, so results are bit-identical to recall without Ring-2.  A page written
 * again after a rewind comes back to HBM first.  Pages shared with a fork stay
 * in HBM.  Spilled pages return to the pool's free list (later positions reuse
 * them), so a long session's HBM footprint stops growing with its context.
 * Any time; forks inherit it.  No effect while recall is off. */
int  sp_hipkv_set_ring2(sp_kvdecode_handle *h, int on);
/* This handle's page-table entries in host memory and in HBM, and the pool's
 * spills and fetch-backs so far. */
int  sp_hipkv_ring2_stats(const sp_kvdecode_handle *h, long long out[4]);
/* The recall sidecar of a global layer for positions [p0, p0+n): [n][n_kv_heads][r]
 * floats (the reference's projk rows, include/sp/arm.h:60-67). */
int  sp_hipkv_read_recall_sidecar(const sp_kvdecode_handle *h, int layer, int p0, int n, float *out);
/* Register the backend on a session: open(sp_session_qwen3_model(s), pmax) +
 * sp_session_register_kvdecode_backend + ownership (closed with the session) +
 * lifecycle routing (spx_session_route_kv_lifecycle: prefill, rewind and clone
 * reach the backend).  The session must be at position 0 (SP_EBADSTATE
 * otherwise).  A session created with SP_KV_SPINOR or SP_KV_SPINOR_REF gets
 * codec 1. */
sp_status sp_hipkv_attach(sp_session *s, int pmax, int exact);

/* Batched decode across sessions (many concurrent sessions of one model): hs[i]
 * (opened on the same model, with the same mode, pmax and window ring) decodes
 * tokens[i] at its own position and advances by one.  The projections run once
 * for all rows as int8-MFMA GEMMs; each row's attention reads its own session's
 * pages.  logits: n x vocab floats, row-major, host memory (may be NULL);
 * next_tokens: n greedy tokens (lowest index on ties, may be NULL).  Exact mode
 * gives the logits sp_hipkv_decode_step gives on each handle, bit for bit.  No
 * counterpart in the reference's table (sp_l1.h:403-410 decodes one session per
 * call); it serves the batched multi-session configuration. */
int  sp_hipkv_decode_batch(sp_kvdecode_handle *const *hs, int n, const int32_t *tokens, float *logits,
                           int32_t *next_tokens);

/* ---- device-resident driver entry points (bench / tests) ---- */
/* n greedy steps entirely on the device (argmax feeds the next token, no host
 * round trip), starting with `first_token` at dpos; writes the n generated
 * tokens and the device time of the n steps (HIP events on the backend's stream). */
int  sp_hipkv_greedy(sp_kvdecode_handle *h, int32_t first_token, int n, int32_t *out_tokens,
                     double *device_ms);
/* Per-kernel-class device times over n greedy steps, each launch bracketed by HIP
 * events on the backend's stream.  Classes: 0 QKV GEMV, 1 O GEMV, 2 gate/up GEMV
 * (+ activation), 3 down GEMV, 4 LM-head GEMV, 5 attention (global layers),
 * 6 attention (window layers), 7 q/k prep + append, 8 embed + RoPE table + argmax.
 * ms, launches, bytes: SP_HIPKV_NCLASS entries; bytes = algorithmic HBM bytes. */
#define SP_HIPKV_NCLASS 9
int  sp_hipkv_kernel_times(sp_kvdecode_handle *h, int32_t first_token, int n,
                           double ms[SP_HIPKV_NCLASS], long long launches[SP_HIPKV_NCLASS],
                           double bytes[SP_HIPKV_NCLASS]);
/* One sp_hipkv_decode_batch step (greedy tokens only, logits stay on the device)
 * with each kernel class of the batched step bracketed by HIP events: the same
 * classes as sp_hipkv_kernel_times, each GEMM class including its staging
 * kernel; bytes = algorithmic HBM bytes (weights once per batch, every row's
 * K/V span).  Fails for model shapes without the batched path. */
int  sp_hipkv_decode_batch_times(sp_kvdecode_handle *const *hs, int n, const int32_t *tokens, int32_t *next_tokens,
                                 double ms[SP_HIPKV_NCLASS], long long launches[SP_HIPKV_NCLASS],
                                 double bytes[SP_HIPKV_NCLASS]);
/* Read K/V of one layer for positions [p0, p0+n) in the reference slab layout
 * ([n][n_kv_heads*head_dim] floats, or int32 grid values in exact mode). */
int  sp_hipkv_read_kv(const sp_kvdecode_handle *h, int layer, int p0, int n, float *k, float *v);
/* Write K/V of one layer for positions [p0, p0+n) from the reference slab
 * layout (the inverse of sp_hipkv_read_kv: [n][n_kv_heads*head_dim] floats, or
 * int32 grid values in exact mode) and make them resident: p0 <= dpos, and
 * dpos becomes max(dpos, p0+n), as if those positions had been prefilled.
 * Pages shared with a fork are copied first.  Plain K/V rows only (not float
 * mode with the Spinor codec), recall off.  Restores a session's K/V kept on
 * the host (the oracle's set_kv counterpart); no counterpart in the reference,
 * whose host KV slab is the session's own memory (core/session/sp_session.c:240-245). */
int  sp_hipkv_write_kv(sp_kvdecode_handle *h, int layer, int p0, int n, const float *k, const float *v);
/* Use a captured HIP graph for each step body (1, default) or plain launches (0). */
int  sp_hipkv_set_graph(sp_kvdecode_handle *h, int on);
/* Exact-mode window layers (sliding window of at most 1 922 positions) run
 * their attention in one launch (1, default) whose workgroups hand data to each
 * other through the handle's slots, or in the score + V-sum launches of the
 * full-context layers (0).  Both give bit-identical results; 0 is the fallback
 * should a deployment run so many concurrent handles that a launch of up to
 * 32 x n_kv_heads workgroups could not be resident at once.  No counterpart in
 * the reference (a CPU attention). */
int  sp_hipkv_set_window_one_launch(sp_kvdecode_handle *h, int on);
/* Prefill through the batched path (1, default: 128 tokens per pass, int8-MFMA
 * GEMMs, token-batched attention) or one decode step per token (0).  Both
 * leave the same K/V (bit-identical in exact mode). */
int  sp_hipkv_set_batch_prefill(sp_kvdecode_handle *h, int on);
/* Exact mode stores V as vq = rne(v * 2^16) clamped to +-(2^23 - 1), which
 * keeps the exact V-sum inside int64 (|v| below 128).  This counts the V heads
 * this handle stored with at least one clamped element since it was opened or
 * forked (batched decodes count on the first handle of the batch); 0 means
 * every stored V is exact.  Synchronizes the handle's stream.  No counterpart
 * in the reference (its V slab is f32). */
int  sp_hipkv_v_clamps(const sp_kvdecode_handle *h, long long *count);
/* Validate a model for this backend on the host only (no device call): the
 * checks sp_hipkv_open makes before it uploads anything -- architecture, head
 * geometry, OK_Q4B tensors found through the arena, norm lengths, window.
 * out: weight bytes (codes + block scales), LM-head bytes, layers, hidden,
 * vocab, ffn, sliding window, 1 if some tensor needs the int128 GEMV path.
 * No counterpart in the reference (a registrant's pre-flight check). */
int  sp_hipkv_check_model(const void *qm_opaque, long long out[8]);
/* Bytes of model weights resident in HBM and KV bytes per token per layer. */
int  sp_hipkv_info(const sp_kvdecode_handle *h, long long out[8]);

#ifdef __cplusplus
}
#endif
#endif
