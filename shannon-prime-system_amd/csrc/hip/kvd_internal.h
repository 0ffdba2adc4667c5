// kvd_internal.h -- shared definitions of the HIP kvdecode backend (device
// layouts, kernel argument blocks, launchers).  Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvd {

constexpr int PAGE = 64;            // positions per KV page
constexpr int GEMV_WAVES = 8;       // waves per GEMV workgroup (512 threads)
constexpr int GEMV_R = 8;           // rows per wave pass
constexpr int NDIG = 6;             // balanced base-16 digit planes of an activation (|xq| < 2^22)
// replicas of the exact V-sum accumulators (chunk c adds into c % VREP).
// One: spreading the same-address atomics over 2, 4, 8 or 16 replicas was
// measured slower at every decode shape (the merge reads every replica);
// Gemma-3-12B window layer 14.1 us with one, 14.9 with four.
constexpr int VREP = 1;

enum Mode { FLOAT = 0, EXACT = 1 };

// One OK_Q4B weight tensor on the device, reference row layout:
// codes [rows][cols/2] nibbles (low = even column), scales [rows][cols/32] f16,
// plus ebase[rows + 8] = smallest block exponent of the row (for the int64 fast path;
// 8 bytes of padding: the GEMV reads 8 rows at a time), and the scales again
// interleaved by il rows, bs8[ceil(rows/il)][nblk][il] (zero-padded rows): one
// load gives a GEMV lane a block's scales for the rows of its task in this
// matrix -- il = 8 for the GEMV's unpaired rows, 4 for the gate and up
// matrices, which it reads 4 rows each per task.
struct DevW {
    const uint8_t  *codes;
    const uint16_t *bs;
    const int8_t   *ebase;
    const uint16_t *bs8;
    int rows, cols, nblk, wide;   // wide: a row's exponent spread needs the int128 path
    int il;
};

// Whole-vector statistics that the kernel producing a vector accumulates while
// it writes it, for the next GEMV's input transform: the exact sum of
// llround(v * 2^16)^2 (int64, order-free) and max |v| (float bits; atomic max
// of non-negative floats orders like the float).  Zeroed at the start of every
// decode step.  A statistic is STAT_REP consecutive VecStat replicas.
struct VecStat {
    unsigned long long ss;      // int64 two's complement
    unsigned int maxbits;
    unsigned int pad;
};
enum StatSlot { STAT_AO = 0, STAT_AP = 1, STAT_HH = 2, STAT_DN = 3, STAT_PER_LAYER = 4 };
constexpr int STAT_REP = 32;        // replicas per statistic (spread the producers' atomics)

// Input transform run by every GEMV workgroup before the matrix pass.
enum ProKind { PRO_PLAIN = 0, PRO_NORM = 1, PRO_RESID = 2 };
struct ProArgs {
    const float *x;        // residual stream (or plain input)
    const float *delta;    // PRO_RESID: branch output added into x
    // norm weights are [w (n floats) | roundf(w * 2^16) (n floats)]: exact mode
    // reads the second half where it needs the Q16 integers
    const float *post_w;   // PRO_RESID: sandwich norm weight on delta (NULL = add raw)
    const float *norm_w;   // PRO_NORM / PRO_RESID: pre-norm weight
    float       *x_out;    // PRO_RESID: updated residual (written by workgroup 0)
    // statistics of the input the producer accumulated (NULL: computed here):
    // PRO_PLAIN takes max |x|, PRO_RESID in exact mode the sum of squares of delta
    const VecStat *stat;
    int   kind, n;
    float eps;
};

// Per-session device-side step state (graph-replay friendly: kernels read it).
struct DState {
    int pos;           // position of the token being processed
    int tok;           // token id being processed (DRIVE_HOST)
    int drive;         // DRIVE_HOST / DRIVE_GREEDY / DRIVE_STREAM
    int pad;
};
enum Drive {
    DRIVE_HOST = 0,    // host sets pos/tok before every step
    DRIVE_GREEDY = 1,  // argmax writes the next tok and advances pos
    DRIVE_STREAM = 2,  // embed reads tokbuf[pos]; the advance kernel moves pos on
};

struct AttnArgs {
    const float *q;          // un-rotated q [NH*HD] (GEMV output)
    const float *k;          // new k [KVD]
    const float *v;          // new v [KVD]
    const float *q_norm, *k_norm;
    float *qr;               // rotated+normed q [NH*HD]
    float *const *pages;     // page table of this layer: device page pointers
    int   ring_pages;        // 0 = full table, else number of ring slots
    float *ao;               // output [NH*HD]
    float *part;             // partials [NKV*G][max_chunks][HD]
    float *part_ml;          // [NKV*G][max_chunks][2] (max, sum) or exact (max, S lo/hi)
    int   *counter;          // [NKV] arrival counters (self-resetting)
    int   *zscratch;         // exact mode: int32 score grid [NH][max_chunks*16] by absolute position
    int64_t *vacc;           // exact mode: V-sum totals [VREP][NH][HD] (atomic, order-free)
    int64_t *vacc_s;         // exact mode: softmax denominators [VREP][NH]
    const DState *st;
    const float *rope_cs;    // this step's rotation table for the layer's base: cos[HD/2], sin[HD/2]
    int NH, NKV, HD, win, max_chunks, chunk, mode;
    int vchunk;              // exact decode: positions per V-sum chunk, a multiple of chunk (0: chunk)
    int kvc;                 // KV codec: 0 plain, 1 Spinor-63 (float mode: code rows)
    float eps, base, ascale;
    int zstride;             // positions per q-head row of zscratch (>= pmax)
    // batched prefill: nt tokens at positions pos0.. (token = blockIdx.y of
    // qk_prep, blockIdx.z of attention); every per-token buffer is [nt][...]
    int nt, pos0, rope_stride;
    // batched decode over several sessions: token t's position and this
    // layer's page table (NULL: pos0 + t and `pages`)
    const int *tpos;
    float *const *const *tpages;
    VecStat *stat_out;       // decode: statistics of ao for the O GEMV (NULL: none)
    int *vclamp;             // exact mode: +1 per stored V head with a clamped element (NULL: not counted)
    // batched decode over sessions, full-context layers: the (token, chunk)
    // work items, one workgroup each per kv head (NULL: the token x chunk grid)
    const int2 *work;
    int nwork;
    // recall sidecar: rec_r > 0 writes each new K head's projection on the
    // frozen +-1 matrix (sign bits rec_R [rec_r][HD/32]) into the layer's
    // sidecar array rec_side [pmax][NKV][rec_r] at its position
    const uint32_t *rec_R;
    int rec_r;
    float *rec_side;
    float *rec_pq;           // routed step: each q head's projection [NH][rec_r] (NULL: not needed)
    // exact decode, window layer: scores and V-sum in one launch, whose grid
    // the host has checked fits the device at once (window_capacity), handing
    // data between workgroups through tagged slots (window_slot_bytes, zero
    // between launches)
    int one_launch;
    int64_t *wslot;
};

// ARM recall over one global layer's pages (decode): the router picks each q
// head's positions from the K sidecar, the attention reads only those.
struct RecallArgs {
    const float *pq;         // each q head's projection [NH][r] (written by the head preparation)
    const float *qr;         // rotated, normed q [NH*HD]
    float *const *pages;     // this layer's page table (full: no ring)
    const float *side;       // this layer's K sidecar [pmax][NKV][r]
    const DState *st;
    float *ao;               // output [NH*HD]
    VecStat *stat_out;       // statistics of ao for the O GEMV
    uint32_t *keys;          // [NH][kstride] order keys of the candidates' projected scores
    int *lists;              // [NH][lstride] recalled positions
    int *counts;             // [NH] recall set sizes
    int *zs;                 // [NH][lstride] exact: Q14 score grid; float: score bits
    int *cmax;               // [NH][mchunks] chunk maxima (exact: int; float: float bits)
    int64_t *vacc, *vs;      // exact: V-sum totals [NH][HD] and denominators [NH] (zero between launches)
    float *part, *psum;      // float: chunk V-sums [NH][mchunks][HD] and weight sums [NH][mchunks]
    int *counter;            // [NH] arrival counters (self-resetting)
    int kstride, lstride, mchunks, score_blocks;   // kstride: a multiple of 4, >= pmax
    int NH, NKV, HD, r, B, W, sink, mode;
    float ascale;
    const uint32_t *Rb;      // KVSEL: the projection's sign bits [r][HD/32]
    int kvsel;               // SP_RECALL_KVSEL: one selection per kv head from the group-centroid query
};
void launch_recall_attention(const RecallArgs &rc, hipStream_t s);
// exact-mode attention of one session's batched prefill on global layers
// (token-shared K/V reads, the score pass on the int8 matrix cores)
bool prefill_attention_tiled(const AttnArgs &a);
void launch_prefill_attention(const AttnArgs &a, hipStream_t s);
constexpr int RECALL_CHUNK = 64;        // recalled positions per attention workgroup
constexpr int RECALL_SCORE_BLOCKS = 64; // router scoring workgroups per kv head (grid-stride)
constexpr int RECALL_MAX_GROUP = 8;     // q heads per kv head the router serves

struct Seg { DevW w; float *out; };
enum Act { ACT_NONE = 0, ACT_GELU = 1, ACT_SILU = 2 };
struct GemvArgs {
    ProArgs pro;
    Seg  seg[3];
    int  nseg;
    int  cols;
    int  act;          // paired gate/up with activation: seg[0] = gate, seg[1] = up
    float *act_out;    // h = act(gate) * up
    int  mode;
    int64_t *accbuf;   // split-K row totals [acc_rows] (zero between launches)
    int  *gcnt;        // split arrival counters per row group [acc_rows] (zero between launches)
    int  acc_rows;
    int  nsplit, bps, groups;   // filled in by launch_gemv
    VecStat *stat_out;          // statistics of the output (paired: of act_out), NULL: none
};
struct GemvPlan { int groups, nsplit, bps, grid; };

// Per-token GEMM input staging (batched prefill): the GEMV input transform of
// token t's vector (pro pointers + t * n), then xq's three balanced base-256
// digit planes in the GEMM's operand layout, planes[p][b][t][32], t < TP.
struct StageArgs {
    ProArgs pro;
    int8_t *planes;
    int *sh;           // [TP] grid exponent per token (SH_ZERO: all-zero input)
    int T, TP, mode;   // tokens, padded token count (multiple of 32)
};
// OK_Q4B GEMM over T staged tokens: seg[i].out is [T][seg rows]; paired
// gate/up write gate, up and act(gate)*up ([T][rows]).
struct GemmArgs {
    Seg  seg[3];
    int  nseg, cols;
    const int8_t *planes;
    const int *sh;
    int  T, TP;
    int  act;
    float *act_out;
    int  mode;
    // split K (the launcher picks the split count): each split's exact int64
    // partials [TP][arows] (arows: the launch's rows, paired: gate rows then up
    // rows) in its own slice of part, one arrival counter per output tile in
    // cnt (zero between launches).  NULL: no split.
    int64_t *part;
    int *cnt;
    size_t part_cap;   // int64 elements of part
    int cnt_cap;       // counters in cnt
    int arows;
};

// Hand-off between workgroups of one launch without cache-wide fences: all data
// one workgroup passes to another goes through agent-scope atomic operations
// (coherent across the XCDs' L2s by themselves), and the arrival counter is
// bumped only after the wave's own memory operations have completed.  An
// agent-scope release/acquire fence would instead write back / invalidate the
// whole L2 of the XCD, which costs far more than the hand-off itself.
__device__ __forceinline__ void mem_complete() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
template <typename T> __device__ __forceinline__ void st_agent(T *p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T> __device__ __forceinline__ T ld_agent(const T *p) {
    return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int arrive(int *counter) {
    return __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void reset_counter(int *counter) {
    __hip_atomic_exchange(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Loads through a pointer read from memory (a page table entry): the compiler
// cannot tell its address space and would issue flat loads, which count with
// the LDS operations too, so that every wait for an LDS read in the same loop
// would also wait for the rows still streaming in.  KV pages are device
// memory, so the global-space view keeps the address.
// (The host pass of these device functions has no such address space.)
#if defined(__HIP_DEVICE_COMPILE__)
#define KVD_GLOBAL __attribute__((address_space(1)))
#else
#define KVD_GLOBAL
#endif
template <typename T> __device__ __forceinline__ const KVD_GLOBAL T *gmem(const T *p) { return (const KVD_GLOBAL T *)p; }
template <typename T> __device__ __forceinline__ KVD_GLOBAL T *gmem(T *p) { return (KVD_GLOBAL T *)p; }

// A launcher whose arguments fall outside its kernel's limits launches nothing
// and records the first such error of the calling thread; the step drivers
// collect it after enqueueing (launch_take_error: the message, then clears it;
// NULL when every launch went out).  The open-time checks keep every shape the
// backend builds inside these limits, so this is a second line of defence.
void launch_fail(const char *msg);
const char *launch_take_error();

// launchers (kvd_kernels.hip)
void launch_embed(const DevW &embd, const DState *st, const int *tokbuf, float *x, float scale, hipStream_t s,
                  VecStat *stats = nullptr, int nstats = 0);
void launch_embed_batch(const DevW &embd, const int *tokbuf, int pos0, int T, float *x, float scale, hipStream_t s,
                        const int *toks = nullptr);
void launch_rope_table_batch(int pos0, int T, int HD, int mode, float base_g, float base_l,
                             const int64_t *fq_g, const int64_t *fq_l, float *out, hipStream_t s,
                             const int *tpos = nullptr);
void launch_argmax_rows(const float *logits, int V, int T, int *out, hipStream_t s);
void launch_stage(const StageArgs &a, hipStream_t s);
void launch_gemm(const GemmArgs &a, int nrows_total, hipStream_t s);
bool gemm_supported(const DevW &w);
void launch_advance(DState *st, hipStream_t s);
void launch_gemv(const GemvArgs &a, int nrows_total, hipStream_t s);
void gemv_time_next(hipEvent_t start, hipEvent_t stop);   // events of the calling thread's next GEMV launch
void attn_time_next(hipEvent_t start, hipEvent_t stop);   // ... and of its next (score/V-sum or one-launch) attention
void launch_qk_prep(const AttnArgs &a, hipStream_t s);
void launch_embed_rope(const DevW &embd, const DState *st, const int *tokbuf, float *x, float scale, VecStat *stats,
                       int nstats, int HD, int mode, const int64_t *fq_g, const int64_t *fq_l, float *rope, hipStream_t s);
void launch_rope_table(const DState *st, int HD, int mode, float base_g, float base_l,
                       const int64_t *fq_g, const int64_t *fq_l, float *out, hipStream_t s);
void launch_attention(const AttnArgs &a, int grid_chunks, hipStream_t s);
int  attn_capacity(int HD, int G);
int  window_capacity(int HD, int G);   // workgroups of the one-launch window attention resident at once (0: none)
size_t window_slot_bytes(int NKV, int HD, int G);   // its tagged slots (zeroed once, kept zero by the kernel)
constexpr int WIN_MAXCH_HOST = 32;      // chunks per kv head it takes (the window of at most 1 922 positions)
constexpr int ATTN_MAXCH = 512;         // largest chunk of the two-kernel attention
void launch_prep_attention(const AttnArgs &a, int grid_chunks, hipStream_t s);   // qk_prep + attention, fused where possible
bool attention_fuses_prep(const AttnArgs &a);
void set_rope_tables(const int64_t atan_q60[64], int64_t kinv_q62);
void launch_argmax(const float *logits, int V, float *pval, int *pidx, int *counter,
                   DState *st, int *gen_log, int nblocks, hipStream_t s);
int  argmax_blocks(int V);
GemvPlan gemv_plan(int nrows_total, int cols, int paired, int wide, int one_per_cu);

}  // namespace kvd
