// kvd_backend.hip -- host side of the HIP section-6b kvdecode backend: model
// upload, the paged KV pool (page tables, copy-on-write forks, O(1) rewind,
// optional window ring), the per-step kernel sequence (eager or one captured
// HIP graph per step shape) and the C ABI of include/sp_hipkv.h.
//
// Reference boundary: include/sp/sp_l1.h:384-427 (dispatch table semantics),
// core/session/sp_session.c:737-746 (how sp_decode_step drives decode_step).
// Model access goes through the frozen model ABI only: qwen3_model fields,
// sp_arena_find (include/sp/arena.h:52) and sp_as_f32 (forward_dispatch.h:44).
#include "sp_l1_abi.h"
#include "sp_model_abi.h"
#include "sp_hipkv.h"
#include "kvd_internal.h"
#include "kvd_spinor.h"
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

using namespace kvd;

namespace kvd {
namespace {
thread_local std::string t_launch_err;
}
void launch_fail(const char *msg) { if (t_launch_err.empty()) t_launch_err = msg; }
const char *launch_take_error() {
    static thread_local std::string taken;
    if (t_launch_err.empty()) return nullptr;
    taken.swap(t_launch_err);
    t_launch_err.clear();
    return taken.c_str();
}
}  // namespace kvd

namespace {

// Largest pmax a handle takes: the decode attention runs at most 4096 chunks
// of at most 512 positions, the batched passes 4096 chunks of 256.
constexpr int PMAX_LIMIT = 1 << 20;

typedef __int128 i128;
typedef unsigned __int128 u128;

std::mutex g_mu;

int fail(const char *fmt, const char *a = nullptr, long long b = 0) {
    char buf[400];
    snprintf(buf, sizeof buf, fmt, a ? a : "", b);
    sp_set_error(buf);
    return 1;
}
// A launch error recorded by a launcher (shape outside a kernel's limits)
// becomes this call's error.
int take_launch_error(const char *who) {
    const char *e = launch_take_error();
    if (!e) return 0;
    char b[300];
    snprintf(b, sizeof b, "sp_hipkv: %s: %s", who, e);
    sp_set_error(b);
    return 1;
}

#define HIPCHK(call, what) do { hipError_t e_ = (call); if (e_ != hipSuccess) { \
        char b_[300]; snprintf(b_, sizeof b_, "sp_hipkv: %s: %s", (what), hipGetErrorString(e_)); \
        sp_set_error(b_); return 1; } } while (0)

// ------------------------------------------------------------ integer RoPE constants
// Host computation of the exact-mode RoPE tables: atan(2^-i) (Q60), the CORDIC
// gain inverse (Q62) and base^(-2i/d) (Q60), all by integer arithmetic.
constexpr int64_t HALF_PI_Q60 = 1811004864519280711LL;
u128 isqrt128(u128 v) {
    u128 x = 0, b = (u128)1 << 126;
    while (b > v) b >>= 2;
    while (b) {
        if (v >= x + b) { v -= x + b; x = (x >> 1) + b; } else x >>= 1;
        b >>= 2;
    }
    return x;
}
struct RopeConst { int64_t atan_q60[64]; int64_t kinv_q62; int64_t exp2neg_q62[64]; };
const RopeConst &rope_const() {
    static RopeConst rc;
    static bool ready = false;
    if (ready) return rc;
    rc.atan_q60[0] = HALF_PI_Q60 / 2;                      // atan(1) = pi/4
    for (int i = 1; i < 64; i++) {                         // atan(2^-i) = sum (-1)^k 2^-i(2k+1)/(2k+1)
        i128 sum = 0; int sgn = 1;
        for (int k = 0;; k++) {
            const int pw = i * (2 * k + 1);
            if (pw >= 120) break;
            const i128 term = ((i128)1 << (120 - pw)) / (2 * k + 1);
            sum += sgn > 0 ? term : -term; sgn = -sgn;
        }
        rc.atan_q60[i] = (int64_t)((sum + ((i128)1 << 59)) >> 60);
    }
    u128 k = (u128)1 << 62;                                // prod 1/sqrt(1 + 4^-i)
    for (int i = 0; i < 62; i++) {
        const u128 r = isqrt128(((u128)1 << 124) + ((u128)1 << (124 - 2 * i)));
        k = (k * (((u128)1 << 124) / r)) >> 62;
    }
    rc.kinv_q62 = (int64_t)k;
    u128 c = (u128)1 << 61;                                // 2^(-2^-j) by repeated sqrt of 1/2
    rc.exp2neg_q62[0] = 0;
    for (int j = 1; j < 64; j++) { c = isqrt128(c << 62); rc.exp2neg_q62[j] = (int64_t)c; }
    ready = true;
    return rc;
}
i128 log2_q62(float v) {                                   // normal positive floats
    uint32_t bits; memcpy(&bits, &v, 4);
    const int e = (int)((bits >> 23) & 255u) - 127;
    u128 y = (u128)((bits & 0x7FFFFFu) | 0x800000u) << (62 - 23);
    i128 frac = 0;
    for (int b = 61; b >= 0; b--) {
        y = (y * y) >> 62;
        if (y >= ((u128)2 << 62)) { y >>= 1; frac |= (i128)1 << b; }
    }
    return ((i128)e << 62) + frac;
}
int64_t rope_freq_q60(float base, int i, int d) {
    const RopeConst &rc = rope_const();
    if (i == 0) return (int64_t)1 << 60;
    i128 t = (log2_q62(base) * (i128)(2 * i)) / (i128)d;
    if (t < 0) t = 0;
    const int64_t n = (int64_t)(t >> 62);
    const uint64_t r = (uint64_t)(t & (((i128)1 << 62) - 1));
    u128 acc = (u128)1 << 62;
    for (int j = 1; j <= 62; j++)
        if ((r >> (62 - j)) & 1u) acc = (acc * (u128)rc.exp2neg_q62[j]) >> 62;
    if (n >= 62) return 0;
    return (int64_t)((acc >> 2) >> n);
}

// ------------------------------------------------------------ device model
struct DevLayer {
    DevW q, k, v, o, gate, up, down;
    const float *attn_norm, *q_norm, *k_norm, *ffn_norm, *post_attn, *post_ffw;
};
struct DevModel {
    const qwen3_model *qm = nullptr;
    int refs = 0, gemma = 0;
    int E = 0, FF = 0, NH = 0, NKV = 0, HD = 0, V = 0, NL = 0, SW = 0;
    float base = 0, eps = 0;
    DevW embd{}, out{};
    const float *out_norm = nullptr;
    std::vector<DevLayer> L;
    void *buf = nullptr;
    size_t bytes = 0, weight_bytes = 0, lm_bytes = 0, layer_bytes = 0, embd_bytes = 0;
    int64_t *freq_global = nullptr, *freq_local = nullptr;
    // closed handles kept for reuse (stream, tables, scratch, batch buffers and
    // captured graphs intact): a fork or open with the same pmax and window ring
    // takes one instead of allocating; they hold no model reference
    std::vector<sp_kvdecode_handle *> shells;
};
std::map<const qwen3_model *, DevModel *> g_models;
void free_handle(sp_kvdecode_handle *h);

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Uploader {                         // one allocation, arrays carved at 256 B
    std::vector<std::pair<const void *, size_t>> src;
    std::vector<size_t> off;
    size_t total = 0;
    size_t add(const void *p, size_t n) { off.push_back(total); src.push_back({p, n}); size_t o = total; total = align_up(total + n, 256); return o; }
};

int load_weight(const qwen3_model *qm, const gguf_tensor *t, int rows, int cols, Uploader &up,
                std::vector<std::vector<int8_t>> &ebase_store, std::vector<std::vector<uint16_t>> &bs8_store,
                DevW &w, size_t offs[4], int il) {
    if (!t) return fail("sp_hipkv_open: model lacks a weight tensor%s", "");
    const sp_arena_tensor *at = sp_arena_find(qm->arena, t->name);
    if (!at) return fail("sp_hipkv_open: weight %s not in the packed arena", t->name);
    const sp_frob_packed_tensor &p = at->pt;
    if (!p.bscale || p.bs_nblk != (cols + 31) / 32)
        return fail("sp_hipkv_open: %s is not OK_Q4B (block-scaled 4-bit); only OK_Q4B is served", t->name);
    if (p.rows != rows || p.cols != cols) return fail("sp_hipkv_open: %s has unexpected shape", t->name);
    const size_t rb = (size_t)(cols + 1) / 2, nb = (size_t)p.bs_nblk;
    for (int r = 0; r < rows; r++)
        if (p.row_prec[r] == 8u || p.row_off[r] != (size_t)r * rb)
            return fail("sp_hipkv_open: %s has Q8-promoted or non-contiguous rows", t->name);
    if (cols % 32 != 0) return fail("sp_hipkv_open: %s: cols must be a multiple of 32", t->name);
    // per-row smallest block exponent; rows whose exponent spread could overflow
    // the int64 accumulator (see kvd_gemv.hip) switch the tensor to int128
    // (8 zero bytes of padding: the GEMV reads a task's 8 rows in one load)
    ebase_store.emplace_back(rows + 8);
    std::vector<int8_t> &eb = ebase_store.back();
    int lg = 0; while ((1 << lg) < (int)nb) lg++;
    const int max_spread = 21 - lg;
    int wide = 0;
    for (int r = 0; r < rows; r++) {
        int emin = 127, emax = -127;
        const uint16_t *bs = p.bscale + (size_t)r * nb;
        for (size_t b = 0; b < nb; b++) {
            const int E5 = (bs[b] >> 10) & 31, mant = bs[b] & 1023;
            if (E5 == 31) return fail("sp_hipkv_open: %s has a non-finite block scale", t->name);
            if (!E5 && !mant) continue;
            const int e = E5 ? E5 - 25 : -24;
            emin = std::min(emin, e); emax = std::max(emax, e);
        }
        if (emin > emax) emin = emax = 0;
        eb[r] = (int8_t)emin;
        if (emax - emin > max_spread) wide = 1;
    }
    // the GEMV's copy of the scales, il rows interleaved per block
    bs8_store.emplace_back((size_t)(rows + il - 1) / il * il * nb, (uint16_t)0);
    std::vector<uint16_t> &b8 = bs8_store.back();
    for (int r = 0; r < rows; r++) {
        const uint16_t *bs = p.bscale + (size_t)r * nb;
        uint16_t *dst = b8.data() + (size_t)(r / il) * nb * il + r % il;
        for (size_t b = 0; b < nb; b++) dst[b * il] = bs[b];
    }
    offs[0] = up.add(p.codes, rb * rows);
    offs[1] = up.add(p.bscale, nb * 2 * rows);
    offs[2] = up.add(eb.data(), (size_t)rows + 8);
    offs[3] = up.add(b8.data(), b8.size() * 2);
    w.rows = rows; w.cols = cols; w.nblk = (int)nb; w.wide = wide; w.il = il;
    return 0;
}

// The device model of qm: validated, then uploaded once and shared (refcounted).
// upload = false validates only (host work, no device call) and returns a
// DevModel without buffers that the caller deletes.
DevModel *model_get(const qwen3_model *qm, bool upload = true) {
    if (upload) {
        auto it = g_models.find(qm);
        if (it != g_models.end()) { it->second->refs++; return it->second; }
    }
    const qwen3_config &c = qm->cfg;
    if (c.arch != SP_ARCH_QWEN3 && c.arch != SP_ARCH_GEMMA3) { fail("sp_hipkv_open: architecture %s not served (Qwen3 / Gemma3 only)", ""); return nullptr; }
    if (!qm->arena) { fail("sp_hipkv_open: model has no packed arena%s", ""); return nullptr; }
    if (c.head_dim % 64 || c.head_dim > 512 || !c.n_head_kv || c.n_head % c.n_head_kv) {
        fail("sp_hipkv_open: unsupported head geometry (head_dim %s%lld)", "", (long long)c.head_dim); return nullptr;
    }
    const int G = (int)(c.n_head / c.n_head_kv), HD = (int)c.head_dim;
    if (!((HD == 256 && (G == 2 || G == 4)) || (HD == 128 && (G == 2 || G == 4)) || (HD == 64 && (G == 2 || G == 4)))) {
        fail("sp_hipkv_open: unsupported (head_dim, group) combination%s", ""); return nullptr;
    }
    if (c.n_layers == 0 || c.n_embd == 0 || c.n_vocab == 0 || c.n_ff == 0) {
        fail("sp_hipkv_open: model has a zero dimension%s"); return nullptr;
    }
    if (c.n_ff % GEMV_R) { fail("sp_hipkv_open: n_ff must be a multiple of %s%lld", "", (long long)GEMV_R); return nullptr; }
    if (c.arch == SP_ARCH_GEMMA3 && (c.sliding_window <= 0 || c.sliding_window > (4096 - 2) * 64)) {
        // window layers run 64-position chunks, at most 4096 per launch
        fail("sp_hipkv_open: sliding window outside [1, %s%lld]", "", (long long)((4096 - 2) * 64)); return nullptr;
    }
    std::unique_ptr<DevModel> m(new DevModel);
    m->qm = qm; m->gemma = c.arch == SP_ARCH_GEMMA3;
    m->E = (int)c.n_embd; m->FF = (int)c.n_ff; m->NH = (int)c.n_head; m->NKV = (int)c.n_head_kv;
    m->HD = HD; m->V = (int)c.n_vocab; m->NL = (int)c.n_layers; m->SW = (int)c.sliding_window;
    m->base = c.rope_freq_base; m->eps = c.rms_eps;
    const int QD = m->NH * HD, KVD = m->NKV * HD;
    Uploader up;
    std::vector<std::vector<int8_t>> ebs;
    std::vector<std::vector<uint16_t>> b8s;
    ebs.reserve((size_t)m->NL * 7 + 2);
    b8s.reserve((size_t)m->NL * 7 + 2);
    struct Pending { DevW *w; size_t o[4]; };
    std::vector<Pending> pend;
    auto addw = [&](const gguf_tensor *t, int rows, int cols, DevW &w, int il = 8) -> int {
        Pending pd; pd.w = &w;
        if (load_weight(qm, t, rows, cols, up, ebs, b8s, w, pd.o, il)) return 1;
        pend.push_back(pd);
        return 0;
    };
    std::vector<std::pair<const float *, size_t>> norms;   // (host src, len)
    std::vector<const float **> norm_slots;
    std::vector<size_t> norm_off;
    // every norm weight vector goes up as [w (n) | roundf(w * 2^16) (n)]: the
    // exact mode's input transforms read the Q16 half instead of rounding the
    // weights in every workgroup (roundf of the exact float product, the value
    // the device's own rounding gives)
    std::vector<std::vector<float>> nq;
    nq.reserve((size_t)m->NL * 6 + 2);
    auto addn = [&](const gguf_tensor *t, int n, const float **slot) -> int {
        const float *src = t ? sp_as_f32(qm, t) : nullptr;
        if (!src) return fail("sp_hipkv_open: missing norm tensor %s", t ? t->name : "(null)");
        // the copy behind sp_as_f32 has the tensor's element count: both bridges
        // (ours and sp_model_bridge.c:217-222) carry the on-disk dims
        uint64_t ne = t->n_dims ? 1 : 0;
        for (uint32_t d = 0; d < t->n_dims && d < GGUF_MAX_DIMS; d++) ne *= t->dims[d];
        if (t->n_dims > GGUF_MAX_DIMS || ne != (uint64_t)n)
            return fail("sp_hipkv_open: norm tensor %s has the wrong length", t->name);
        nq.emplace_back(2 * (size_t)n);
        std::vector<float> &v = nq.back();
        for (int i = 0; i < n; i++) { v[i] = src[i]; v[(size_t)n + i] = roundf(src[i] * 65536.0f); }
        norm_off.push_back(up.add(v.data(), (size_t)n * 8));
        norm_slots.push_back(slot);
        return 0;
    };
    m->L.resize(m->NL);
    if (addw(qm->token_embd, m->V, m->E, m->embd)) return nullptr;
    if (qm->output != qm->token_embd) { if (addw(qm->output, m->V, m->E, m->out)) return nullptr; }
    if (addn(qm->output_norm, m->E, &m->out_norm)) return nullptr;
    for (int l = 0; l < m->NL; l++) {
        const qwen3_layer &y = qm->layers[l];
        DevLayer &d = m->L[l];
        if (addw(y.attn_q, QD, m->E, d.q) || addw(y.attn_k, KVD, m->E, d.k) || addw(y.attn_v, KVD, m->E, d.v) ||
            addw(y.attn_output, m->E, QD, d.o) || addw(y.ffn_gate, m->FF, m->E, d.gate, 4) ||
            addw(y.ffn_up, m->FF, m->E, d.up, 4) || addw(y.ffn_down, m->E, m->FF, d.down)) return nullptr;
        if (addn(y.attn_norm, m->E, &d.attn_norm) || addn(y.attn_q_norm, HD, &d.q_norm) ||
            addn(y.attn_k_norm, HD, &d.k_norm) || addn(y.ffn_norm, m->E, &d.ffn_norm)) return nullptr;
        d.post_attn = d.post_ffw = nullptr;
        if (m->gemma && (addn(y.post_attn_norm, m->E, &d.post_attn) || addn(y.post_ffw_norm, m->E, &d.post_ffw))) return nullptr;
    }
    // RoPE frequency tables (global base, and 1e4 for Gemma window layers): per
    // base HD/2 exact-mode frequencies in Q60, then HD/2 float-mode frequencies
    // powf(base, -2i/d), formed here by the host's libm as the reference forms
    // them (core/forward_kernels/forward_kernels.c:34): theta = p * freq is then
    // the reference's float, where a one-ulp difference in freq would move
    // theta by p ulps (2e-3 rad at p = 32767)
    const int half = HD / 2;
    std::vector<int64_t> fg(HD), fl(HD);
    for (int i = 0; i < half; i++) {
        fg[i] = rope_freq_q60(m->base, i, HD); fl[i] = rope_freq_q60(10000.0f, i, HD);
        const float e = -2.0f * (float)i / (float)HD;
        const float pg = powf(m->base, e), pl = powf(10000.0f, e);
        memcpy((float *)(fg.data() + half) + i, &pg, 4);
        memcpy((float *)(fl.data() + half) + i, &pl, 4);
    }
    const size_t o_fg = up.add(fg.data(), fg.size() * 8), o_fl = up.add(fl.data(), fl.size() * 8);
    for (auto &pd : pend)
        m->weight_bytes += (size_t)pd.w->rows * (pd.w->cols / 2) + (size_t)pd.w->rows * pd.w->nblk * 2;
    const bool tied = qm->output == qm->token_embd;
    if (tied) m->out = m->embd;
    m->embd_bytes = (size_t)m->embd.rows * (m->embd.cols / 2) + (size_t)m->embd.rows * m->embd.nblk * 2;
    m->lm_bytes = (size_t)m->out.rows * (m->out.cols / 2) + (size_t)m->out.rows * m->out.nblk * 2;
    m->layer_bytes = m->weight_bytes - m->embd_bytes - (tied ? 0 : m->lm_bytes);
    m->bytes = up.total;
    if (!upload) return m.release();

    if (hipMalloc(&m->buf, up.total) != hipSuccess) {
        fail("sp_hipkv_open: hipMalloc of %s%lld weight bytes failed", "", (long long)up.total); return nullptr;
    }
    uint8_t *base = (uint8_t *)m->buf;
    for (size_t i = 0; i < up.src.size(); i++)
        if (hipMemcpy(base + up.off[i], up.src[i].first, up.src[i].second, hipMemcpyHostToDevice) != hipSuccess) {
            hipFree(m->buf); fail("sp_hipkv_open: weight upload failed%s", ""); return nullptr;
        }
    for (auto &pd : pend) {
        pd.w->codes = base + pd.o[0];
        pd.w->bs = (const uint16_t *)(base + pd.o[1]);
        pd.w->ebase = (const int8_t *)(base + pd.o[2]);
        pd.w->bs8 = (const uint16_t *)(base + pd.o[3]);
    }
    for (size_t i = 0; i < norm_slots.size(); i++) *norm_slots[i] = (const float *)(base + norm_off[i]);
    if (tied) m->out = m->embd;
    m->freq_global = (int64_t *)(base + o_fg);
    m->freq_local = (int64_t *)(base + o_fl);
    const RopeConst &rc = rope_const();
    set_rope_tables(rc.atan_q60, rc.kinv_q62);
    // the uploads above run on the null stream, which the handles' non-blocking
    // streams do not wait for: finish them before any handle launches work
    if (hipDeviceSynchronize() != hipSuccess) {
        hipFree(m->buf); fail("sp_hipkv_open: weight upload failed%s", ""); return nullptr;
    }
    m->refs = 1;
    DevModel *raw = m.release();
    g_models[qm] = raw;
    return raw;
}
void model_put(DevModel *m) {
    if (!m || --m->refs > 0) return;
    for (sp_kvdecode_handle *sh : m->shells) free_handle(sh);
    m->shells.clear();
    g_models.erase(m->qm);
    hipFree(m->buf);
    delete m;
}

// ------------------------------------------------------------ KV page pool
// Device pages have ids >= 0.  With Ring-2 (sp_hipkv_set_ring2) a page that
// left the attention window moves to pinned host memory: a host page, named in
// the page tables by id HOST_ID(hid) <= -2 (-1 is an unmapped slot).  Device
// and host pages are both refcounted (forks share them).
constexpr int NO_PAGE = -1;
constexpr int HOST_ID(int hid) { return -2 - hid; }
constexpr int HID_OF(int id) { return -2 - id; }
struct KvPool {
    std::mutex mu;                            // shared by a handle and its forks
    size_t page_bytes = 0;
    std::vector<void *> chunks;
    std::vector<float *> ptr;
    std::vector<int> refc, free_ids;
    int pages_per_chunk = 0;
    // host pages (Ring-2): pinned chunks, device-visible pointers
    std::vector<void *> hchunks;
    std::vector<float *> hptr;
    std::vector<int> hrefc, hfree;
    long long spills = 0, fetches = 0;
    ~KvPool() {
        for (void *c : chunks) hipFree(c);
        for (void *c : hchunks) hipHostFree(c);
    }
    float *page_ptr(int id) const { return id >= 0 ? ptr[id] : (id <= -2 ? hptr[HID_OF(id)] : nullptr); }
    void retain(int id) { if (id >= 0) refc[id]++; else if (id <= -2) hrefc[HID_OF(id)]++; }
    void release(int id) {
        if (id >= 0) unref(id);
        else if (id <= -2 && --hrefc[HID_OF(id)] == 0) hfree.push_back(HID_OF(id));
    }
    int refcount(int id) const { return id >= 0 ? refc[id] : (id <= -2 ? hrefc[HID_OF(id)] : 0); }
    // one host page (growing the host store by about 256 MiB), or -1
    int host_alloc() {
        if (hfree.empty()) {
            const int n = (int)std::max<size_t>(4, ((size_t)256 << 20) / page_bytes);
            void *c = nullptr;
            if (hipHostMalloc(&c, (size_t)n * page_bytes, hipHostMallocDefault) != hipSuccess) return -1;
            void *dc = nullptr;
            if (hipHostGetDevicePointer(&dc, c, 0) != hipSuccess) { hipHostFree(c); return -1; }
            hchunks.push_back(c);
            for (int i = 0; i < n; i++) {
                hptr.push_back((float *)((uint8_t *)dc + (size_t)i * page_bytes));
                hrefc.push_back(0);
                hfree.push_back((int)hptr.size() - 1);
            }
            std::reverse(hfree.end() - n, hfree.end());
        }
        const int hid = hfree.back(); hfree.pop_back();
        hrefc[hid] = 1;
        return hid;
    }
    int grow(int min_pages) {
        const int n = std::max(min_pages, pages_per_chunk);
        void *c = nullptr;
        if (hipMalloc(&c, (size_t)n * page_bytes) != hipSuccess) return 1;
        chunks.push_back(c);
        for (int i = 0; i < n; i++) {
            ptr.push_back((float *)((uint8_t *)c + (size_t)i * page_bytes));
            refc.push_back(0);
            free_ids.push_back((int)ptr.size() - 1);
        }
        std::reverse(free_ids.end() - n, free_ids.end());
        return 0;
    }
    // may_grow = false: only pages already in the pool (no device allocation)
    int alloc(bool may_grow = true) {
        if (free_ids.empty() && (!may_grow || grow(1))) return -1;
        const int id = free_ids.back(); free_ids.pop_back();
        refc[id] = 1;
        return id;
    }
    void unref(int id) { if (id >= 0 && --refc[id] == 0) free_ids.push_back(id); }
};

// The transient device memory of one decode step: GEMV split-K row totals and
// arrival counters, attention partials, chunk maxima / sums, arrival counters,
// the exact score grid and V-sum accumulators, and the per-layer vector
// statistics.  Every accumulator and counter is back at zero when the step's
// kernels end; the statistics are cleared by the step's first kernel.
struct StepScratch {
    int64_t *gacc = nullptr; int *gcnt = nullptr; int acc_rows = 0;
    float *part = nullptr, *part_ml = nullptr;
    int *counter = nullptr, *zscratch = nullptr;
    int64_t *vacc = nullptr, *vacc_s = nullptr;
    VecStat *stats = nullptr;
    int64_t *wslot = nullptr;                // one-launch window attention slots (NULL: two-kernel path)
};

}  // namespace

// ------------------------------------------------------------ the handle
struct sp_kvdecode_handle {
    DevModel *m = nullptr;
    std::shared_ptr<KvPool> pool;
    int mode = FLOAT, pmax = 0, dpos = 0, use_graph = 1, hwm = 0;
    int kvc = KVC_PLAIN;                     // KV codec (KVC_SPINOR: SP_KV_SPINOR sessions)
    int use_batch = 1;                       // batched (MFMA) prefill where the shapes allow it
    int max_rewind = 0;                      // 0: full tables for window layers
    int pool_growth = 0;                     // pages per pool growth (0: ~1 GiB)
    int recall_kvsel = 0;                    // SP_RECALL_KVSEL: one recall selection per kv head
    int win_one = 1;                         // exact window layers in one launch (0: the two-kernel path)
    int ring2 = 0;                           // Ring-2: spill full-context pages outside sinks + window to host
    int full_pages = 0, ring_pages = 0;
    std::vector<std::vector<int>> pt;        // [NL][slots] page ids (-1 = unmapped)
    std::vector<int> slots;                  // per layer: number of slots
    float **d_pt = nullptr;                  // device: concatenated per-layer pointer tables
    float **h_pt = nullptr;                  // pinned mirror
    std::vector<size_t> pt_off;              // per layer offset into d_pt
    hipStream_t stream = nullptr;
    DState *d_st = nullptr;
    DState *h_st = nullptr;                  // pinned
    float *x0 = nullptr, *x1 = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *qr = nullptr,
          *ao = nullptr, *ap = nullptr, *gg = nullptr, *uu = nullptr, *hh = nullptr, *dn = nullptr,
          *logits = nullptr, *part = nullptr, *part_ml = nullptr, *am_v = nullptr;
    int *counter = nullptr, *zscratch = nullptr, *am_i = nullptr, *am_cnt = nullptr, *gen_log = nullptr;
    int *vclamp = nullptr;                   // exact mode: V heads stored with a clamped element
    int *tokbuf = nullptr;                   // DRIVE_STREAM tokens by absolute position
    float *rope = nullptr;                   // [2][HD] rotation table of the current step
    int64_t *vacc = nullptr, *vacc_s = nullptr;
    int64_t *gacc = nullptr;                 // GEMV split-K row totals (zero between launches)
    VecStat *stats = nullptr;                // [NL][STAT_PER_LAYER][STAT_REP] vector statistics of the step
    int *gcnt = nullptr;                     // GEMV split arrival counters
    int acc_rows = 0;
    float *h_logits = nullptr;               // pinned staging
    int max_chunks = 0;
    StepScratch ss;                          // the step scratch above, carved from `scratch` (this handle's)
    // ARM recall (sp_hipkv_set_recall): budget B, window W, sinks, projection
    // rows r (B = 0: off).  The K sidecar lives in the KV pages (forks,
    // copy-on-write and rewind carry it); the router's buffers live here and
    // are back at zero (accumulators, counters) between launches.
    struct Recall {
        int B = 0, W = 0, sink = 0, r = 0;
        void *buf = nullptr;
        float *side = nullptr;               // K sidecar [global layers][pmax][NKV][r] (zeroed at allocation)
        size_t side_layer = 0;               // floats per global layer
        uint32_t *Rb = nullptr, *keys = nullptr;
        int *lists = nullptr, *counts = nullptr, *zs = nullptr, *cmax = nullptr, *counter = nullptr;
        int64_t *vacc = nullptr, *vs = nullptr;
        float *part = nullptr, *psum = nullptr, *pq = nullptr;
        int lstride = 0, mchunks = 0, kstride = 0;
    } rec;
    int attn_cap = 0;                        // exact decode attention workgroups resident at once
    int win_cap = 0;                         // one-launch window attention workgroups resident at once
    void *scratch = nullptr;
    int built = 0;                           // tables and scratch allocated (reusable as a shell)
    // batched prefill buffers ([TB][...] per token), allocated on first use
    struct Batch {
        void *buf = nullptr;
        int TB = 0, mcb = 0;                 // tokens per batch, chunk capacity per q-head
        float *x0, *x1, *q, *k, *v, *qr, *ao, *ap, *gg, *uu, *hh, *dn, *rope, *part, *part_ml;
        int8_t *planes; int *sh, *counter, *zs;
        int64_t *vacc, *vacc_s;
        int64_t *gpart; int *gcnt;           // GEMM split-K partial slices and tile arrival counters
        // batched decode over sessions (allocated on first use): logits rows,
        // greedy tokens, per-token token / position / per-layer page tables
        void *dbuf = nullptr;
        float *logits; int *next, *toks, *tpos; float *const **tpages;
        int2 *work; int nwork = 0, wcap = 0;   // full-context layers' (token, chunk) work items
        void *hstage = nullptr;              // pinned upload staging for toks/tpos/tpages
    } b;
    // graph cache: key (logits?, argmax?, grid_global, grid_local, chunk_global)
    struct GKey { int lg, am, gg, gl, cg, rt; bool operator<(const GKey &o) const {
        return std::tie(lg, am, gg, gl, cg, rt) < std::tie(o.lg, o.am, o.gg, o.gl, o.cg, o.rt); } };
    std::map<GKey, hipGraphExec_t> graphs;
};

namespace {

bool is_global(const DevModel *m, int l) { return !m->gemma || (l % 6) == 5; }

void free_graphs(sp_kvdecode_handle *h) {
    for (auto &g : h->graphs) hipGraphExecDestroy(g.second);
    h->graphs.clear();
}

int layer_slots(const sp_kvdecode_handle *h, int l) {
    if (!is_global(h->m, l) && h->max_rewind > 0 && h->m->SW > 0) return h->ring_pages;
    return h->full_pages;
}

// Bytes of one stored K or V row: f32 / int32 values, or in float mode with
// the Spinor codec the row of int8 codes and chunk multipliers.
size_t kv_row_bytes(const DevModel *m, int mode, int kvc) {
    return mode == FLOAT && kvc == KVC_SPINOR ? (size_t)spn_row_bytes(m->HD) : (size_t)m->HD * 4;
}
// the bytes of such a row the attention needs (no alignment padding)
double kv_row_payload(const DevModel *m, int mode, int kvc) {
    return mode == FLOAT && kvc == KVC_SPINOR ? (double)(m->HD + 4 * spn_blocks(m->HD)) : 4.0 * m->HD;
}
// A page: K and V rows of PAGE positions of every kv head.
size_t page_bytes_of(const DevModel *m, int mode, int kvc) {
    return (size_t)2 * m->NKV * PAGE * kv_row_bytes(m, mode, kvc);
}
// growth: pages per device allocation when the pool grows (0: about 1 GiB of
// pages, at least 16)
int pool_growth_pages(size_t page_bytes, int growth) {
    return growth > 0 ? growth : (int)std::max<size_t>(16, ((size_t)1 << 30) / page_bytes);
}
std::shared_ptr<KvPool> make_pool(const DevModel *m, int mode, int kvc, int growth) {
    auto pool = std::make_shared<KvPool>();
    pool->page_bytes = page_bytes_of(m, mode, kvc);
    pool->pages_per_chunk = pool_growth_pages(pool->page_bytes, growth);
    return pool;
}

int build_tables(sp_kvdecode_handle *h) {
    const DevModel *m = h->m;
    h->full_pages = (h->pmax + PAGE - 1) / PAGE;
    h->ring_pages = h->max_rewind > 0 ? std::min(h->full_pages, (m->SW + h->max_rewind + PAGE - 1) / PAGE + 1) : 0;
    h->pt.assign(m->NL, {});
    h->slots.assign(m->NL, 0);
    h->pt_off.assign(m->NL, 0);
    size_t tot = 0;
    for (int l = 0; l < m->NL; l++) {
        h->slots[l] = layer_slots(h, l);
        h->pt[l].assign(h->slots[l], -1);
        h->pt_off[l] = tot; tot += (size_t)h->slots[l];
    }
    if (h->d_pt) { hipFree(h->d_pt); h->d_pt = nullptr; }
    if (h->h_pt) { hipHostFree(h->h_pt); h->h_pt = nullptr; }
    HIPCHK(hipMalloc(&h->d_pt, tot * sizeof(float *)), "page table alloc");
    HIPCHK(hipHostMalloc(&h->h_pt, tot * sizeof(float *), hipHostMallocDefault), "page table mirror alloc");
    for (size_t i = 0; i < tot; i++) h->h_pt[i] = nullptr;
    HIPCHK(hipMemcpyAsync(h->d_pt, h->h_pt, tot * sizeof(float *), hipMemcpyHostToDevice, h->stream), "page table init");
    HIPCHK(hipStreamSynchronize(h->stream), "page table init sync");
    return 0;
}

// Make the pages holding positions [p0, p1) present and exclusively owned in
// every layer (allocate on first touch, copy-on-write when shared by a fork).
//
// Two phases, so that a failure changes nothing: first the pages the call
// needs (unmapped slots plus slots shared with a fork) are counted and taken
// from the pool's free list, growing the pool once when allowed; only then are
// the tables changed, and the changed span is uploaded before any return.
int ensure_pages(sp_kvdecode_handle *h, int p0, int p1, bool may_grow = true) {
    const DevModel *m = h->m;
    if (p1 <= p0) return 0;
    std::lock_guard<std::mutex> lk(h->pool->mu);
    KvPool &pool = *h->pool;
    const int lp0 = p0 / PAGE, lp1 = (p1 - 1) / PAGE;
    // the distinct slots of [lp0, lp1] in layer l: a ring visits at most S of them
    auto slots_of = [&](int l, int &n) { const int S = h->slots[l]; n = std::min(lp1 - lp0 + 1, S); return S; };
    size_t need = 0;
    for (int l = 0; l < m->NL; l++) {
        int n = 0;
        const int S = slots_of(l, n);
        for (int i = 0; i < n; i++) {
            const int lp = lp0 + i, slot = (S == h->full_pages) ? lp : lp % S;
            const int id = h->pt[l][slot];
            if (id < 0 || pool.refc[id] > 1) need++;     // unmapped, host (Ring-2) or shared with a fork
        }
    }
    if (need > pool.free_ids.size()) {
        if (!may_grow)
            return fail("sp_hipkv: %s%lld free KV pages needed without growing the pool (nothing changed)", "",
                        (long long)need);
        if (pool.grow((int)(need - pool.free_ids.size())))
            return fail("sp_hipkv: KV pool exhausted (hipMalloc failed; nothing changed)%s");
    }
    size_t lo = SIZE_MAX, hi = 0;                // changed entries of the concatenated table
    hipError_t err = hipSuccess;
    for (int l = 0; l < m->NL && err == hipSuccess; l++) {
        int n = 0;
        const int S = slots_of(l, n);
        for (int i = 0; i < n; i++) {
            const int lp = lp0 + i, slot = (S == h->full_pages) ? lp : lp % S;
            int &id = h->pt[l][slot];
            if (id >= 0 && pool.refc[id] <= 1) continue;
            const int nid = pool.alloc(false);   // reserved above: cannot fail
            if (id != NO_PAGE) {                 // shared with a fork, or in host memory: copy, then drop this reference
                err = hipMemcpyAsync(pool.ptr[nid], pool.page_ptr(id), pool.page_bytes, hipMemcpyDefault, h->stream);
                if (err != hipSuccess) { pool.unref(nid); break; }
                if (id <= -2) pool.fetches++;
                pool.release(id);
            }
            id = nid;
            h->h_pt[h->pt_off[l] + slot] = pool.ptr[nid];
            lo = std::min(lo, h->pt_off[l] + slot); hi = std::max(hi, h->pt_off[l] + slot + 1);
        }
    }
    if (hi > lo) {
        // one upload of the changed span (the pinned mirror is authoritative),
        // also after a failed copy so the device table matches the host's; the
        // wait also covers the copy-on-write copies issued above
        HIPCHK(hipMemcpyAsync(h->d_pt + lo, h->h_pt + lo, (hi - lo) * sizeof(float *), hipMemcpyHostToDevice, h->stream),
               "page table update");
        HIPCHK(hipStreamSynchronize(h->stream), "page table update sync");
    }
    HIPCHK(err, "copy-on-write page copy");
    return 0;
}

// Ring-2 (the reference's SP_RING2 with the SP_RECALL_FUSE boundary,
// core/forward/decode.c:117-131, 233-237, 408-440, 518-556): with recall on,
// the full-context (global) layers keep in HBM only the pages that hold a sink
// position or reach into the recall window of the position about to be
// decoded (the Ring-1 set, sp_arm_r1slot's sinks + W-window by page); every
// other page this handle owns alone moves to pinned host memory and its
// table entry points there.  The recall attention reads the recalled rows of
// such pages over the bus, the same bytes, so results are bit-identical; a
// page written again (after a rewind) comes back first (ensure_pages).
// Pages shared with a fork stay in HBM.  Best effort: when the host store
// cannot grow, the remaining pages stay where they are.
int ring2_spill(sp_kvdecode_handle *h, int pos) {
    if (!h->ring2 || h->rec.B <= 0) return 0;
    const DevModel *m = h->m;
    const int lo = pos + 1 - h->rec.W;                 // the window's first position
    if (lo <= 0) return 0;
    const int lp_begin = (h->rec.sink + PAGE - 1) / PAGE, lp_end = lo / PAGE;
    if (lp_begin >= lp_end) return 0;
    std::lock_guard<std::mutex> lk(h->pool->mu);
    KvPool &pool = *h->pool;
    std::vector<int> moved;                            // device ids whose pages were copied out
    size_t lo_i = SIZE_MAX, hi_i = 0;
    hipError_t err = hipSuccess;
    for (int l = 0; l < m->NL && err == hipSuccess; l++) {
        if (!is_global(m, l) || h->slots[l] != h->full_pages) continue;
        for (int lp = lp_begin; lp < lp_end; lp++) {
            int &id = h->pt[l][lp];
            if (id < 0 || pool.refc[id] != 1) continue;
            const int hid = pool.host_alloc();
            if (hid < 0) { l = m->NL; break; }         // the host store is full: stop here
            err = hipMemcpyAsync(pool.hptr[hid], pool.ptr[id], pool.page_bytes, hipMemcpyDefault, h->stream);
            if (err != hipSuccess) { pool.release(HOST_ID(hid)); break; }
            moved.push_back(id);
            const size_t ti = h->pt_off[l] + lp;
            id = HOST_ID(hid);
            h->h_pt[ti] = pool.hptr[hid];
            lo_i = std::min(lo_i, ti); hi_i = std::max(hi_i, ti + 1);
        }
    }
    if (hi_i > lo_i) {
        // the copies complete before their device pages can be reused, and the
        // device table is updated before the step's kernels read it
        hipError_t e2 = hipMemcpyAsync(h->d_pt + lo_i, h->h_pt + lo_i, (hi_i - lo_i) * sizeof(float *),
                                       hipMemcpyHostToDevice, h->stream);
        const hipError_t e3 = hipStreamSynchronize(h->stream);
        if (e2 == hipSuccess) e2 = e3;
        if (e2 != hipSuccess) err = e2;
        else for (int id : moved) { pool.unref(id); pool.spills++; }
    }
    HIPCHK(err, "Ring-2 page spill");
    return 0;
}

// Bytes of the one-launch window attention's slots: models with window
// layers whose window spans at most WIN_MAXCH_HOST chunks (0: none).
size_t window_slots(const DevModel *m) {
    if (!m->gemma || m->SW <= 0 || (m->SW - 1) / 64 + 2 > WIN_MAXCH_HOST) return 0;
    return window_slot_bytes(m->NKV, m->HD, m->NH / m->NKV);
}

int alloc_scratch(sp_kvdecode_handle *h) {
    const DevModel *m = h->m;
    const int QD = m->NH * m->HD, KVD = m->NKV * m->HD;
    h->max_chunks = (h->pmax + 15) / 16 + 2;
    h->attn_cap = attn_capacity(m->HD, m->NH / m->NKV);
    h->win_cap = window_capacity(m->HD, m->NH / m->NKV);
    struct Item { void **p; size_t n; };
    const size_t part_bytes = (size_t)m->NH * h->max_chunks * m->HD * 8;
    const size_t ml_bytes = (size_t)m->NH * h->max_chunks * 16;
    const size_t z_bytes = (size_t)m->NH * h->max_chunks * 16 * 4;   // one int32 per (q-head, position)
    const int amb = argmax_blocks(m->V);
    h->acc_rows = std::max(std::max(QD + 2 * KVD, 2 * m->FF), std::max(m->E, m->V));
    Item items[] = {
        {(void **)&h->gacc, (size_t)h->acc_rows * 8}, {(void **)&h->gcnt, (size_t)h->acc_rows * 4},
        {(void **)&h->x0, (size_t)m->E * 4}, {(void **)&h->x1, (size_t)m->E * 4}, {(void **)&h->q, (size_t)QD * 4},
        {(void **)&h->k, (size_t)KVD * 4}, {(void **)&h->v, (size_t)KVD * 4}, {(void **)&h->qr, (size_t)QD * 4},
        {(void **)&h->ao, (size_t)QD * 4}, {(void **)&h->ap, (size_t)m->E * 4}, {(void **)&h->gg, (size_t)m->FF * 4},
        {(void **)&h->uu, (size_t)m->FF * 4}, {(void **)&h->hh, (size_t)m->FF * 4}, {(void **)&h->dn, (size_t)m->E * 4},
        {(void **)&h->logits, (size_t)m->V * 4}, {(void **)&h->part, part_bytes}, {(void **)&h->part_ml, ml_bytes},
        {(void **)&h->zscratch, z_bytes}, {(void **)&h->counter, 64 * 4}, {(void **)&h->am_v, (size_t)amb * 4},
        {(void **)&h->am_i, (size_t)amb * 4}, {(void **)&h->am_cnt, 64}, {(void **)&h->gen_log, (size_t)h->pmax * 4 + 64},
        {(void **)&h->tokbuf, (size_t)h->pmax * 4 + 64}, {(void **)&h->rope, (size_t)m->HD * 2 * 4},
        {(void **)&h->vacc, (size_t)QD * 8 * VREP}, {(void **)&h->vacc_s, (size_t)m->NH * 8 * VREP},
        {(void **)&h->d_st, sizeof(DState) * 4}, {(void **)&h->vclamp, 64},
        {(void **)&h->stats, (size_t)m->NL * STAT_PER_LAYER * STAT_REP * sizeof(VecStat)},
        {(void **)&h->ss.wslot, window_slots(m)},
    };
    size_t tot = 0;
    for (auto &it : items) tot = align_up(tot + it.n, 256);
    HIPCHK(hipMalloc(&h->scratch, tot), "scratch alloc");
    // cleared on the handle's stream: a null-stream memset is not ordered
    // before the handle's (non-blocking) kernels
    HIPCHK(hipMemsetAsync(h->scratch, 0, tot, h->stream), "scratch clear");
    size_t off = 0;
    for (auto &it : items) { *it.p = (uint8_t *)h->scratch + off; off = align_up(off + it.n, 256); }
    h->ss.gacc = h->gacc; h->ss.gcnt = h->gcnt; h->ss.acc_rows = h->acc_rows;
    h->ss.part = h->part; h->ss.part_ml = h->part_ml; h->ss.counter = h->counter; h->ss.zscratch = h->zscratch;
    h->ss.vacc = h->vacc; h->ss.vacc_s = h->vacc_s; h->ss.stats = h->stats;
    if (!window_slots(m)) h->ss.wslot = nullptr;
    HIPCHK(hipHostMalloc(&h->h_st, sizeof(DState) * 4, hipHostMallocDefault), "pinned state alloc");
    HIPCHK(hipHostMalloc(&h->h_logits, (size_t)m->V * 4, hipHostMallocDefault), "pinned logits alloc");
    h->built = 1;
    return 0;
}

// Drop the batch buffers and captured graphs when the arithmetic mode changes
// (both are mode-specific); everything else of the handle is mode-independent.
void set_handle_mode(sp_kvdecode_handle *h, int mode) {
    if (h->mode == mode) return;
    h->mode = mode;
    free_graphs(h);
    if (h->b.buf || h->b.dbuf) {
        hipStreamSynchronize(h->stream);
        if (h->b.buf) hipFree(h->b.buf);
        if (h->b.dbuf) hipFree(h->b.dbuf);
        if (h->b.hstage) hipHostFree(h->b.hstage);
        h->b = sp_kvdecode_handle::Batch{};
    }
}

// A fresh pool when the stored row format changes (mode or codec, only before
// the first token): unmaps every page and rebuilds the empty tables.
int repage(sp_kvdecode_handle *h, const char *who) {
    const size_t want = page_bytes_of(h->m, h->mode, h->kvc);
    if (h->pool->page_bytes == want) return 0;
    if (h->pool.use_count() > 1) return fail("%s: the KV pages are shared with a fork", who);
    { std::lock_guard<std::mutex> pl(h->pool->mu); for (auto &v : h->pt) for (int id : v) h->pool->release(id); }
    h->pool = make_pool(h->m, h->mode, h->kvc, h->pool_growth);
    free_graphs(h);
    return build_tables(h);
}

void free_recall(sp_kvdecode_handle *h) {
    if (h->rec.buf) { hipStreamSynchronize(h->stream); hipFree(h->rec.buf); }
    h->rec = sp_kvdecode_handle::Recall{};
}

// The frozen +-1 projection of core/arm/arm.c:17-27 (SplitMix64 from the seed
// of include/sp/arm.h:49, element i = p * HD + d of R is +1 when the low bit of
// the i-th draw is set) as sign bits, row p at [p * HD/32].
std::vector<uint32_t> recall_sign_bits(int r, int HD) {
    std::vector<uint32_t> bits((size_t)r * HD / 32, 0u);
    uint64_t st = 0x5350524F4A2BULL;
    for (int i = 0; i < r * HD; i++) {
        uint64_t z = (st += 0x9E3779B97F4A7C15ULL);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        z ^= z >> 31;
        if (z & 1) bits[(size_t)i / 32] |= 1u << (i % 32);
    }
    return bits;
}

// The router's buffers for budget B (> 0), window W, sinks, r rows.  A recall
// set holds at most max(B, W + sink) positions (and at most pmax).
int alloc_recall(sp_kvdecode_handle *h, int B, int W, int sink, int r) {
    free_recall(h);
    if (B <= 0) return 0;
    const DevModel *m = h->m;
    auto &R = h->rec;
    const int P = h->pmax;
    R.lstride = std::min(P, std::max(std::min(B, P), std::min(W, P) + std::min(sink, P)));
    R.mchunks = (R.lstride + RECALL_CHUNK - 1) / RECALL_CHUNK;
    R.kstride = (int)align_up((size_t)P, 64);
    const size_t NH = m->NH, HD = m->HD, mc = R.mchunks, ls = R.lstride;
    struct Item { void **p; size_t n; };
    int ng = 0;
    for (int l = 0; l < m->NL; l++) ng += is_global(m, l) ? 1 : 0;
    R.side_layer = (size_t)P * m->NKV * r;
    Item items[] = {
        {(void **)&R.side, (size_t)ng * R.side_layer * 4},
        {(void **)&R.Rb, (size_t)r * HD / 8}, {(void **)&R.keys, NH * R.kstride * 4}, {(void **)&R.pq, NH * r * 4},
        {(void **)&R.lists, NH * ls * 4},
        {(void **)&R.zs, NH * ls * 4}, {(void **)&R.counts, NH * 4}, {(void **)&R.cmax, NH * mc * 4},
        {(void **)&R.counter, NH * 4}, {(void **)&R.vacc, NH * HD * 8}, {(void **)&R.vs, NH * 8},
        {(void **)&R.part, NH * mc * HD * 4}, {(void **)&R.psum, NH * mc * 4},
    };
    size_t tot = 0;
    for (auto &it : items) tot = align_up(tot + it.n, 256);
    void *buf = nullptr;
    HIPCHK(hipMalloc(&buf, tot), "recall buffers alloc");
    R.buf = buf;
    size_t off = 0;
    for (auto &it : items) { *it.p = (uint8_t *)buf + off; off = align_up(off + it.n, 256); }
    const std::vector<uint32_t> bits = recall_sign_bits(r, (int)HD);
    HIPCHK(hipMemsetAsync(buf, 0, tot, h->stream), "recall buffers clear");
    HIPCHK(hipMemcpyAsync(R.Rb, bits.data(), bits.size() * 4, hipMemcpyHostToDevice, h->stream), "recall projection upload");
    HIPCHK(hipStreamSynchronize(h->stream), "recall buffers");
    R.B = B; R.W = W; R.sink = sink; R.r = r;
    return 0;
}

// layer l's K sidecar array [pmax][NKV][r] (global layers; null otherwise)
float *side_of(const sp_kvdecode_handle *h, int l) {
    if (!h->rec.side || !is_global(h->m, l)) return nullptr;
    int g = 0;
    for (int i = 0; i < l; i++) g += is_global(h->m, i) ? 1 : 0;
    return h->rec.side + (size_t)g * h->rec.side_layer;
}

// The recall set's geometry at position pos (the device router's sel_geom,
// sp_arm_select's clamps): identity, sinks, candidate end, top-k, set size.
struct RecallGeom { bool ident; int sink, cand_hi, topk, m; };
RecallGeom recall_geom(const sp_kvdecode_handle::Recall &R, int pos) {
    RecallGeom g;
    g.ident = R.B <= 0 || pos + 1 <= R.B;
    const int W = std::min(R.W, pos + 1);
    g.sink = std::min(R.sink, pos + 1);
    g.cand_hi = std::min(std::max(pos + 1 - W, g.sink), pos + 1);
    g.topk = std::min(std::max(R.B - W - g.sink, 0), g.cand_hi - g.sink);
    g.m = g.ident ? pos + 1 : g.sink + g.topk + (pos + 1 - g.cand_hi);
    return g;
}

// A kept shell of m with this pmax and window ring, or null (caller holds g_mu).
// Its page tables are unmapped, its scratch in the between-launch state
// (zero accumulators and counters), its graphs still valid.
sp_kvdecode_handle *take_shell(DevModel *m, int pmax, int max_rewind) {
    for (size_t i = m->shells.size(); i-- > 0;) {
        sp_kvdecode_handle *h = m->shells[i];
        if (h->pmax == pmax && h->max_rewind == max_rewind) {
            m->shells.erase(m->shells.begin() + (ptrdiff_t)i);
            return h;
        }
    }
    return nullptr;
}
constexpr size_t MAX_SHELLS = 256;

void free_handle(sp_kvdecode_handle *h) {
    if (h->stream) hipStreamSynchronize(h->stream);
    free_graphs(h);
    if (h->rec.buf) hipFree(h->rec.buf);
    if (h->d_pt) hipFree(h->d_pt);
    if (h->h_pt) hipHostFree(h->h_pt);
    if (h->scratch) hipFree(h->scratch);
    if (h->b.buf) hipFree(h->b.buf);
    if (h->b.dbuf) hipFree(h->b.dbuf);
    if (h->b.hstage) hipHostFree(h->b.hstage);
    if (h->h_st) hipHostFree(h->h_st);
    if (h->h_logits) hipHostFree(h->h_logits);
    if (h->stream) hipStreamDestroy(h->stream);
    delete h;
}

// ------------------------------------------------------------ one step body
// route: global layers attend over the recall router's positions (decode
// steps of a handle with recall on; prefill attends densely)
struct StepShape { int logits, argmax, grid_global, grid_local, chunk_global, chunk_local, route, vchunk_global; };

int attn_chunks(const sp_kvdecode_handle *h, int pos_hi, StepShape &sh) {
    const DevModel *m = h->m;
    // global layers: the smallest chunk (a multiple of 16, from 64 to
    // ATTN_MAXCH) whose workgroups fit the device in R rounds, R as small as
    // possible: a launch a few workgroups over one round would run a second,
    // nearly empty round at the length of the first.  Below 64 positions a
    // workgroup's fixed costs (head preparation, the exchange, 4x more adds on
    // each accumulator) outweigh the extra parallelism: at the Qwen3-0.6B
    // shape and 4 352 positions, 32-position chunks took 27.3 us, 64 and 128
    // 19.4 us.
    const int per_head = std::max(1, (h->attn_cap > 0 ? h->attn_cap : 1024) / m->NKV);
    int cg = 64;
    for (int R = 1;; R++) {
        cg = 64;
        while (cg < ATTN_MAXCH && pos_hi / cg + 1 > R * per_head) cg += 16;
        if (pos_hi / cg + 1 <= R * per_head) break;
    }
    while ((pos_hi / cg + 1) > 4096) cg *= 2;
    sh.chunk_global = cg;
    sh.grid_global = pos_hi / cg + 1;
    // exact-mode V-sum: a head with many short score chunks sums V over k of
    // them per workgroup (about 24 V-sum workgroups per head, at most
    // ATTN_MAXCH positions), so fewer workgroups arrive on each head's
    // counter.  Qwen3-0.6B shape, 4 352 positions, 64-position score chunks:
    // V-sum chunks of 192 took the attention 19.4 -> 17.0 us (128: 17.5, 256:
    // 17.6); the Gemma-3-12B shape's 272- and 512-position chunks gain nothing.
    const int k = std::min(ATTN_MAXCH / cg, (sh.grid_global + 12) / 24);
    sh.vchunk_global = k >= 2 ? k * cg : 0;
    // window layers: 64-position chunks; a window of W positions touches at most
    // (W-1)/64 + 2 of them whatever its alignment
    const int cl = 64;
    sh.chunk_local = cl;
    const int span = m->SW > 0 ? std::min(m->SW, pos_hi + 1) : pos_hi + 1;
    sh.grid_local = std::min((span - 1) / cl + 2, pos_hi / cl + 1);
    return 0;
}

typedef void (*TimeCb)(void *ctx, int cls, bool begin);

RecallArgs recall_args(const sp_kvdecode_handle *h, int layer, float *const *pages, VecStat *stat_out) {
    const DevModel *m = h->m;
    const auto &R = h->rec;
    RecallArgs rc{};
    rc.pq = R.pq; rc.qr = h->qr; rc.pages = pages; rc.st = h->d_st; rc.ao = h->ao; rc.stat_out = stat_out;
    rc.side = side_of(h, layer);
    rc.keys = R.keys; rc.lists = R.lists; rc.counts = R.counts; rc.zs = R.zs; rc.cmax = R.cmax;
    rc.vacc = R.vacc; rc.vs = R.vs; rc.part = R.part; rc.psum = R.psum; rc.counter = R.counter;
    rc.kstride = R.kstride; rc.lstride = R.lstride; rc.mchunks = R.mchunks;
    rc.score_blocks = std::min(RECALL_SCORE_BLOCKS, (h->pmax + 255) / 256);
    rc.NH = m->NH; rc.NKV = m->NKV; rc.HD = m->HD; rc.r = R.r; rc.B = R.B; rc.W = R.W; rc.sink = R.sink;
    rc.mode = h->mode; rc.ascale = 1.0f / sqrtf((float)m->HD);
    rc.Rb = R.Rb; rc.kvsel = h->recall_kvsel;
    return rc;
}

void enqueue_body(sp_kvdecode_handle *h, const StepShape &sh, TimeCb cb, void *ctx, const StepScratch &ss) {
    const DevModel *m = h->m;
    hipStream_t s = h->stream;
    const int QD = m->NH * m->HD, KVD = m->NKV * m->HD;
    auto T = [&](int cls, bool b) { if (cb) cb(ctx, cls, b); };
    T(8, true);
    // per layer: statistics of ao, ap, hh, dn, accumulated by the kernel that
    // writes the vector and read by the GEMV that consumes it
    VecStat *stat = ss.stats;
    auto st = [&](int l, int k) { return stat + ((size_t)l * STAT_PER_LAYER + k) * STAT_REP; };
    // the embedding and the step's rotation tables (independent) in one launch
    launch_embed_rope(m->embd, h->d_st, h->tokbuf, h->x1, m->gemma ? sqrtf((float)m->E) : 0.0f,
                      stat, m->NL * STAT_PER_LAYER * STAT_REP, m->HD, h->mode,
                      m->freq_global, m->gemma ? m->freq_local : m->freq_global, h->rope, s);
    T(8, false);
    for (int l = 0; l < m->NL; l++) {
        const DevLayer &d = m->L[l];
        const bool glob = is_global(m, l);
        GemvArgs g{};
        g.accbuf = ss.gacc; g.gcnt = ss.gcnt; g.acc_rows = ss.acc_rows;
        g.mode = h->mode; g.cols = m->E; g.act = ACT_NONE; g.nseg = 3;
        if (l == 0) { g.pro.kind = PRO_NORM; g.pro.x = h->x1; }
        else {
            g.pro.kind = PRO_RESID; g.pro.x = h->x0; g.pro.delta = h->dn; g.pro.x_out = h->x1;
            g.pro.post_w = m->gemma ? m->L[l - 1].post_ffw : nullptr;
            g.pro.stat = st(l - 1, STAT_DN);
        }
        g.pro.norm_w = d.attn_norm; g.pro.n = m->E; g.pro.eps = m->eps;
        g.seg[0] = {d.q, h->q}; g.seg[1] = {d.k, h->k}; g.seg[2] = {d.v, h->v};
        T(0, true); launch_gemv(g, QD + 2 * KVD, s); T(0, false);

        AttnArgs a{};
        a.q = h->q; a.k = h->k; a.v = h->v; a.q_norm = d.q_norm; a.k_norm = d.k_norm; a.qr = h->qr;
        a.pages = h->d_pt + h->pt_off[l];
        a.ring_pages = h->slots[l] == h->full_pages ? 0 : h->slots[l];
        a.ao = h->ao; a.part = ss.part; a.part_ml = ss.part_ml; a.counter = ss.counter; a.zscratch = ss.zscratch;
        a.vacc = ss.vacc; a.vacc_s = ss.vacc_s;
        a.st = h->d_st; a.rope_cs = h->rope + ((m->gemma && !glob) ? m->HD : 0);
        a.NH = m->NH; a.NKV = m->NKV; a.HD = m->HD;
        a.win = (m->gemma && !glob) ? m->SW : -1;
        a.max_chunks = h->max_chunks; a.mode = h->mode; a.kvc = h->kvc; a.eps = m->eps;
        a.zstride = h->max_chunks * 16; a.nt = 0; a.vclamp = h->vclamp;
        a.base = (m->gemma && !glob) ? 10000.0f : m->base;
        a.ascale = 1.0f / sqrtf((float)m->HD);
        a.chunk = glob ? sh.chunk_global : sh.chunk_local;
        a.vchunk = glob ? sh.vchunk_global : 0;
        a.stat_out = st(l, STAT_AO);
        // window layers in exact mode: one launch when its grid, 4 times over
        // (one per hardware queue), fits the device at once
        a.wslot = ss.wslot;
        a.one_launch = h->win_one && a.win >= 0 && h->mode == EXACT && ss.wslot && sh.grid_local <= WIN_MAXCH_HOST &&
                       (size_t)sh.grid_local * m->NKV * 4 <= (size_t)h->win_cap;
        if (h->rec.B > 0 && a.win < 0) { a.rec_R = h->rec.Rb; a.rec_r = h->rec.r; a.rec_side = side_of(h, l); }
        const int cls = (glob || a.win < 0) ? 5 : 6, grid = glob ? sh.grid_global : sh.grid_local;
        if (sh.route && a.rec_r) {
            a.rec_pq = h->rec.pq;                       // the router's query projections
            T(7, true); launch_qk_prep(a, s); T(7, false);
            T(cls, true); launch_recall_attention(recall_args(h, l, a.pages, a.stat_out), s); T(cls, false);
        } else if (attention_fuses_prep(a)) {
            T(cls, true); launch_prep_attention(a, grid, s); T(cls, false);
        } else {
            T(7, true); launch_qk_prep(a, s); T(7, false);
            T(cls, true); launch_attention(a, grid, s); T(cls, false);
        }

        GemvArgs o{};
        o.accbuf = ss.gacc; o.gcnt = ss.gcnt; o.acc_rows = ss.acc_rows;
        o.mode = h->mode; o.cols = QD; o.act = ACT_NONE; o.nseg = 1;
        o.pro.kind = PRO_PLAIN; o.pro.x = h->ao; o.pro.n = QD; o.pro.stat = st(l, STAT_AO);
        o.seg[0] = {d.o, h->ap}; o.stat_out = st(l, STAT_AP);
        T(1, true); launch_gemv(o, m->E, s); T(1, false);

        GemvArgs f{};
        f.accbuf = ss.gacc; f.gcnt = ss.gcnt; f.acc_rows = ss.acc_rows;
        f.mode = h->mode; f.cols = m->E; f.act = m->gemma ? ACT_GELU : ACT_SILU; f.nseg = 2;
        f.pro.kind = PRO_RESID; f.pro.x = h->x1; f.pro.delta = h->ap; f.pro.post_w = d.post_attn;
        f.pro.norm_w = d.ffn_norm; f.pro.x_out = h->x0; f.pro.n = m->E; f.pro.eps = m->eps;
        f.seg[0] = {d.gate, h->gg}; f.seg[1] = {d.up, h->uu}; f.act_out = h->hh;
        f.pro.stat = st(l, STAT_AP); f.stat_out = st(l, STAT_HH);
        T(2, true); launch_gemv(f, m->FF, s); T(2, false);

        GemvArgs dd{};
        dd.accbuf = ss.gacc; dd.gcnt = ss.gcnt; dd.acc_rows = ss.acc_rows;
        dd.mode = h->mode; dd.cols = m->FF; dd.act = ACT_NONE; dd.nseg = 1;
        dd.pro.kind = PRO_PLAIN; dd.pro.x = h->hh; dd.pro.n = m->FF; dd.pro.stat = st(l, STAT_HH);
        dd.seg[0] = {d.down, h->dn}; dd.stat_out = st(l, STAT_DN);
        T(3, true); launch_gemv(dd, m->E, s); T(3, false);
    }
    if (sh.logits) {
        GemvArgs lm{};
        lm.accbuf = ss.gacc; lm.gcnt = ss.gcnt; lm.acc_rows = ss.acc_rows;
        lm.mode = h->mode; lm.cols = m->E; lm.act = ACT_NONE; lm.nseg = 1;
        lm.pro.kind = PRO_RESID; lm.pro.x = h->x0; lm.pro.delta = h->dn;
        lm.pro.post_w = m->gemma ? m->L[m->NL - 1].post_ffw : nullptr;
        lm.pro.norm_w = m->out_norm; lm.pro.x_out = nullptr; lm.pro.n = m->E; lm.pro.eps = m->eps;
        lm.pro.stat = st(m->NL - 1, STAT_DN);
        lm.seg[0] = {m->out, h->logits};
        T(4, true); launch_gemv(lm, m->V, s); T(4, false);
        if (sh.argmax) {
            T(8, true);
            launch_argmax(h->logits, m->V, h->am_v, h->am_i, h->am_cnt, h->d_st, h->gen_log, argmax_blocks(m->V), s);
            T(8, false);
        }
    } else {
        launch_advance(h->d_st, s);
    }
}

// ------------------------------------------------------------ batched prefill
// Tokens go through the model TB at a time: per layer one staging kernel per
// GEMM input (one workgroup per token), the int8-MFMA GEMMs, and the decode
// attention kernels with a token grid dimension.  Each token's K/V and every
// intermediate are the same integers/floats a decode step computes.
constexpr int PREFILL_TB = 128;
constexpr size_t GEMM_PART_BYTES = (size_t)64 << 20;    // split-K partials of the batched GEMMs
constexpr int GEMM_TILE_COUNTERS = 8192;

bool batch_supported(const sp_kvdecode_handle *h) {
    const DevModel *m = h->m;
    const int G = m->NH / m->NKV;
    const bool attn_ok = (m->HD == 64 || m->HD == 128 || m->HD == 256) && (G == 2 || G == 4);
    if (!attn_ok || m->E % 256 || m->FF % 256 || (m->NH * m->HD) % 256) return false;
    for (const DevLayer &d : m->L)
        for (const DevW *w : {&d.q, &d.k, &d.v, &d.o, &d.gate, &d.up, &d.down})
            if (!gemm_supported(*w)) return false;
    return true;
}

int alloc_batch(sp_kvdecode_handle *h) {
    if (h->b.buf) return 0;
    const DevModel *m = h->m;
    auto &b = h->b;
    const size_t TB = PREFILL_TB, QD = (size_t)m->NH * m->HD, KVD = (size_t)m->NKV * m->HD;
    const size_t E = m->E, FF = m->FF;
    b.TB = PREFILL_TB;
    b.mcb = h->pmax / 64 + 2;                // batched attention chunks hold >= 64 positions
    const size_t nmax = std::max(std::max(E, QD), FF);
    struct Item { void **p; size_t n; };
    Item items[] = {
        {(void **)&b.x0, TB * E * 4}, {(void **)&b.x1, TB * E * 4}, {(void **)&b.q, TB * QD * 4},
        {(void **)&b.k, TB * KVD * 4}, {(void **)&b.v, TB * KVD * 4}, {(void **)&b.qr, TB * QD * 4},
        {(void **)&b.ao, TB * QD * 4}, {(void **)&b.ap, TB * E * 4}, {(void **)&b.gg, TB * FF * 4},
        {(void **)&b.uu, TB * FF * 4}, {(void **)&b.hh, TB * FF * 4}, {(void **)&b.dn, TB * E * 4},
        {(void **)&b.rope, TB * 2 * m->HD * 4}, {(void **)&b.planes, 3 * (nmax / 32) * TB * 32},
        {(void **)&b.sh, TB * 4}, {(void **)&b.counter, TB * m->NKV * 4},
        {(void **)&b.zs, TB * m->NH * (size_t)h->max_chunks * 16 * 4},
        {(void **)&b.part_ml, TB * m->NH * (size_t)b.mcb * 16},
        {(void **)&b.part, h->mode == FLOAT ? TB * m->NH * (size_t)b.mcb * m->HD * 4 : 256},
        {(void **)&b.vacc, TB * QD * 8 * VREP}, {(void **)&b.vacc_s, TB * m->NH * 8 * VREP},
        {(void **)&b.gpart, GEMM_PART_BYTES}, {(void **)&b.gcnt, GEMM_TILE_COUNTERS * 4},
    };
    size_t tot = 0;
    for (auto &it : items) tot = align_up(tot + it.n, 256);
    HIPCHK(hipMalloc(&b.buf, tot), "prefill batch alloc");
    HIPCHK(hipMemsetAsync(b.buf, 0, tot, h->stream), "prefill batch clear");     // ordered before the batch kernels
    size_t off = 0;
    for (auto &it : items) { *it.p = (uint8_t *)b.buf + off; off = align_up(off + it.n, 256); }
    return 0;
}

// T tokens through the model on h's stream and batch buffers.  One session's
// prefill: positions pos0.., tokens in h->tokbuf, h's page tables.  Several
// sessions' decode (multi): token t's id, position and page tables come from
// b.toks / b.tpos / b.tpages; then the LM head writes b.logits and b.next.
int run_batch(sp_kvdecode_handle *h, int T, int pos0, int pos_hi, bool multi, TimeCb cb = nullptr, void *ctx = nullptr) {
    const DevModel *m = h->m;
    auto &b = h->b;
    hipStream_t s = h->stream;
    const int QD = m->NH * m->HD, KVD = m->NKV * m->HD, TP = (T + 31) / 32 * 32;
    auto TM = [&](int cls, bool begin) { if (cb) cb(ctx, cls, begin); };
    TM(8, true);
    launch_embed_batch(m->embd, h->tokbuf, pos0, T, b.x1, m->gemma ? sqrtf((float)m->E) : 0.0f, s,
                       multi ? b.toks : nullptr);
    launch_rope_table_batch(pos0, T, m->HD, h->mode, m->base, m->gemma ? 10000.0f : m->base,
                            m->freq_global, m->gemma ? m->freq_local : m->freq_global, b.rope, s,
                            multi ? b.tpos : nullptr);
    TM(8, false);
    auto stage = [&](int kind, const float *x, const float *delta, const float *post_w, const float *norm_w,
                     float *x_out, int n) {
        StageArgs a{};
        a.pro.kind = kind; a.pro.x = x; a.pro.delta = delta; a.pro.post_w = post_w; a.pro.norm_w = norm_w;
        a.pro.x_out = x_out; a.pro.n = n; a.pro.eps = m->eps;
        a.planes = b.planes; a.sh = b.sh; a.T = T; a.TP = TP; a.mode = h->mode;
        launch_stage(a, s);
    };
    auto gemm = [&](int cols) {
        GemmArgs g{};
        g.cols = cols; g.planes = b.planes; g.sh = b.sh; g.T = T; g.TP = TP; g.mode = h->mode; g.act = ACT_NONE;
        g.part = b.gpart; g.part_cap = GEMM_PART_BYTES / 8; g.cnt = b.gcnt; g.cnt_cap = GEMM_TILE_COUNTERS;
        return g;
    };
    for (int l = 0; l < m->NL; l++) {
        const DevLayer &d = m->L[l];
        const bool glob = is_global(m, l);
        TM(0, true);
        if (l == 0) stage(PRO_NORM, b.x1, nullptr, nullptr, d.attn_norm, nullptr, m->E);
        else stage(PRO_RESID, b.x0, b.dn, m->gemma ? m->L[l - 1].post_ffw : nullptr, d.attn_norm, b.x1, m->E);
        GemmArgs g = gemm(m->E);
        g.nseg = 3; g.seg[0] = {d.q, b.q}; g.seg[1] = {d.k, b.k}; g.seg[2] = {d.v, b.v};
        launch_gemm(g, QD + 2 * KVD, s);
        TM(0, false);

        AttnArgs a{};
        a.q = b.q; a.k = b.k; a.v = b.v; a.q_norm = d.q_norm; a.k_norm = d.k_norm; a.qr = b.qr;
        a.pages = h->d_pt + h->pt_off[l];
        a.ring_pages = h->slots[l] == h->full_pages ? 0 : h->slots[l];
        a.ao = b.ao; a.part = b.part; a.part_ml = b.part_ml; a.counter = b.counter; a.zscratch = b.zs;
        a.vacc = b.vacc; a.vacc_s = b.vacc_s;
        a.st = nullptr; a.rope_cs = b.rope + ((m->gemma && !glob) ? m->HD : 0);
        a.NH = m->NH; a.NKV = m->NKV; a.HD = m->HD;
        a.win = (m->gemma && !glob) ? m->SW : -1;
        a.max_chunks = b.mcb; a.zstride = h->max_chunks * 16; a.mode = h->mode; a.kvc = h->kvc; a.eps = m->eps;
        a.base = (m->gemma && !glob) ? 10000.0f : m->base;
        a.ascale = 1.0f / sqrtf((float)m->HD);
        a.nt = T; a.pos0 = pos0; a.rope_stride = 2 * m->HD; a.vclamp = h->vclamp;
        if (multi) {
            a.tpos = b.tpos; a.tpages = b.tpages + (size_t)l * b.TB;
            if (glob || a.win < 0) { a.work = b.work; a.nwork = b.nwork; }
        }
        else if (h->rec.B > 0 && a.win < 0) {                   // prefill: the sidecar
            a.rec_R = h->rec.Rb; a.rec_r = h->rec.r; a.rec_side = side_of(h, l);
        }
        // batched decode over sessions: the longest chunks the kernels take,
        // so that the many sessions' rows make fewer, longer workgroups
        a.chunk = (glob || a.win < 0) ? (multi ? ATTN_MAXCH : 256) : 64;
        TM(7, true); launch_qk_prep(a, s); TM(7, false);
        // chunks of the batch's longest span: a window of W positions covers at
        // most (W-1)/chunk + 2 chunks whatever its alignment
        int nch = pos_hi / a.chunk + 1;
        if (a.win >= 0) nch = std::min(nch, (a.win - 1) / a.chunk + 2);
        TM(a.win >= 0 ? 6 : 5, true); launch_attention(a, nch, s); TM(a.win >= 0 ? 6 : 5, false);

        TM(1, true);
        stage(PRO_PLAIN, b.ao, nullptr, nullptr, nullptr, nullptr, QD);
        GemmArgs o = gemm(QD);
        o.nseg = 1; o.seg[0] = {d.o, b.ap};
        launch_gemm(o, m->E, s);
        TM(1, false);

        TM(2, true);
        stage(PRO_RESID, b.x1, b.ap, d.post_attn, d.ffn_norm, b.x0, m->E);
        GemmArgs f = gemm(m->E);
        f.nseg = 2; f.act = m->gemma ? ACT_GELU : ACT_SILU;
        f.seg[0] = {d.gate, b.gg}; f.seg[1] = {d.up, b.uu}; f.act_out = b.hh;
        launch_gemm(f, m->FF, s);
        TM(2, false);

        TM(3, true);
        stage(PRO_PLAIN, b.hh, nullptr, nullptr, nullptr, nullptr, m->FF);
        GemmArgs dd = gemm(m->FF);
        dd.nseg = 1; dd.seg[0] = {d.down, b.dn};
        launch_gemm(dd, m->E, s);
        TM(3, false);
    }
    if (multi) {
        // LM head over the T rows, then each row's greedy token
        TM(4, true);
        stage(PRO_RESID, b.x0, b.dn, m->gemma ? m->L[m->NL - 1].post_ffw : nullptr, m->out_norm, nullptr, m->E);
        GemmArgs lm = gemm(m->E);
        lm.nseg = 1; lm.seg[0] = {m->out, b.logits};
        launch_gemm(lm, m->V, s);
        launch_argmax_rows(b.logits, m->V, T, b.next, s);
        TM(4, false);
    }
    if (take_launch_error("batched pass")) return 1;
    HIPCHK(hipGetLastError(), "batch launch");
    return 0;
}

int prefill_batch(sp_kvdecode_handle *h, int pos0, int T) { return run_batch(h, T, pos0, pos0 + T - 1, false); }

constexpr size_t MAX_GRAPHS = 64;

// The captured step graph of this shape, capturing it on first use.  Past
// MAX_GRAPHS entries the cache is emptied after the stream has drained (a
// graph exec still running must not be destroyed).
int graph_for(sp_kvdecode_handle *h, const StepShape &sh, hipGraphExec_t *out) {
    sp_kvdecode_handle::GKey key{sh.logits, sh.argmax, sh.grid_global, sh.grid_local, sh.chunk_global, sh.route};
    auto it = h->graphs.find(key);
    if (it != h->graphs.end()) { *out = it->second; return 0; }
    hipGraph_t g;
    HIPCHK(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal), "graph capture begin");
    enqueue_body(h, sh, nullptr, nullptr, h->ss);
    const hipError_t ec = hipStreamEndCapture(h->stream, &g);
    if (take_launch_error("step capture")) { if (ec == hipSuccess) hipGraphDestroy(g); return 1; }
    HIPCHK(ec, "graph capture end");
    hipGraphExec_t ge;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    HIPCHK(e, "graph instantiate");
    if (h->graphs.size() >= MAX_GRAPHS) {
        const hipError_t es = hipStreamSynchronize(h->stream);
        free_graphs(h);
        if (es != hipSuccess) { hipGraphExecDestroy(ge); HIPCHK(es, "graph cache eviction"); }
    }
    h->graphs.insert({key, ge});
    *out = ge;
    return 0;
}

int run_body(sp_kvdecode_handle *h, const StepShape &sh) {
    if (!h->use_graph) {
        enqueue_body(h, sh, nullptr, nullptr, h->ss);
        if (take_launch_error("step launch")) return 1;
        HIPCHK(hipGetLastError(), "kernel launch");
        return 0;
    }
    hipGraphExec_t ge;
    if (graph_for(h, sh, &ge)) return 1;
    HIPCHK(hipGraphLaunch(ge, h->stream), "graph launch");
    return 0;
}

// round the attention grids up so one captured graph serves a run of positions
StepShape shape_for(const sp_kvdecode_handle *h, int pos, int logits, int argmax, bool decode = true) {
    StepShape sh{};
    sh.logits = logits; sh.argmax = argmax; sh.route = decode && h->rec.B > 0;
    const int hi = std::min(h->pmax - 1, ((pos / 256) + 1) * 256 - 1);
    attn_chunks(h, h->use_graph ? hi : pos, sh);
    return sh;
}

int set_state(sp_kvdecode_handle *h, int pos, int tok, int drive) {
    // one pinned slot per in-flight step: callers synchronize before reusing it
    h->h_st->pos = pos; h->h_st->tok = tok; h->h_st->drive = drive; h->h_st->pad = 0;
    HIPCHK(hipMemcpyAsync(h->d_st, h->h_st, sizeof(DState), hipMemcpyHostToDevice, h->stream), "state upload");
    return 0;
}

int check_tok(const sp_kvdecode_handle *h, int32_t tok) {
    if (tok < 0 || tok >= h->m->V) return fail("sp_hipkv: token %s%lld out of vocabulary range", "", (long long)tok);
    return 0;
}

int step_one(sp_kvdecode_handle *h, int32_t tok, int want_logits) {
    if (check_tok(h, tok)) return 1;
    if (h->dpos >= h->pmax) return fail("sp_hipkv: context full (dpos == pmax %s%lld)", "", (long long)h->pmax);
    if (ensure_pages(h, h->dpos, h->dpos + 1) || ring2_spill(h, h->dpos)) return 1;
    if (set_state(h, h->dpos, tok, DRIVE_HOST)) return 1;
    StepShape sh = shape_for(h, h->dpos, want_logits, 0);
    if (run_body(h, sh)) return 1;
    return 0;
}

}  // namespace

// ------------------------------------------------------------ allocation-free decode step
// Step scratch shared by every allocation-free decode step on a device
// (sp_hipkv_decode_step_noalloc).  Host code reaches it only through the
// device address hipGetSymbolAddress returns for the current device.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {

__global__ void k_zero_words(uint32_t *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[NOALLOC_MAX_DEVICES];        // per device: the device address of `scratch`
// per device: held by an allocation-free step from carving the scratch to its
// final synchronize, so calls that share a GPU's array run one after another
std::mutex g_noalloc_mu[NOALLOC_MAX_DEVICES];

// Carve a step scratch for h out of base[0, NOALLOC_SCRATCH_BYTES); false when
// h's shape needs more.  *used = bytes to clear.
bool carve_noalloc(const sp_kvdecode_handle *h, uint8_t *base, StepScratch &ss, size_t *used) {
    const DevModel *m = h->m;
    const size_t QD = (size_t)m->NH * m->HD, mc = (size_t)h->max_chunks;
    const bool exact = h->mode == EXACT;
    struct Item { void **p; size_t n; };
    Item items[] = {
        {(void **)&ss.gacc, (size_t)h->acc_rows * 8}, {(void **)&ss.gcnt, (size_t)h->acc_rows * 4},
        {(void **)&ss.part, exact ? 256 : (size_t)m->NH * mc * m->HD * 8}, {(void **)&ss.part_ml, (size_t)m->NH * mc * 16},
        {(void **)&ss.zscratch, exact ? (size_t)m->NH * mc * 16 * 4 : 256}, {(void **)&ss.counter, 256},
        {(void **)&ss.vacc, QD * 8 * VREP}, {(void **)&ss.vacc_s, (size_t)m->NH * 8 * VREP},
        {(void **)&ss.stats, (size_t)m->NL * STAT_PER_LAYER * STAT_REP * sizeof(VecStat)},
        {(void **)&ss.wslot, exact ? window_slots(m) : 0},
    };
    size_t off = 0;
    for (auto &it : items) { *it.p = base + off; off = align_up(off + it.n, 256); }
    if (!exact || !window_slots(m)) ss.wslot = nullptr;
    ss.acc_rows = h->acc_rows;
    *used = off;
    return off <= NOALLOC_SCRATCH_BYTES;
}

}  // namespace

// ================================================================ C ABI
extern "C" {

int sp_hipkv_open(const void *qm_opaque, int pmax, sp_kvdecode_handle **out) {
    if (!out) return fail("sp_hipkv_open: null out%s");
    *out = nullptr;
    if (!qm_opaque || pmax <= 0) return fail("sp_hipkv_open: null model or pmax <= 0%s");
    if (pmax > PMAX_LIMIT) return fail("sp_hipkv_open: pmax exceeds the backend's limit of %s%lld positions", "", (long long)PMAX_LIMIT);
    std::lock_guard<std::mutex> lk(g_mu);
    const qwen3_model *qm = (const qwen3_model *)qm_opaque;
    if (!g_models.count(qm)) {
        // the model is validated on the host before any device is touched
        DevModel *chk = model_get(qm, false);
        if (!chk) return 1;
        delete chk;
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
        return fail("sp_hipkv_open: no HIP device visible (this backend runs on MI355X / gfx950)%s");
    DevModel *m = model_get(qm);
    if (!m) return 1;
    auto new_pool = [m]() { return make_pool(m, FLOAT, KVC_PLAIN, 0); };
    if (sp_kvdecode_handle *sh = take_shell(m, pmax, 0)) {
        // a kept shell: reset to the open defaults, unmapped tables
        set_handle_mode(sh, FLOAT);
        if (sh->kvc != KVC_PLAIN) { sh->kvc = KVC_PLAIN; free_graphs(sh); }   // graphs bake in the codec
        sh->use_graph = 1; sh->use_batch = 1; sh->dpos = 0; sh->hwm = 0; sh->pool_growth = 0;
        if (sh->recall_kvsel) { sh->recall_kvsel = 0; free_graphs(sh); }
        if (!sh->win_one) { sh->win_one = 1; free_graphs(sh); }
        sh->ring2 = 0;
        if (sh->rec.B) { free_recall(sh); free_graphs(sh); }
        sh->pool = new_pool();
        if (hipMemsetAsync(sh->vclamp, 0, sizeof(int), sh->stream) != hipSuccess) {
            free_handle(sh); model_put(m); return fail("sp_hipkv_open: clamp counter reset failed%s");
        }
        size_t tot = 0; for (int l = 0; l < m->NL; l++) tot += (size_t)sh->slots[l];
        for (size_t i = 0; i < tot; i++) sh->h_pt[i] = nullptr;
        if (hipMemcpyAsync(sh->d_pt, sh->h_pt, tot * sizeof(float *), hipMemcpyHostToDevice, sh->stream) != hipSuccess ||
            hipStreamSynchronize(sh->stream) != hipSuccess) {
            free_handle(sh); model_put(m); return fail("sp_hipkv_open: page table reset failed%s");
        }
        *out = sh;
        return 0;
    }
    std::unique_ptr<sp_kvdecode_handle> h(new sp_kvdecode_handle);
    h->m = m; h->pmax = pmax;
    h->pool = new_pool();
    if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess) { model_put(m); return fail("sp_hipkv_open: stream creation failed%s"); }
    if (build_tables(h.get()) || alloc_scratch(h.get())) { free_handle(h.release()); model_put(m); return 1; }
    *out = h.release();
    return 0;
}

void sp_hipkv_close(sp_kvdecode_handle *h) {
    if (!h) return;
    std::lock_guard<std::mutex> lk(g_mu);
    const bool idle = !h->stream || hipStreamSynchronize(h->stream) == hipSuccess;
    if (h->pool) { std::lock_guard<std::mutex> pl(h->pool->mu); for (auto &v : h->pt) for (int id : v) h->pool->release(id); }
    h->pool.reset();
    for (auto &v : h->pt) std::fill(v.begin(), v.end(), -1);
    DevModel *m = h->m;
    if (idle && h->built && m->refs > 1 && m->shells.size() < MAX_SHELLS) {
        // other handles keep the model alive: keep this one as a shell
        h->dpos = 0; h->hwm = 0;
        m->shells.push_back(h);
        m->refs--;
        return;
    }
    free_handle(h);
    model_put(m);
}


int sp_hipkv_position(const sp_kvdecode_handle *h) { return h ? h->dpos : -1; }

int sp_hipkv_rewind(sp_kvdecode_handle *h, int n) {
    if (!h) return fail("sp_hipkv_rewind: null handle%s");
    if (n < 0 || n > h->dpos) return fail("sp_hipkv_rewind: n %s%lld exceeds the resident position", "", (long long)n);
    if (h->ring_pages > 0) {
        // window layers keep ring_pages*PAGE positions: the window of the new
        // position must not have been overwritten by a later position
        const int cap = h->ring_pages * PAGE - h->m->SW;
        if (h->hwm - (h->dpos - n) > cap)
            return fail("sp_hipkv_rewind: rewinding %s%lld positions leaves the window ring (set a larger max_rewind)", "", (long long)n);
    }
    h->dpos -= n;          // stale slots past dpos are overwritten by the next steps
    return 0;
}

int sp_hipkv_prefill(sp_kvdecode_handle *h, const int32_t *tokens, int n_tok) {
    if (!h || (!tokens && n_tok > 0) || n_tok < 0) return fail("sp_hipkv_prefill: bad argument%s");
    if (n_tok > h->pmax - h->dpos) return fail("sp_hipkv_prefill: context full%s");
    if (n_tok == 0) return 0;
    for (int i = 0; i < n_tok; i++) if (check_tok(h, tokens[i])) return 1;
    if (ensure_pages(h, h->dpos, h->dpos + n_tok)) return 1;
    HIPCHK(hipStreamSynchronize(h->stream), "prefill staging");
    HIPCHK(hipMemcpyAsync(h->tokbuf + h->dpos, tokens, (size_t)n_tok * 4, hipMemcpyHostToDevice, h->stream),
           "prefill tokens");
    if (h->use_batch && batch_supported(h)) {
        if (alloc_batch(h)) return 1;
        // window layers on a ring: writing position q reuses the page slot of
        // the page ring_pages back, i.e. drops positions up to q - ring*PAGE + PAGE-1;
        // a batch must not drop positions its first token still attends to
        int tb = h->b.TB;
        if (h->ring_pages > 0) tb = std::min(tb, h->ring_pages * PAGE - h->m->SW - (PAGE - 1));
        if (tb < 1) tb = 1;
        for (int i = 0; i < n_tok; i += tb)
            if (prefill_batch(h, h->dpos + i, std::min(tb, n_tok - i))) return 1;
    } else {
        if (set_state(h, h->dpos, 0, DRIVE_STREAM)) return 1;
        for (int i = 0; i < n_tok; i++) {
            StepShape sh = shape_for(h, h->dpos + i, 0, 0, false);
            if (run_body(h, sh)) return 1;
        }
    }
    HIPCHK(hipStreamSynchronize(h->stream), "prefill");
    h->dpos += n_tok;
    h->hwm = std::max(h->hwm, h->dpos);
    return 0;
}

// Several sessions of one model decode one token each, batched: the GEMMs run
// once for all rows (int8 MFMA), attention reads each session's own pages.
// cb/ctx: optional per-kernel-class event hooks (run_batch's classes).
static int decode_batch_impl(sp_kvdecode_handle *const *hs, int n, const int32_t *tokens, float *logits,
                             int32_t *next_tokens, TimeCb cb, void *ctx) {
    if (!hs || !tokens || n <= 0) return fail("sp_hipkv_decode_batch: bad argument%s");
    sp_kvdecode_handle *L = hs[0];
    if (!L) return fail("sp_hipkv_decode_batch: null handle%s");
    const DevModel *m = L->m;
    for (int i = 0; i < n; i++) {
        sp_kvdecode_handle *h = hs[i];
        if (!h || h->m != m) return fail("sp_hipkv_decode_batch: handles must share one model%s");
        if (h->mode != L->mode || h->kvc != L->kvc || h->pmax != L->pmax || h->slots != L->slots)
            return fail("sp_hipkv_decode_batch: handles differ in mode, KV codec, pmax or window ring%s");
        if (check_tok(h, tokens[i])) return 1;
        if (h->dpos >= h->pmax) return fail("sp_hipkv_decode_batch: context full (dpos == pmax %s%lld)", "", (long long)h->pmax);
        for (int j = 0; j < i; j++)
            if (hs[j] == h) return fail("sp_hipkv_decode_batch: a handle appears twice%s");
    }
    bool routed = false;
    for (int i = 0; i < n; i++) routed |= hs[i]->rec.B > 0;
    const bool batched = batch_supported(L) && gemm_supported(m->out) && !routed;
    if (!batched) {                                   // shapes the GEMM does not take, recall: one step each
        if (cb) return fail("sp_hipkv_decode_batch_times: no batched path for this model shape or with recall%s");
        for (int i = 0; i < n; i++) {
            if (step_one(hs[i], tokens[i], 1)) return 1;
            if (logits) HIPCHK(hipMemcpyAsync(logits + (size_t)i * m->V, hs[i]->logits, (size_t)m->V * 4,
                                              hipMemcpyDeviceToHost, hs[i]->stream), "logits download");
            if (next_tokens) {
                launch_argmax_rows(hs[i]->logits, m->V, 1, hs[i]->am_i, hs[i]->stream);
                HIPCHK(hipMemcpyAsync(next_tokens + i, hs[i]->am_i, 4, hipMemcpyDeviceToHost, hs[i]->stream), "token download");
            }
            HIPCHK(hipStreamSynchronize(hs[i]->stream), "decode step");
            hs[i]->dpos++;
            hs[i]->hwm = std::max(hs[i]->hwm, hs[i]->dpos);
        }
        return 0;
    }
    for (int i = 0; i < n; i++) if (ensure_pages(hs[i], hs[i]->dpos, hs[i]->dpos + 1)) return 1;
    if (alloc_batch(L)) return 1;
    auto &b = L->b;
    const int TB = b.TB;
    if (!b.dbuf) {
        const size_t lb = (size_t)TB * m->V * 4, nb = (size_t)TB * 4, pb = (size_t)m->NL * TB * sizeof(void *);
        b.wcap = TB * (L->pmax / ATTN_MAXCH + 2);
        const size_t wb = (size_t)b.wcap * sizeof(int2);
        HIPCHK(hipMalloc(&b.dbuf, align_up(lb, 256) + 3 * align_up(nb, 256) + align_up(pb, 256) + wb), "batch decode alloc");
        uint8_t *p = (uint8_t *)b.dbuf;
        b.logits = (float *)p; p += align_up(lb, 256);
        b.next = (int *)p; p += align_up(nb, 256);
        b.toks = (int *)p; p += align_up(nb, 256);
        b.tpos = (int *)p; p += align_up(nb, 256);
        b.tpages = (float *const **)p; p += align_up(pb, 256);
        b.work = (int2 *)p;
        HIPCHK(hipHostMalloc(&b.hstage, 2 * nb + pb + wb, hipHostMallocDefault), "batch decode staging");
    }
    for (int g0 = 0; g0 < n; g0 += TB) {
        const int T = std::min(TB, n - g0);
        int *htok = (int *)b.hstage, *hpos = htok + TB;
        float *const **hpg = (float *const **)(hpos + TB);
        int2 *hwork = (int2 *)(hpg + (size_t)m->NL * TB);
        int pos_hi = 0;
        b.nwork = 0;
        for (int t = 0; t < T; t++) {
            sp_kvdecode_handle *h = hs[g0 + t];
            htok[t] = tokens[g0 + t]; hpos[t] = h->dpos;
            pos_hi = std::max(pos_hi, h->dpos);
            for (int l = 0; l < m->NL; l++) hpg[(size_t)l * TB + t] = h->d_pt + h->pt_off[l];
            // full-context layers: ATTN_MAXCH-position chunks up to this session's position
            for (int c = 0; c <= h->dpos / ATTN_MAXCH && b.nwork < b.wcap; c++) hwork[b.nwork++] = make_int2(t, c);
        }
        HIPCHK(hipMemcpyAsync(b.toks, htok, (size_t)TB * 4, hipMemcpyHostToDevice, L->stream), "batch tokens");
        HIPCHK(hipMemcpyAsync(b.tpos, hpos, (size_t)TB * 4, hipMemcpyHostToDevice, L->stream), "batch positions");
        HIPCHK(hipMemcpyAsync((void *)b.tpages, hpg, (size_t)m->NL * TB * sizeof(void *), hipMemcpyHostToDevice, L->stream),
               "batch page tables");
        HIPCHK(hipMemcpyAsync(b.work, hwork, (size_t)b.nwork * sizeof(int2), hipMemcpyHostToDevice, L->stream),
               "batch work items");
        if (run_batch(L, T, 0, pos_hi, true, cb, ctx)) return 1;
        if (logits) HIPCHK(hipMemcpyAsync(logits + (size_t)g0 * m->V, b.logits, (size_t)T * m->V * 4,
                                          hipMemcpyDeviceToHost, L->stream), "batch logits download");
        if (next_tokens) HIPCHK(hipMemcpyAsync(next_tokens + g0, b.next, (size_t)T * 4, hipMemcpyDeviceToHost, L->stream),
                                "batch tokens download");
        HIPCHK(hipStreamSynchronize(L->stream), "batch decode");
        for (int t = 0; t < T; t++) {
            sp_kvdecode_handle *h = hs[g0 + t];
            h->dpos++;
            h->hwm = std::max(h->hwm, h->dpos);
        }
    }
    return 0;
}

int sp_hipkv_decode_batch(sp_kvdecode_handle *const *hs, int n, const int32_t *tokens, float *logits,
                          int32_t *next_tokens) {
    return decode_batch_impl(hs, n, tokens, logits, next_tokens, nullptr, nullptr);
}

int sp_hipkv_decode_batch_times(sp_kvdecode_handle *const *hs, int n, const int32_t *tokens, int32_t *next_tokens,
                                double ms[SP_HIPKV_NCLASS], long long launches[SP_HIPKV_NCLASS],
                                double bytes[SP_HIPKV_NCLASS]) {
    if (!hs || n <= 0 || !hs[0] || !ms || !launches || !bytes) return fail("sp_hipkv_decode_batch_times: bad argument%s");
    const DevModel *m = hs[0]->m;
    for (int i = 0; i < SP_HIPKV_NCLASS; i++) { ms[i] = 0; launches[i] = 0; bytes[i] = 0; }
    // algorithmic bytes: each weight matrix once for all rows (Q4B codes + f16
    // scales), per row its GEMM input (f32) and output (f32); attention reads
    // each row's K/V span; q/k prep reads the projections and writes q and K/V
    const double rows_n = std::min(n, PREFILL_TB);
    auto wb = [](const DevW &w) { return (double)w.rows * (w.cols / 2) + 2.0 * w.rows * w.nblk; };
    auto io = [&](const DevW &w) { return rows_n * 4.0 * ((double)w.cols + w.rows); };
    double per[SP_HIPKV_NCLASS] = {0};
    const int QD = m->NH * m->HD, KVD = m->NKV * m->HD;
    for (const DevLayer &d : m->L) {
        per[0] += wb(d.q) + wb(d.k) + wb(d.v) + io(d.q) + 4.0 * rows_n * (d.k.rows + d.v.rows);
        per[1] += wb(d.o) + io(d.o);
        per[2] += wb(d.gate) + wb(d.up) + io(d.gate) + 8.0 * rows_n * d.up.rows;
        per[3] += wb(d.down) + io(d.down);
        per[7] += rows_n * 8.0 * (QD + 2.0 * KVD);
    }
    per[4] = wb(m->out) + io(m->out) + rows_n * 4.0 * m->V;
    per[8] = rows_n * ((double)(m->embd.cols / 2 + m->embd.nblk * 2) + 4.0 * m->E);
    const double kvb = (double)m->NKV * kv_row_payload(m, hs[0]->mode, hs[0]->kvc) * 2;
    for (int i = 0; i < n; i++) {
        const int pos = hs[i]->dpos;
        for (int l = 0; l < m->NL; l++) {
            const bool glob = is_global(m, l);
            const int s0 = (!glob && m->SW > 0 && pos - m->SW + 1 > 0) ? pos - m->SW + 1 : 0;
            bytes[(glob || m->SW <= 0) ? 5 : 6] += kvb * (pos - s0 + 1);
        }
    }
    struct Ctx { hipStream_t s; std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> ev; hipEvent_t cur; };
    Ctx c; c.s = hs[0]->stream;
    auto cb = [](void *vp, int cls, bool begin) {
        Ctx *cc = (Ctx *)vp;
        hipEvent_t e; hipEventCreate(&e); hipEventRecord(e, cc->s);
        if (begin) cc->cur = e; else cc->ev.push_back({cls, {cc->cur, e}});
    };
    const int rc = decode_batch_impl(hs, n, tokens, nullptr, next_tokens, cb, &c);
    for (auto &e : c.ev) {
        float t = 0; hipEventElapsedTime(&t, e.second.first, e.second.second);
        ms[e.first] += t; launches[e.first]++;
        hipEventDestroy(e.second.first); hipEventDestroy(e.second.second);
    }
    if (rc) return rc;
    const double groups = (double)((n + PREFILL_TB - 1) / PREFILL_TB);
    for (int k = 0; k < SP_HIPKV_NCLASS; k++) if (k != 5 && k != 6) bytes[k] = per[k] * groups;
    return 0;
}

int sp_hipkv_decode_step(sp_kvdecode_handle *h, int32_t token, float *logits) {
    if (!h || !logits) return fail("sp_hipkv_decode_step: null argument%s");
    if (step_one(h, token, 1)) return 1;
    HIPCHK(hipMemcpyAsync(h->h_logits, h->logits, (size_t)h->m->V * 4, hipMemcpyDeviceToHost, h->stream), "logits download");
    HIPCHK(hipStreamSynchronize(h->stream), "decode step");
    memcpy(logits, h->h_logits, (size_t)h->m->V * 4);
    h->dpos++;
    h->hwm = std::max(h->hwm, h->dpos);
    return 0;
}

int sp_hipkv_decode_step_noalloc(sp_kvdecode_handle *h, int32_t token, float *logits) {
    if (!h || !logits) return fail("sp_hipkv_decode_step_noalloc: null argument%s");
    if (check_tok(h, token)) return 1;
    if (h->dpos >= h->pmax) return fail("sp_hipkv_decode_step_noalloc: context full (dpos == pmax %s%lld)", "", (long long)h->pmax);
    int dev = 0;
    HIPCHK(hipGetDevice(&dev), "sp_hipkv_decode_step_noalloc: device query");
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return fail("sp_hipkv_decode_step_noalloc: device index %s%lld out of range", "", (long long)dev);
    // every call on this device shares its array: the lock orders them, and
    // each call has finished on the device (its final synchronize) before the
    // next one clears the array
    std::lock_guard<std::mutex> serial(g_noalloc_mu[dev]);
    uint8_t *base = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (!g_scratch_ptr[dev]) {
            void *p = nullptr;
            HIPCHK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "sp_hipkv_decode_step_noalloc: scratch address");
            g_scratch_ptr[dev] = (uint8_t *)p;
        }
        base = g_scratch_ptr[dev];
    }
    StepScratch ss;
    size_t used = 0;
    if (!carve_noalloc(h, base, ss, &used))
        return fail("sp_hipkv_decode_step_noalloc: this model and pmax need %s%lld bytes of step scratch, above the "
                    "33554432-byte static buffer", "", (long long)used);
    // the pages of this position must exist already (or come from free pages
    // of the pool): nothing may grow the pool here
    if (ensure_pages(h, h->dpos, h->dpos + 1, false)) return 1;
    if (set_state(h, h->dpos, token, DRIVE_HOST)) return 1;
    // accumulators and counters start at zero (the previous call on this
    // device left its own contents)
    hipLaunchKernelGGL(k_zero_words, dim3(256), dim3(256), 0, h->stream, (uint32_t *)base, used / 4);
    enqueue_body(h, shape_for(h, h->dpos, 1, 0), nullptr, nullptr, ss);    // plain launches: no graph instantiation
    if (take_launch_error("sp_hipkv_decode_step_noalloc")) return 1;
    HIPCHK(hipGetLastError(), "sp_hipkv_decode_step_noalloc: launch");
    HIPCHK(hipMemcpyAsync(h->h_logits, h->logits, (size_t)h->m->V * 4, hipMemcpyDeviceToHost, h->stream), "logits download");
    HIPCHK(hipStreamSynchronize(h->stream), "sp_hipkv_decode_step_noalloc");
    memcpy(logits, h->h_logits, (size_t)h->m->V * 4);
    h->dpos++;
    h->hwm = std::max(h->hwm, h->dpos);
    return 0;
}

int sp_hipkv_set_mode(sp_kvdecode_handle *h, int exact) {
    if (!h) return fail("sp_hipkv_set_mode: null handle%s");
    const int m = exact ? EXACT : FLOAT;
    if (m == h->mode) return 0;
    if (h->dpos != 0) return fail("sp_hipkv_set_mode: the mode is fixed once tokens are resident%s");
    // exact V-sum: weights <= 2^22, |vq| < 2^23, so int64 totals hold 2^18 positions
    if (m == EXACT && h->pmax > (1 << 18)) return fail("sp_hipkv_set_mode: exact mode holds at most %s%lld positions", "", (long long)(1 << 18));
    if (m == FLOAT && h->kvc == KVC_SPINOR && h->rec.B > 0)
        return fail("sp_hipkv_set_mode: recall in float mode reads plain K/V rows (not Spinor code rows)%s");
    set_handle_mode(h, m);
    return repage(h, "sp_hipkv_set_mode");
}

int sp_hipkv_set_kv_codec(sp_kvdecode_handle *h, int codec) {
    if (!h) return fail("sp_hipkv_set_kv_codec: null handle%s");
    if (codec != KVC_PLAIN && codec != KVC_SPINOR) return fail("sp_hipkv_set_kv_codec: unknown codec%s");
    if (codec == h->kvc) return 0;
    if (h->dpos != 0) return fail("sp_hipkv_set_kv_codec: the codec is fixed once tokens are resident%s");
    if (codec == KVC_SPINOR && h->m->HD != 64 && h->m->HD != 128 && h->m->HD != 256)
        return fail("sp_hipkv_set_kv_codec: Spinor KV serves head_dim 64, 128 and 256%s");
    if (codec == KVC_SPINOR && h->mode == FLOAT && h->rec.B > 0)
        return fail("sp_hipkv_set_kv_codec: recall in float mode reads plain K/V rows (not Spinor code rows)%s");
    h->kvc = codec;
    free_graphs(h);
    return repage(h, "sp_hipkv_set_kv_codec");
}

int sp_hipkv_set_max_rewind(sp_kvdecode_handle *h, int max_rewind) {
    if (!h || max_rewind < 0) return fail("sp_hipkv_set_max_rewind: bad argument%s");
    if (h->dpos != 0) return fail("sp_hipkv_set_max_rewind: only before the first token%s");
    { std::lock_guard<std::mutex> pl(h->pool->mu); for (auto &v : h->pt) for (int id : v) h->pool->release(id); }
    h->max_rewind = max_rewind;
    free_graphs(h);
    return build_tables(h);
}

int sp_hipkv_set_pool_growth(sp_kvdecode_handle *h, int pages) {
    if (!h || pages < 0) return fail("sp_hipkv_set_pool_growth: bad argument%s");
    h->pool_growth = pages;
    std::lock_guard<std::mutex> pl(h->pool->mu);
    h->pool->pages_per_chunk = pool_growth_pages(h->pool->page_bytes, pages);
    return 0;
}

int sp_hipkv_set_graph(sp_kvdecode_handle *h, int on) {
    if (!h) return fail("sp_hipkv_set_graph: null handle%s");
    h->use_graph = on ? 1 : 0;
    if (!on) free_graphs(h);
    return 0;
}

int sp_hipkv_set_window_one_launch(sp_kvdecode_handle *h, int on) {
    if (!h) return fail("sp_hipkv_set_window_one_launch: null handle%s");
    if ((on ? 1 : 0) == h->win_one) return 0;
    h->win_one = on ? 1 : 0;
    free_graphs(h);                          // the captured steps bake the attention launches
    return 0;
}

int sp_hipkv_set_batch_prefill(sp_kvdecode_handle *h, int on) {
    if (!h) return fail("sp_hipkv_set_batch_prefill: null handle%s");
    h->use_batch = on ? 1 : 0;
    return 0;
}

int sp_hipkv_set_recall(sp_kvdecode_handle *h, int B, int W, int sink, int r) {
    if (!h) return fail("sp_hipkv_set_recall: null handle%s");
    if (B < 0 || W < 0 || sink < 0) return fail("sp_hipkv_set_recall: negative budget, window or sink count%s");
    if (B > 0 && (r < 1 || r > 64)) return fail("sp_hipkv_set_recall: projection rows r must lie in [1, 64]%s");
    if (B == 0) r = 0;
    if (B == h->rec.B && W == h->rec.W && sink == h->rec.sink && r == h->rec.r) return 0;
    if (h->dpos != 0) return fail("sp_hipkv_set_recall: recall is fixed once tokens are resident%s");
    if (B > 0 && h->m->HD != 64 && h->m->HD != 128 && h->m->HD != 256)
        return fail("sp_hipkv_set_recall: recall serves head_dim 64, 128 and 256%s");
    if (B > 0 && h->m->NH / h->m->NKV > RECALL_MAX_GROUP)
        return fail("sp_hipkv_set_recall: recall serves at most 8 q heads per kv head%s");
    if (B > 0 && h->mode == FLOAT && h->kvc == KVC_SPINOR)
        return fail("sp_hipkv_set_recall: recall in float mode reads plain K/V rows (not Spinor code rows)%s");
    if (h->pool.use_count() > 1) return fail("sp_hipkv_set_recall: the KV pages are shared with a fork%s");
    free_graphs(h);
    if (alloc_recall(h, B, W, sink, r)) return 1;
    return repage(h, "sp_hipkv_set_recall");
}

int sp_hipkv_set_recall_kvsel(sp_kvdecode_handle *h, int on) {
    if (!h) return fail("sp_hipkv_set_recall_kvsel: null handle%s");
    if ((on ? 1 : 0) == h->recall_kvsel) return 0;
    if (on && h->m->HD > 256) return fail("sp_hipkv_set_recall_kvsel: head_dim above 256%s");
    h->recall_kvsel = on ? 1 : 0;
    free_graphs(h);                          // the captured steps bake the router's arguments
    return 0;
}

int sp_hipkv_set_ring2(sp_kvdecode_handle *h, int on) {
    if (!h) return fail("sp_hipkv_set_ring2: null handle%s");
    h->ring2 = on ? 1 : 0;
    return 0;
}

int sp_hipkv_ring2_stats(const sp_kvdecode_handle *h, long long out[4]) {
    if (!h || !out) return fail("sp_hipkv_ring2_stats: null argument%s");
    std::lock_guard<std::mutex> lk(h->pool->mu);
    long long host = 0, dev = 0;
    for (const auto &v : h->pt)
        for (int id : v) { host += id <= -2; dev += id >= 0; }
    out[0] = host; out[1] = dev; out[2] = h->pool->spills; out[3] = h->pool->fetches;
    return 0;
}

int sp_hipkv_read_recall_sidecar(const sp_kvdecode_handle *h, int layer, int p0, int n, float *out) {
    if (!h || !out || layer < 0 || layer >= h->m->NL || p0 < 0 || n < 0 || p0 + n > h->dpos)
        return fail("sp_hipkv_read_recall_sidecar: bad argument%s");
    if (h->rec.B <= 0) return fail("sp_hipkv_read_recall_sidecar: recall is off%s");
    const DevModel *m = h->m;
    if (!is_global(m, layer)) return fail("sp_hipkv_read_recall_sidecar: window layers keep no sidecar%s");
    const int NKV = m->NKV, r = h->rec.r;
    HIPCHK(hipStreamSynchronize(h->stream), "sidecar read sync");
    if (n > 0)
        HIPCHK(hipMemcpy(out, side_of(h, layer) + (size_t)p0 * NKV * r, (size_t)n * NKV * r * 4, hipMemcpyDeviceToHost),
               "sidecar read");
    return 0;
}

int sp_hipkv_fork(const sp_kvdecode_handle *p, sp_kvdecode_handle **out) {
    if (!p || !out) return fail("sp_hipkv_fork: null argument%s");
    *out = nullptr;
    std::unique_ptr<sp_kvdecode_handle> h;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        p->m->refs++;
        h.reset(take_shell(p->m, p->pmax, p->max_rewind));
    }
    if (h) {
        set_handle_mode(h.get(), p->mode);
    } else {
        h.reset(new sp_kvdecode_handle);
        h->m = p->m; h->pmax = p->pmax; h->max_rewind = p->max_rewind; h->mode = p->mode;
        if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess) {
            std::lock_guard<std::mutex> lk(g_mu); model_put(p->m); return fail("sp_hipkv_fork: stream creation failed%s");
        }
        if (build_tables(h.get()) || alloc_scratch(h.get())) {
            std::lock_guard<std::mutex> lk(g_mu); free_handle(h.release()); model_put(p->m); return 1;
        }
    }
    if (h->kvc != p->kvc) { h->kvc = p->kvc; free_graphs(h.get()); }        // a recycled shell's graphs
    if (h->rec.B != p->rec.B || h->rec.W != p->rec.W || h->rec.sink != p->rec.sink || h->rec.r != p->rec.r) {
        free_graphs(h.get());
        if (alloc_recall(h.get(), p->rec.B, p->rec.W, p->rec.sink, p->rec.r)) {
            sp_hipkv_close(h.release()); return 1;
        }
    }
    h->pool = p->pool; h->dpos = p->dpos; h->hwm = p->hwm;
    if (p->rec.side && p->dpos > 0) {
        // the sidecar array is per handle: the child starts with the parent's
        hipStreamSynchronize(p->stream);
        int ng = 0;
        for (int l = 0; l < h->m->NL; l++) ng += is_global(h->m, l) ? 1 : 0;
        if (hipMemcpyAsync(h->rec.side, p->rec.side, (size_t)ng * p->rec.side_layer * 4, hipMemcpyDeviceToDevice,
                           h->stream) != hipSuccess) {
            sp_hipkv_close(h.release()); return fail("sp_hipkv_fork: sidecar copy failed%s");
        }
    }
    if (hipMemsetAsync(h->vclamp, 0, sizeof(int), h->stream) != hipSuccess) {
        sp_hipkv_close(h.release()); return fail("sp_hipkv_fork: clamp counter reset failed%s");
    }
    h->use_batch = p->use_batch; h->use_graph = p->use_graph; h->pool_growth = p->pool_growth;
    if (h->recall_kvsel != p->recall_kvsel) { h->recall_kvsel = p->recall_kvsel; free_graphs(h.get()); }
    if (h->win_one != p->win_one) { h->win_one = p->win_one; free_graphs(h.get()); }
    h->ring2 = p->ring2;
    hipStreamSynchronize(p->stream);
    // share every mapped page (copy-on-write on the next append into it)
    {
        std::lock_guard<std::mutex> pl(h->pool->mu);
        for (int l = 0; l < h->m->NL; l++) {
            for (int s = 0; s < h->slots[l]; s++) {
                const int id = p->pt[l][s];
                h->pt[l][s] = id;
                h->pool->retain(id);
                h->h_pt[h->pt_off[l] + s] = h->pool->page_ptr(id);
            }
        }
    }
    size_t tot = 0; for (int l = 0; l < h->m->NL; l++) tot += (size_t)h->slots[l];
    if (hipMemcpyAsync(h->d_pt, h->h_pt, tot * sizeof(float *), hipMemcpyHostToDevice, h->stream) != hipSuccess ||
        hipStreamSynchronize(h->stream) != hipSuccess) {
        sp_hipkv_close(h.release()); return fail("sp_hipkv_fork: page table upload failed%s");
    }
    *out = h.release();
    return 0;
}

sp_status sp_hipkv_attach(sp_session *s, int pmax, int exact) {
    if (!s || pmax <= 0) { sp_set_error("sp_hipkv_attach: bad argument"); return SP_EBADARG; }
    size_t spos = 0;
    if (sp_session_position(s, &spos) != SP_OK) return SP_EBADARG;
    if (spos != 0) {
        // a fresh handle starts at dpos 0: attaching it to a session with
        // history would decode at the wrong position
        sp_set_error("sp_hipkv_attach: the session already holds tokens (attach before the first prefill)");
        return SP_EBADSTATE;
    }
    sp_kvdecode_handle *h = nullptr;
    if (sp_hipkv_open(sp_session_qwen3_model(s), pmax, &h)) return SP_EBACKEND_OOM;
    if (exact && sp_hipkv_set_mode(h, 1)) { sp_hipkv_close(h); return SP_EBADSTATE; }
    if ((spx_session_flags(s) & (SP_KV_SPINOR | SP_KV_SPINOR_REF)) && sp_hipkv_set_kv_codec(h, KVC_SPINOR)) {
        sp_hipkv_close(h); return SP_EUNSUPPORTED;
    }
    sp_status st = sp_session_register_kvdecode_backend(s, h, &sp_hipkv_dispatch);
    if (st != SP_OK) { sp_hipkv_close(h); return st; }
    st = spx_session_own_kvdecode(s, 1);
    return st != SP_OK ? st : spx_session_route_kv_lifecycle(s, 1);
}

int sp_hipkv_greedy(sp_kvdecode_handle *h, int32_t first_token, int n, int32_t *out_tokens, double *device_ms) {
    if (!h || n < 0) return fail("sp_hipkv_greedy: bad argument%s");
    if (check_tok(h, first_token)) return 1;
    if (n > h->pmax - h->dpos) return fail("sp_hipkv_greedy: context full%s");
    if (n == 0) { if (device_ms) *device_ms = 0; return 0; }
    if (ensure_pages(h, h->dpos, h->dpos + n) || ring2_spill(h, h->dpos)) return 1;
    if (set_state(h, h->dpos, first_token, DRIVE_GREEDY)) return 1;
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0), "event"); HIPCHK(hipEventCreate(&e1), "event");
    // pre-instantiate the graphs this run needs so capture is outside the timed
    // region (runs over more windows than the cache holds re-capture later ones)
    for (int w = h->dpos / 256; w <= (h->dpos + n - 1) / 256 && h->use_graph; w++) {
        StepShape sh = shape_for(h, std::max(h->dpos, w * 256), 1, 1);
        hipGraphExec_t ge;
        if (graph_for(h, sh, &ge)) return 1;
    }
    // the argmax kernel logs each position's token into gen_log[pos]
    HIPCHK(hipEventRecord(e0, h->stream), "event record");
    for (int i = 0; i < n; i++) {
        StepShape sh = shape_for(h, h->dpos + i, 1, 1);
        if (run_body(h, sh)) return 1;
    }
    HIPCHK(hipEventRecord(e1, h->stream), "event record");
    HIPCHK(hipStreamSynchronize(h->stream), "greedy run");
    float ms = 0; hipEventElapsedTime(&ms, e0, e1);
    if (device_ms) *device_ms = ms;
    hipEventDestroy(e0); hipEventDestroy(e1);
    if (out_tokens)
        HIPCHK(hipMemcpy(out_tokens, h->gen_log + h->dpos, (size_t)n * 4, hipMemcpyDeviceToHost), "token log read");
    h->dpos += n;
    h->hwm = std::max(h->hwm, h->dpos);
    return 0;
}

int sp_hipkv_kernel_times(sp_kvdecode_handle *h, int32_t first_token, int n, double ms[SP_HIPKV_NCLASS],
                          long long launches[SP_HIPKV_NCLASS], double bytes[SP_HIPKV_NCLASS]) {
    if (!h || n <= 0 || !ms || !launches || !bytes) return fail("sp_hipkv_kernel_times: bad argument%s");
    if (check_tok(h, first_token)) return 1;
    if (n > h->pmax - h->dpos) return fail("sp_hipkv_kernel_times: context full%s");
    if (ensure_pages(h, h->dpos, h->dpos + n) || ring2_spill(h, h->dpos)) return 1;
    if (set_state(h, h->dpos, first_token, DRIVE_GREEDY)) return 1;
    // the GEMV classes (0-4, one launch each) are timed by events the launch
    // itself records at the kernel's start and end; the others (several
    // kernels, or not GEMVs) by events recorded on the stream around them
    struct Ctx { hipStream_t s; bool routed; std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> ev; hipEvent_t cur, cur2; };
    Ctx c; c.s = h->stream; c.routed = h->rec.B > 0;
    auto cb = [](void *vp, int cls, bool begin) {
        Ctx *cc = (Ctx *)vp;
        // GEMVs (0-4) and the score/V-sum or one-launch attention (5, 6; not
        // the routed recall kernels): events recorded by the launches
        const bool gemv = cls <= 4, attn = (cls == 5 && !cc->routed) || cls == 6;
        if (gemv || attn) {
            if (begin) {
                hipEventCreate(&cc->cur); hipEventCreate(&cc->cur2);
                if (gemv) gemv_time_next(cc->cur, cc->cur2); else attn_time_next(cc->cur, cc->cur2);
            } else {
                gemv_time_next(nullptr, nullptr); attn_time_next(nullptr, nullptr);   // consumed unless a launch failed
                cc->ev.push_back({cls, {cc->cur, cc->cur2}});
            }
            return;
        }
        hipEvent_t e; hipEventCreate(&e); hipEventRecord(e, cc->s);
        if (begin) cc->cur = e; else cc->ev.push_back({cls, {cc->cur, e}});
    };
    for (int i = 0; i < SP_HIPKV_NCLASS; i++) { ms[i] = 0; launches[i] = 0; bytes[i] = 0; }
    const DevModel *m = h->m;
    const double kvb = (double)m->NKV * kv_row_payload(m, h->mode, h->kvc) * 2;     // K+V bytes per position per layer
    // algorithmic bytes of one GEMV: Q4B codes + f16 block scales, input and output vectors
    auto gb = [](const DevW &w) {
        return (double)w.rows * (w.cols / 2) + 2.0 * w.rows * w.nblk + 4.0 * w.cols + 4.0 * w.rows;
    };
    double per_step[SP_HIPKV_NCLASS] = {0};
    for (const DevLayer &d : m->L) {
        per_step[0] += gb(d.q) + gb(d.k) + gb(d.v) - 8.0 * d.k.cols;   // one shared input vector
        per_step[1] += gb(d.o);
        per_step[2] += gb(d.gate) + gb(d.up) + 4.0 * d.gate.rows - 4.0 * d.gate.cols;   // + act output
        per_step[3] += gb(d.down);
    }
    per_step[4] = gb(m->out);
    per_step[8] = (double)(m->embd.cols / 2 + m->embd.nblk * 2) + 4.0 * m->V;   // one embedding row + logits read by argmax
    for (int i = 0; i < n; i++) {
        const int pos = h->dpos + i;
        StepShape sh = shape_for(h, pos, 1, 1);
        enqueue_body(h, sh, cb, &c, h->ss);
        if (take_launch_error("timed step")) { hipStreamSynchronize(h->stream); return 1; }
        for (int k = 0; k < SP_HIPKV_NCLASS; k++) bytes[k] += per_step[k];
        for (int l = 0; l < m->NL; l++) {
            const bool glob = is_global(m, l);
            if (glob && h->rec.B > 0) {
                // recall: each q head scans its kv head's sidecar over the
                // candidates and reads the K and V rows of its recall set
                const RecallGeom g = recall_geom(h->rec, pos);
                const double scan = (g.ident || !g.topk) ? 0.0 : (double)(g.cand_hi - g.sink) * h->rec.r * 4.0;
                bytes[5] += (double)m->NH * (scan + (double)g.m * kv_row_payload(m, h->mode, h->kvc) * 2);
                continue;
            }
            const int s0 = (!glob && m->SW > 0 && pos - m->SW + 1 > 0) ? pos - m->SW + 1 : 0;
            bytes[(glob || m->SW <= 0) ? 5 : 6] += kvb * (pos - s0 + 1);
        }
    }
    HIPCHK(hipStreamSynchronize(h->stream), "timed run");
    for (auto &e : c.ev) {
        float t = 0; hipEventElapsedTime(&t, e.second.first, e.second.second);
        ms[e.first] += t; launches[e.first]++;
        hipEventDestroy(e.second.first); hipEventDestroy(e.second.second);
    }
    h->dpos += n;
    h->hwm = std::max(h->hwm, h->dpos);
    return 0;
}

int sp_hipkv_read_kv(const sp_kvdecode_handle *h, int layer, int p0, int n, float *k, float *v) {
    if (!h || !k || !v || layer < 0 || layer >= h->m->NL || p0 < 0 || n < 0 || p0 + n > h->dpos)
        return fail("sp_hipkv_read_kv: bad argument%s");
    const DevModel *m = h->m;
    const int HD = m->HD, NKV = m->NKV, S = h->slots[layer], KVD = NKV * HD;
    HIPCHK(hipStreamSynchronize(h->stream), "kv read sync");
    std::vector<float> page(h->pool->page_bytes / 4);
    const size_t RB = kv_row_bytes(m, h->mode, h->kvc);
    // one stored row -> HD floats (code rows decode to code * chunk multiplier)
    auto row_out = [&](const uint8_t *row, float *dst) {
        if (RB == (size_t)HD * 4) { memcpy(dst, row, (size_t)HD * 4); return; }
        const float *mul = (const float *)(row + HD);
        for (int e = 0; e < HD; e++) dst[e] = (float)(int8_t)row[e] * mul[spn_block_of(HD, e)];
    };
    for (int lp = p0 / PAGE; lp <= (p0 + n - 1) / PAGE && n > 0; lp++) {
        const int slot = S == h->full_pages ? lp : lp % S;
        const int id = h->pt[layer][slot];
        if (id == NO_PAGE) return fail("sp_hipkv_read_kv: position not resident%s");
        HIPCHK(hipMemcpy(page.data(), h->pool->page_ptr(id), h->pool->page_bytes, hipMemcpyDefault), "kv page read");
        const int a = std::max(p0, lp * PAGE), b = std::min(p0 + n, (lp + 1) * PAGE);
        for (int p = a; p < b; p++)
            for (int hh = 0; hh < NKV; hh++) {
                const uint8_t *pb = (const uint8_t *)page.data();
                row_out(pb + ((size_t)hh * PAGE + p % PAGE) * RB, k + (size_t)(p - p0) * KVD + (size_t)hh * HD);
                row_out(pb + ((size_t)NKV * PAGE + (size_t)hh * PAGE + p % PAGE) * RB, v + (size_t)(p - p0) * KVD + (size_t)hh * HD);
            }
    }
    return 0;
}

int sp_hipkv_write_kv(sp_kvdecode_handle *h, int layer, int p0, int n, const float *k, const float *v) {
    if (!h || !k || !v || layer < 0 || layer >= h->m->NL || p0 < 0 || n < 0 || p0 > h->dpos || n > h->pmax - p0)
        return fail("sp_hipkv_write_kv: bad argument (positions must start at or below the resident position "
                    "and end within pmax)%s");
    if (kv_row_bytes(h->m, h->mode, h->kvc) != (size_t)h->m->HD * 4)
        return fail("sp_hipkv_write_kv: the handle stores Spinor code rows (float mode with SP_KV_SPINOR)%s");
    if (h->rec.B > 0) return fail("sp_hipkv_write_kv: recall is on (the K sidecar is formed by the step itself)%s");
    if (n == 0) return 0;
    const DevModel *m = h->m;
    const int HD = m->HD, NKV = m->NKV, S = h->slots[layer], KVD = NKV * HD;
    if (ensure_pages(h, p0, p0 + n)) return 1;
    // each touched page goes through one pinned page image: read back first
    // when the write covers only part of it, then one copy to the device
    const size_t RB = (size_t)HD * 4, half = (size_t)NKV * PAGE * RB, img = 2 * half;
    uint8_t *stage = nullptr;
    HIPCHK(hipHostMalloc((void **)&stage, img, hipHostMallocDefault), "kv write staging alloc");
    int rc = 0;
    for (int lp = p0 / PAGE; lp <= (p0 + n - 1) / PAGE && !rc; lp++) {
        const int slot = S == h->full_pages ? lp : lp % S;
        uint8_t *page = (uint8_t *)h->pool->ptr[h->pt[layer][slot]];
        const int a = std::max(p0, lp * PAGE), b = std::min(p0 + n, (lp + 1) * PAGE);
        hipError_t e = hipSuccess;
        if (b - a < PAGE) {
            e = hipMemcpyAsync(stage, page, img, hipMemcpyDeviceToHost, h->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
        }
        for (int p = a; p < b && e == hipSuccess; p++)
            for (int hh = 0; hh < NKV; hh++) {
                const size_t src = (size_t)(p - p0) * KVD + (size_t)hh * HD;
                const size_t dst = ((size_t)hh * PAGE + (p & (PAGE - 1))) * RB;
                memcpy(stage + dst, k + src, RB);
                memcpy(stage + half + dst, v + src, RB);
            }
        if (e == hipSuccess) e = hipMemcpyAsync(page, stage, img, hipMemcpyHostToDevice, h->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(h->stream);       // the image is reused by the next page
        if (e != hipSuccess) {
            char b_[300];
            snprintf(b_, sizeof b_, "sp_hipkv_write_kv: page copy: %s", hipGetErrorString(e));
            sp_set_error(b_);
            rc = 1;
        }
    }
    hipHostFree(stage);
    if (rc) return rc;
    h->dpos = std::max(h->dpos, p0 + n);
    h->hwm = std::max(h->hwm, h->dpos);
    return 0;
}

int sp_hipkv_v_clamps(const sp_kvdecode_handle *h, long long *count) {
    if (!h || !count) return fail("sp_hipkv_v_clamps: null argument%s");
    int c = 0;
    HIPCHK(hipStreamSynchronize(h->stream), "clamp counter sync");
    HIPCHK(hipMemcpy(&c, h->vclamp, sizeof c, hipMemcpyDeviceToHost), "clamp counter read");
    *count = c;
    return 0;
}

int sp_hipkv_check_model(const void *qm_opaque, long long out[8]) {
    if (!qm_opaque || !out) return fail("sp_hipkv_check_model: null argument%s");
    std::lock_guard<std::mutex> lk(g_mu);
    DevModel *m = model_get((const qwen3_model *)qm_opaque, false);
    if (!m) return 1;
    out[0] = (long long)m->weight_bytes; out[1] = (long long)m->lm_bytes; out[2] = m->NL;
    out[3] = m->E; out[4] = m->V; out[5] = m->FF; out[6] = m->SW;
    int wide = m->embd.wide | m->out.wide;
    for (const DevLayer &d : m->L)
        for (const DevW *w : {&d.q, &d.k, &d.v, &d.o, &d.gate, &d.up, &d.down}) wide |= w->wide;
    out[7] = wide;
    delete m;
    return 0;
}

int sp_hipkv_info(const sp_kvdecode_handle *h, long long out[8]) {
    if (!h || !out) return fail("sp_hipkv_info: bad argument%s");
    out[0] = (long long)h->m->weight_bytes; out[1] = (long long)h->m->lm_bytes;
    out[2] = (long long)(2 * h->m->NKV * kv_row_bytes(h->m, h->mode, h->kvc)); out[3] = h->mode; out[4] = h->dpos;
    out[5] = (long long)h->pool->ptr.size(); out[6] = (long long)h->pool->page_bytes; out[7] = h->pmax;
    return 0;
}

}  // extern "C"

