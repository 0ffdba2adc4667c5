"""spkv -- Python host mirror of the C ABI (include/sp_l1_abi.h, sp_model_abi.h,
sp_hipkv.h) through ctypes.

The product is the two in-tree shared libraries:
  lib/libsp_l1.so     .sp-model loader / bridge / session verbs / OK_Q4B producer (C11)
  lib/libsp_hipkv.so  the section-6b kvdecode backend on MI355X (HIP, gfx950)
This module only declares their signatures and wraps handles; it computes
nothing itself.  Loading libsp_hipkv.so fails loudly when it has not been built.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# SPKV_LIB_DIR: another build of the two libraries (the sanitizer build, lib-asan)
LIB_DIR = os.environ.get("SPKV_LIB_DIR") or os.path.join(HERE, "lib")

SP_OK, SP_EBADARG, SP_EBADSTATE, SP_EUNSUPPORTED = 0, -3, -4, -5
SP_ECANCEL, SP_ECONTEXT_FULL, SP_EBACKEND_OOM = -2, -33, -43
ARCH_QWEN3, ARCH_GEMMA3 = 2, 3

c_void_p, c_int, c_int32, c_size_t, c_float, c_double = (
    ctypes.c_void_p, ctypes.c_int, ctypes.c_int32, ctypes.c_size_t, ctypes.c_float, ctypes.c_double)
c_char_p, c_uint32, c_uint64, c_longlong = ctypes.c_char_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_longlong


class SynthSpec(ctypes.Structure):
    """sp_synth_spec (include/sp_model_abi.h)."""
    _fields_ = [("arch_id", c_uint32), ("n_layers", c_uint32), ("hidden", c_uint32),
                ("n_heads", c_uint32), ("n_kv_heads", c_uint32), ("head_dim", c_uint32),
                ("n_ff", c_uint32), ("vocab", c_uint32), ("max_context", c_uint32),
                ("swa_window", c_uint32), ("rope_base", c_float), ("rms_eps", c_float),
                ("untied", c_int), ("seed", c_uint64), ("spread_rows", c_uint32), ("spread_mask", c_uint32)]


class SessionConfig(ctypes.Structure):
    """sp_session_config (include/sp/sp_l1.h:160-169)."""
    _fields_ = [("max_context", c_size_t), ("deterministic", c_int), ("arm_bank_kb", c_uint32),
                ("sieve_capacity", c_uint32), ("flags", c_uint32), ("precision_override", c_uint32)]


class DispatchTable(ctypes.Structure):
    """sp_kvdecode_dispatch_fn (include/sp/sp_l1.h:403-410)."""
    _fields_ = [("open", c_void_p), ("prefill", c_void_p), ("decode_step", c_void_p),
                ("rewind", c_void_p), ("position", c_void_p), ("close", c_void_p)]


_l1 = None
_kv = None


def _sig(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args
    return f


def l1():
    """libsp_l1.so: host C library (no GPU needed)."""
    global _l1
    if _l1 is None:
        path = os.path.join(LIB_DIR, "libsp_l1.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: run __graft_entry__.build()")
        lib = ctypes.CDLL(path)
        _sig(lib, "sp_last_error", c_char_p, [])
        _sig(lib, "sp_crc32", c_uint32, [c_void_p, c_size_t])
        _sig(lib, "sp_sha256", None, [c_void_p, c_size_t, c_void_p])
        _sig(lib, "sp_xxh64", c_uint64, [c_void_p, c_size_t, c_uint64])
        _sig(lib, "sp_f16_to_f32", c_float, [ctypes.c_uint16])
        _sig(lib, "sp_f32_to_f16", ctypes.c_uint16, [c_float])
        _sig(lib, "sp_q4b_quantize_row", None, [c_void_p, c_int, c_void_p, c_void_p])
        _sig(lib, "sp_write_synthetic_q4b", c_int, [ctypes.POINTER(SynthSpec), c_char_p, c_char_p, c_int])
        _sig(lib, "sp_model_load", c_int, [c_char_p, c_char_p, ctypes.POINTER(c_void_p)])
        _sig(lib, "sp_model_unload", None, [c_void_p])
        _sig(lib, "sp_model_find_tensor", c_void_p, [c_void_p, c_char_p])
        _sig(lib, "sp_model_tensor_count", c_uint32, [c_void_p])
        _sig(lib, "sp_model_arch", c_int, [c_void_p, c_void_p])
        _sig(lib, "sp_session_create", c_int, [c_void_p, ctypes.POINTER(SessionConfig), c_void_p, ctypes.POINTER(c_void_p)])
        _sig(lib, "sp_session_destroy", None, [c_void_p])
        _sig(lib, "sp_prefill_chunk", c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_size_t])
        _sig(lib, "sp_decode_step", c_int, [c_void_p, c_int32, c_void_p, c_size_t])
        _sig(lib, "sp_session_clone", c_int, [c_void_p, c_void_p, ctypes.POINTER(c_void_p)])
        _sig(lib, "sp_session_rewind", c_int, [c_void_p, c_size_t])
        _sig(lib, "sp_session_position", c_int, [c_void_p, ctypes.POINTER(c_size_t)])
        _sig(lib, "sp_session_qwen3_model", c_void_p, [c_void_p])
        _sig(lib, "sp_session_register_kvdecode_backend", c_int, [c_void_p, c_void_p, c_void_p])
        _sig(lib, "sp_session_kvdecode_backend_handle", c_void_p, [c_void_p])
        _sig(lib, "sp_session_kvdecode_backend_dt", c_void_p, [c_void_p])
        _sig(lib, "spx_session_own_kvdecode", c_int, [c_void_p, c_int])
        _sig(lib, "spx_session_route_kv_lifecycle", c_int, [c_void_p, c_int])
        _sig(lib, "spx_decode_batch", c_int, [c_void_p, c_size_t, c_void_p, c_void_p, c_size_t, c_void_p])
        _l1 = lib
    return _l1


def kv():
    """libsp_hipkv.so: the HIP backend.  Raises if not built (no fallback)."""
    global _kv
    if _kv is None:
        l1()
        path = os.path.join(LIB_DIR, "libsp_hipkv.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: the HIP kvdecode backend is required")
        lib = ctypes.CDLL(path)
        _sig(lib, "sp_hipkv_open", c_int, [c_void_p, c_int, ctypes.POINTER(c_void_p)])
        _sig(lib, "sp_hipkv_prefill", c_int, [c_void_p, c_void_p, c_int])
        _sig(lib, "sp_hipkv_decode_step", c_int, [c_void_p, c_int32, c_void_p])
        _sig(lib, "sp_hipkv_decode_step_noalloc", c_int, [c_void_p, c_int32, c_void_p])
        _sig(lib, "sp_hipkv_rewind", c_int, [c_void_p, c_int])
        _sig(lib, "sp_hipkv_position", c_int, [c_void_p])
        _sig(lib, "sp_hipkv_close", None, [c_void_p])
        _sig(lib, "sp_hipkv_set_mode", c_int, [c_void_p, c_int])
        _sig(lib, "sp_hipkv_set_kv_codec", c_int, [c_void_p, c_int])
        _sig(lib, "sp_hipkv_set_max_rewind", c_int, [c_void_p, c_int])
        _sig(lib, "sp_hipkv_set_graph", c_int, [c_void_p, c_int])
        _sig(lib, "sp_hipkv_set_window_one_launch", c_int, [c_void_p, c_int])
        _sig(lib, "sp_hipkv_set_pool_growth", c_int, [c_void_p, c_int])
        _sig(lib, "sp_hipkv_set_recall_kvsel", c_int, [c_void_p, c_int])
        _sig(lib, "sp_hipkv_set_ring2", c_int, [c_void_p, c_int])
        _sig(lib, "sp_hipkv_ring2_stats", c_int, [c_void_p, c_void_p])
        _sig(lib, "sp_hipkv_write_kv", c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p])
        _sig(lib, "sp_hipkv_set_batch_prefill", c_int, [c_void_p, c_int])
        _sig(lib, "sp_hipkv_fork", c_int, [c_void_p, ctypes.POINTER(c_void_p)])
        _sig(lib, "sp_hipkv_attach", c_int, [c_void_p, c_int, c_int])
        _sig(lib, "sp_hipkv_greedy", c_int, [c_void_p, c_int32, c_int, c_void_p, ctypes.POINTER(c_double)])
        _sig(lib, "sp_hipkv_decode_batch", c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p])
        _sig(lib, "sp_hipkv_kernel_times", c_int, [c_void_p, c_int32, c_int, c_void_p, c_void_p, c_void_p])
        _sig(lib, "sp_hipkv_decode_batch_times", c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p])
        _sig(lib, "sp_hipkv_read_kv", c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p])
        _sig(lib, "sp_hipkv_info", c_int, [c_void_p, c_void_p])
        _sig(lib, "sp_hipkv_check_model", c_int, [c_void_p, c_void_p])
        _sig(lib, "sp_hipkv_v_clamps", c_int, [c_void_p, ctypes.POINTER(c_longlong)])
        _sig(lib, "sp_hipkv_set_recall", c_int, [c_void_p, c_int, c_int, c_int, c_int])
        _sig(lib, "sp_hipkv_read_recall_sidecar", c_int, [c_void_p, c_int, c_int, c_int, c_void_p])
        _kv = lib
    return _kv


def last_error():
    e = l1().sp_last_error()
    return e.decode(errors="replace") if e else ""


def ptr(a):
    """numpy array -> void* (ctypes would otherwise truncate the address to int)."""
    return c_void_p(a.ctypes.data)


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")


# ---------------------------------------------------------------- synthetic inputs
def splitmix_u64(n, seed):
    """The first n outputs of SplitMix64 seeded with `seed` (the generator of
    the synthetic prompts, context lengths and rewind draws)."""
    import numpy as np
    k = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + k * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def splitmix_tokens(n, vocab, seed=1):
    """n prompt tokens uniform in [0, vocab): SplitMix64 output mod vocab."""
    import numpy as np
    return (splitmix_u64(n, seed) % np.uint64(vocab)).astype(np.int32)


# ---------------------------------------------------------------- shapes
SHAPES = {
    # hidden, layers, heads, kv_heads, head_dim, ffn, vocab, arch, rope_base, swa
    "qwen3-0.6b-1layer": dict(arch_id=ARCH_QWEN3, n_layers=1, hidden=1024, n_heads=16, n_kv_heads=8,
                              head_dim=128, n_ff=3072, vocab=151936, rope_base=1e6, swa_window=0),
    "qwen3-0.6b": dict(arch_id=ARCH_QWEN3, n_layers=28, hidden=1024, n_heads=16, n_kv_heads=8,
                       head_dim=128, n_ff=3072, vocab=151936, rope_base=1e6, swa_window=0),
    "gemma3-12b": dict(arch_id=ARCH_GEMMA3, n_layers=48, hidden=3840, n_heads=16, n_kv_heads=8,
                       head_dim=256, n_ff=15360, vocab=262144, rope_base=1e6, swa_window=1024),
    "qwen3-8b": dict(arch_id=ARCH_QWEN3, n_layers=36, hidden=4096, n_heads=32, n_kv_heads=8,
                     head_dim=128, n_ff=12288, vocab=151936, rope_base=1e6, swa_window=0, untied=1),
}


def write_model(path_prefix, shape=None, seed=0, max_context=4096, threads=0, **kw):
    """Write <prefix>.spm/.spt with the seeded OK_Q4B generator (sp_write_synthetic_q4b)."""
    d = dict(SHAPES[shape]) if shape else {}
    d.update(kw)
    spec = SynthSpec(d["arch_id"], d["n_layers"], d["hidden"], d["n_heads"], d["n_kv_heads"],
                     d["head_dim"], d["n_ff"], d["vocab"], max_context, d.get("swa_window", 0),
                     d.get("rope_base", 1e6), d.get("rms_eps", 1e-6), d.get("untied", 0), seed,
                     d.get("spread_rows", 0), d.get("spread_mask", 0))
    spm, spt = path_prefix + ".spm", path_prefix + ".spt"
    check(l1().sp_write_synthetic_q4b(ctypes.byref(spec), spm.encode(), spt.encode(), threads),
          "sp_write_synthetic_q4b")
    return spm, spt


class Model:
    def __init__(self, spm, spt):
        h = c_void_p()
        check(l1().sp_model_load(spm.encode(), spt.encode(), ctypes.byref(h)), "sp_model_load")
        self.h = h

    def close(self):
        if self.h:
            l1().sp_model_unload(self.h)
            self.h = None


class Session:
    """sp_session over a Model; attach() registers the HIP backend (owned)."""

    def __init__(self, model, max_context=0, cancel=None, flags=0):
        cfg = SessionConfig(max_context, 1, 0, 0, flags, 0)
        h = c_void_p()
        self.cancel = cancel
        check(l1().sp_session_create(model.h, ctypes.byref(cfg),
                                     ctypes.addressof(cancel) if cancel is not None else None,
                                     ctypes.byref(h)), "sp_session_create")
        self.h = h

    def attach(self, pmax, exact=False):
        check(kv().sp_hipkv_attach(self.h, pmax, 1 if exact else 0), "sp_hipkv_attach")

    def prefill(self, toks, logits):
        import numpy as np
        t = np.ascontiguousarray(toks, dtype=np.int32)
        return l1().sp_prefill_chunk(self.h, ptr(t), len(t), ptr(logits), logits.size)

    def decode(self, tok, logits):
        return l1().sp_decode_step(self.h, int(tok), ptr(logits), logits.size)

    def position(self):
        p = c_size_t()
        check(l1().sp_session_position(self.h, ctypes.byref(p)), "sp_session_position")
        return p.value

    def rewind(self, n):
        return l1().sp_session_rewind(self.h, n)

    def clone(self):
        c = Session.__new__(Session)
        h = c_void_p()
        rc = l1().sp_session_clone(self.h, None, ctypes.byref(h))
        check(rc, "sp_session_clone")
        c.h = h
        c.cancel = None
        return c

    def backend_handle(self):
        return l1().sp_session_kvdecode_backend_handle(self.h)

    @staticmethod
    def decode_batch(sessions, tokens, vocab, want_logits=True):
        """spx_decode_batch: one token per session in one call; returns
        (status, logits [n][vocab] or None, greedy next tokens [n])."""
        import numpy as np
        n = len(sessions)
        ss = (c_void_p * n)(*[s.h.value if isinstance(s.h, c_void_p) else s.h for s in sessions])
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        lg = np.zeros((n, vocab), np.float32) if want_logits else None
        nxt = np.zeros(n, np.int32)
        rc = l1().spx_decode_batch(ss, n, ptr(toks), ptr(lg) if want_logits else None,
                                   lg.size if want_logits else 0, ptr(nxt))
        return rc, lg, nxt

    def close(self):
        if self.h:
            l1().sp_session_destroy(self.h)
            self.h = None


NCLASS = 9          # kernel classes of sp_hipkv_kernel_times (include/sp_hipkv.h)
KV_PLAIN, KV_SPINOR = 0, 1                    # sp_hipkv_set_kv_codec
SP_KV_SPINOR, SP_KV_SPINOR_REF = 1, 2         # sp_session_config.flags


class Backend:
    """A bare section-6b handle driven through the dispatch functions directly."""

    def __init__(self, qm, pmax, exact=False, graph=True, batch_prefill=True, kv_codec=KV_PLAIN):
        h = c_void_p()
        check(kv().sp_hipkv_open(qm, pmax, ctypes.byref(h)), "sp_hipkv_open")
        self.h = h
        if exact:
            check(kv().sp_hipkv_set_mode(h, 1), "sp_hipkv_set_mode")
        if kv_codec != KV_PLAIN:
            check(kv().sp_hipkv_set_kv_codec(h, kv_codec), "sp_hipkv_set_kv_codec")
        if not graph:
            check(kv().sp_hipkv_set_graph(h, 0), "sp_hipkv_set_graph")
        if not batch_prefill:
            check(kv().sp_hipkv_set_batch_prefill(h, 0), "sp_hipkv_set_batch_prefill")

    @classmethod
    def wrap(cls, h):
        b = cls.__new__(cls)
        b.h = c_void_p(h) if not isinstance(h, c_void_p) else h
        return b

    def prefill(self, toks):
        import numpy as np
        t = np.ascontiguousarray(toks, dtype=np.int32)
        check(kv().sp_hipkv_prefill(self.h, ptr(t), len(t)), "sp_hipkv_prefill")

    def decode(self, tok, logits):
        check(kv().sp_hipkv_decode_step(self.h, int(tok), ptr(logits)), "sp_hipkv_decode_step")

    def rewind(self, n):
        return kv().sp_hipkv_rewind(self.h, n)

    def position(self):
        return kv().sp_hipkv_position(self.h)

    def fork(self):
        c = c_void_p()
        check(kv().sp_hipkv_fork(self.h, ctypes.byref(c)), "sp_hipkv_fork")
        return Backend.wrap(c)

    @staticmethod
    def decode_batch(backends, tokens, vocab, want_logits=True):
        """One batched decode step over several handles of one model: returns
        (logits [n][vocab] or None, greedy next tokens [n])."""
        import numpy as np
        n = len(backends)
        hs = (c_void_p * n)(*[b.h.value if isinstance(b.h, c_void_p) else b.h for b in backends])
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        lg = np.zeros((n, vocab), np.float32) if want_logits else None
        nxt = np.zeros(n, np.int32)
        check(kv().sp_hipkv_decode_batch(hs, n, ptr(toks), ptr(lg) if want_logits else None, ptr(nxt)),
              "sp_hipkv_decode_batch")
        return lg, nxt

    @staticmethod
    def decode_batch_times(backends, tokens):
        """One timed batched step (sp_hipkv_decode_batch_times): returns
        (next tokens, ms[NCLASS], launches[NCLASS], bytes[NCLASS])."""
        import numpy as np
        n = len(backends)
        hs = (c_void_p * n)(*[b.h.value if isinstance(b.h, c_void_p) else b.h for b in backends])
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        nxt = np.zeros(n, np.int32)
        ms = np.zeros(NCLASS, np.float64)
        nl = np.zeros(NCLASS, np.int64)
        by = np.zeros(NCLASS, np.float64)
        check(kv().sp_hipkv_decode_batch_times(hs, n, ptr(toks), ptr(nxt), ptr(ms), ptr(nl), ptr(by)),
              "sp_hipkv_decode_batch_times")
        return nxt, ms, nl, by

    def greedy(self, first_tok, n):
        import numpy as np
        out = np.zeros(n, dtype=np.int32)
        ms = c_double()
        check(kv().sp_hipkv_greedy(self.h, int(first_tok), n, ptr(out), ctypes.byref(ms)), "sp_hipkv_greedy")
        return out, ms.value

    def kernel_times(self, first_tok, n):
        import numpy as np
        ms = np.zeros(NCLASS, np.float64)
        nl = np.zeros(NCLASS, np.int64)
        by = np.zeros(NCLASS, np.float64)
        check(kv().sp_hipkv_kernel_times(self.h, int(first_tok), n, ptr(ms), ptr(nl), ptr(by)),
              "sp_hipkv_kernel_times")
        return ms, nl, by

    def read_kv(self, layer, p0, n, kvd):
        import numpy as np
        k = np.zeros((n, kvd), np.float32)
        v = np.zeros((n, kvd), np.float32)
        check(kv().sp_hipkv_read_kv(self.h, layer, p0, n, ptr(k), ptr(v)), "sp_hipkv_read_kv")
        return k, v

    def write_kv(self, layer, p0, k, v):
        import numpy as np
        k = np.ascontiguousarray(k, dtype=np.float32); v = np.ascontiguousarray(v, dtype=np.float32)
        assert k.shape == v.shape and k.ndim == 2
        check(kv().sp_hipkv_write_kv(self.h, layer, p0, k.shape[0], ptr(k), ptr(v)), "sp_hipkv_write_kv")

    def set_recall(self, B, W=64, sink=4, r=16):
        """ARM recall on the global layers (decode steps route, prefill is dense)."""
        check(kv().sp_hipkv_set_recall(self.h, B, W, sink, r), "sp_hipkv_set_recall")

    def set_window_one_launch(self, on):
        """Exact window layers in one launch (default) or the two-kernel path."""
        check(kv().sp_hipkv_set_window_one_launch(self.h, 1 if on else 0), "sp_hipkv_set_window_one_launch")

    def set_recall_kvsel(self, on):
        """SP_RECALL_KVSEL: one recall set per kv head (group-centroid query)."""
        check(kv().sp_hipkv_set_recall_kvsel(self.h, 1 if on else 0), "sp_hipkv_set_recall_kvsel")

    def set_ring2(self, on):
        """Ring-2: spill full-context pages outside sinks + recall window to host memory."""
        check(kv().sp_hipkv_set_ring2(self.h, 1 if on else 0), "sp_hipkv_set_ring2")

    def ring2_stats(self):
        """(host entries, device entries, pool spills, pool fetch-backs)"""
        import numpy as np
        o = np.zeros(4, np.int64)
        check(kv().sp_hipkv_ring2_stats(self.h, ptr(o)), "sp_hipkv_ring2_stats")
        return [int(x) for x in o]

    def recall_sidecar(self, layer, p0, n, nkv, r):
        import numpy as np
        out = np.zeros((n, nkv, r), np.float32)
        check(kv().sp_hipkv_read_recall_sidecar(self.h, layer, p0, n, ptr(out)), "sp_hipkv_read_recall_sidecar")
        return out

    def v_clamps(self):
        n = c_longlong()
        check(kv().sp_hipkv_v_clamps(self.h, ctypes.byref(n)), "sp_hipkv_v_clamps")
        return n.value

    def info(self):
        import numpy as np
        o = np.zeros(8, np.int64)
        check(kv().sp_hipkv_info(self.h, ptr(o)), "sp_hipkv_info")
        return o

    def close(self):
        if self.h:
            kv().sp_hipkv_close(self.h)
            self.h = None
