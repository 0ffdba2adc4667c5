"""orc -- TEST INFRASTRUCTURE ONLY: ctypes view of oracle/lib/liboracle.so (the
CPU restatement of the reference decode) and of oracle/_ref/libspref.so (the
reference itself, compiled from its sources by oracle/ref.mk).  Imported only by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg."""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
c_void_p, c_int, c_float, c_double = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_double
FLOAT, EXACT = 0, 1
KV_SPINOR, KV_SPINOR_REF = 1, 2          # sp_session_config.flags bits (sp_l1.h:156-157)
_orc = None
_ref = None


def ptr(a):
    return c_void_p(a.ctypes.data)


def lib():
    global _orc
    if _orc is None:
        path = os.path.join(os.environ.get("ORC_LIB_DIR") or os.path.join(HERE, "lib"), "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} not built (make -C oracle)")
        L = ctypes.CDLL(path)
        for name, res, args in [
            ("orc_model_load", c_void_p, [ctypes.c_char_p]), ("orc_model_free", None, [c_void_p]),
            ("orc_model_dims", None, [c_void_p, c_void_p]),
            ("orc_sess_new", c_void_p, [c_void_p, c_int, c_int]), ("orc_sess_free", None, [c_void_p]),
            ("orc_step", c_int, [c_void_p, ctypes.c_int32, c_void_p]), ("orc_rewind", c_int, [c_void_p, c_int]),
            ("orc_pos", c_int, [c_void_p]), ("orc_clone", c_void_p, [c_void_p]), ("orc_set_pos", c_int, [c_void_p, c_int]),
            ("orc_kv_get", c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
            ("orc_kv_set", c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
            ("orc_f16_to_f32", c_float, [ctypes.c_uint16]),
            ("orc_rmsnorm", None, [c_void_p, c_void_p, c_int, c_float, c_void_p]),
            ("orc_rope_neox", None, [c_void_p, c_int, c_int, c_float]),
            ("orc_attn_head", None, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float, c_int, c_void_p, c_void_p]),
            ("orc_q4b_gemv", c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p]),
            ("orc_rmsnorm_exact", None, [c_void_p, c_void_p, c_int, c_void_p]),
            ("orc_softmax_exact", None, [c_void_p, c_int, c_void_p]),
            ("orc_gelu_exact", None, [c_void_p, c_int, c_void_p]),
            ("orc_silu_exact", None, [c_void_p, c_int, c_void_p]),
            ("orc_cordic_sincos", None, [ctypes.c_int64, c_void_p, c_void_p]),
            ("orc_rope_exact", None, [c_void_p, c_int, c_int, c_float]),
            ("orc_q4b_gemv_exact", c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p]),
            ("orc_rope_freq_q60", ctypes.c_int64, [c_float, c_int, c_int]),
            ("orc_sess_new_kv", c_void_p, [c_void_p, c_int, c_int, ctypes.c_uint32]),
            ("orc_set_kv_forced", None, [c_void_p, c_int]),
            ("orc_crc8", ctypes.c_uint8, [c_void_p, c_int]),
            ("orc_spinor_blocks_for", c_int, [c_int]),
            ("orc_spinor_encode", None, [c_void_p, c_int, c_void_p]),
            ("orc_spinor_decode", c_int, [c_void_p, c_void_p, c_int]),
            ("orc_spinor_encode_vec", None, [c_void_p, c_int, c_void_p]),
            ("orc_spinor_decode_vec", c_int, [c_void_p, c_int, c_void_p]),
            ("orc_attn_head_exact", None, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float, c_int, c_void_p]),
            ("orc_i128_div_to_float", c_float, [ctypes.c_int64, ctypes.c_uint64, ctypes.c_int64, c_int]),
            ("orc_vq_of", ctypes.c_int32, [c_float, c_void_p]),
            ("orc_v_clamps", c_int, [c_void_p]),
            ("orc_set_threads", None, [c_int]), ("orc_threads", c_int, []),
            ("orc_arm_build_R", None, [c_void_p, c_int, c_int]),
            ("orc_arm_project", None, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
            ("orc_arm_select", c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                       c_void_p, c_void_p]),
            ("orc_set_recall", c_int, [c_void_p, c_int, c_int, c_int, c_int]),
            ("orc_recall_sidecar", c_int, [c_void_p, c_int, c_int, c_int, c_void_p]),
            ("orc_set_recall_dense", None, [c_void_p, c_int]),
            ("orc_set_recall_kvsel", c_int, [c_void_p, c_int]),
            ("orc_recall_sidecar_set", c_int, [c_void_p, c_int, c_int, c_int, c_void_p]),
        ]:
            f = getattr(L, name); f.restype = res; f.argtypes = args
        _orc = L
    return _orc


def ref_lib():
    """The compiled reference, or None when oracle/_ref was not built."""
    global _ref
    if _ref is None:
        path = os.path.join(HERE, "_ref", "libspref.so")
        if not os.path.exists(path):
            return None
        L = ctypes.CDLL(path)
        L.refh_decode.restype = c_int
        L.refh_decode.argtypes = [ctypes.c_char_p, ctypes.c_char_p, c_void_p, c_int, c_int, c_void_p,
                                  c_void_p, c_void_p, c_void_p]
        L.refh_decode_flags.restype = c_int
        L.refh_decode_flags.argtypes = L.refh_decode.argtypes + [ctypes.c_uint32]
        for name in ("sp_spinor_encode_vec", "sp_spinor_decode_vec"):
            f = getattr(L, name)
            f.restype = None if name.endswith("encode_vec") else c_int
            f.argtypes = [c_void_p, c_int, c_void_p]
        L.sp_crc8.restype = ctypes.c_uint8
        L.sp_crc8.argtypes = [c_void_p, c_int]
        L.refh_qwen3_fixture_sha.restype = c_int
        L.refh_qwen3_fixture_sha.argtypes = [c_void_p, c_void_p]
        for name in ("sp_rmsnorm_exact", "sp_gelu_exact"):
            f = getattr(L, name); f.restype = None; f.argtypes = [c_void_p, c_void_p, c_int, c_void_p] if name == "sp_rmsnorm_exact" else [c_void_p, c_int, c_void_p]
        L.sp_softmax_exact.restype = None
        L.sp_softmax_exact.argtypes = [c_void_p, c_int, c_void_p]
        L.refh_ppl_recall.restype = c_int
        L.refh_ppl_recall.argtypes = [ctypes.c_char_p, ctypes.c_char_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                      c_int, ctypes.POINTER(c_double)]
        L.refh_generate_recall.restype = c_int
        L.refh_generate_recall.argtypes = [ctypes.c_char_p, ctypes.c_char_p, c_void_p, c_int, c_int, c_int, c_int,
                                           c_int, c_int, c_int]
        L.refh_set_kvsel.restype = None
        L.refh_set_kvsel.argtypes = [c_int]
        L.sp_arm_build_R.restype = None
        L.sp_arm_build_R.argtypes = [c_void_p, c_int, c_int]
        L.sp_arm_select.restype = c_int
        L.sp_arm_select.argtypes = [c_void_p, c_int, c_int, c_void_p, c_void_p, ctypes.c_size_t, c_int, c_int, c_int,
                                    c_int, c_int, c_int, c_int, c_void_p, c_void_p]
        _ref = L
    return _ref


class Oracle:
    """One oracle session over a .sp-model file."""

    def __init__(self, spm, max_ctx, mode=FLOAT, kv_flags=0):
        import numpy as np
        L = lib()
        self.m = L.orc_model_load(spm.encode())
        if not self.m:
            raise RuntimeError(f"oracle cannot load {spm}")
        d = np.zeros(9, np.uint32)
        L.orc_model_dims(self.m, ptr(d))
        self.arch, self.V, self.E, self.NL, self.NH, self.NKV, self.HD, self.FF, self.SW = [int(x) for x in d]
        self.s = L.orc_sess_new_kv(self.m, max_ctx, mode, kv_flags)
        if not self.s:
            raise RuntimeError("oracle session allocation failed")

    def step(self, tok, want_logits=True):
        import numpy as np
        lg = np.zeros(self.V, np.float32) if want_logits else None
        rc = lib().orc_step(self.s, int(tok), ptr(lg) if want_logits else None)
        if rc:
            raise RuntimeError("oracle step failed")
        return lg

    def rewind(self, n):
        return lib().orc_rewind(self.s, n)

    def pos(self):
        return lib().orc_pos(self.s)

    def clone(self):
        o = Oracle.__new__(Oracle)
        o.__dict__.update(self.__dict__)
        o.s = lib().orc_clone(self.s)
        o._owns_model = False
        return o

    def kv(self, layer, p0, n):
        import numpy as np
        kvd = self.NKV * self.HD
        k = np.zeros((n, kvd), np.float32); v = np.zeros((n, kvd), np.float32)
        lib().orc_kv_get(self.s, layer, p0, n, ptr(k), ptr(v))
        return k, v

    def set_kv(self, layer, p0, k, v):
        import numpy as np
        k = np.ascontiguousarray(k, np.float32); v = np.ascontiguousarray(v, np.float32)
        return lib().orc_kv_set(self.s, layer, p0, k.shape[0], ptr(k), ptr(v))

    def set_kv_forced(self, on):
        lib().orc_set_kv_forced(self.s, 1 if on else 0)

    def set_recall(self, B, W=64, sink=4, r=16):
        if lib().orc_set_recall(self.s, B, W, sink, r):
            raise RuntimeError("orc_set_recall failed")
        self.rec_r = r

    def set_recall_kvsel(self, on):
        """SP_RECALL_KVSEL: one recall set per kv head from the group-centroid query."""
        if lib().orc_set_recall_kvsel(self.s, 1 if on else 0):
            raise RuntimeError("orc_set_recall_kvsel failed")

    def set_recall_dense(self, on):
        lib().orc_set_recall_dense(self.s, 1 if on else 0)

    def recall_sidecar(self, layer, p0, n):
        import numpy as np
        out = np.zeros((n, self.NKV, self.rec_r), np.float32)
        if lib().orc_recall_sidecar(self.s, layer, p0, n, ptr(out)):
            raise RuntimeError("orc_recall_sidecar failed")
        return out

    def set_recall_sidecar(self, layer, p0, rows):
        import numpy as np
        rows = np.ascontiguousarray(rows, np.float32)
        if lib().orc_recall_sidecar_set(self.s, layer, p0, rows.shape[0], ptr(rows)):
            raise RuntimeError("orc_recall_sidecar_set failed")

    def v_clamps(self):
        return lib().orc_v_clamps(self.s)

    def set_pos(self, p):
        return lib().orc_set_pos(self.s, p)

    def close(self):
        if getattr(self, "s", None):
            lib().orc_sess_free(self.s); self.s = None
        if getattr(self, "m", None) and getattr(self, "_owns_model", True):
            lib().orc_model_free(self.m); self.m = None
