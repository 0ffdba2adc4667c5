"""The section-6b dispatch contract under the reference's own L1, on the CPU.

The compiled reference's session verbs (oracle/_ref/libspref.so, built in the
build container from core/session/sp_session.c and its dependencies; absent on
a fresh checkout, then skipped) and this library's L1 (lib/libsp_l1.so, default
routing) drive the same counting mock table (include/sp/sp_l1.h:386-402, the
table pattern of core/session/arm_genkv_gate.c:200-233) through the same
script.  Their transcripts -- every return code, position, table call and
logits row -- must be identical:

  * sp_decode_step routes to dt->decode_step and nothing else
    (core/session/sp_session.c:737-746), the logits are the table's row;
  * a failing dt->decode_step -> SP_EBADSTATE with the position unchanged (:740-743);
  * guards before dispatch: logits capacity < vocab -> SP_EBADARG, context full
    -> SP_ECONTEXT_FULL, cancel -> SP_ECANCEL, none reaching the table (:726-729);
  * sp_session_rewind moves only the host position (:818-824), rewind > position
    -> SP_EBADARG;
  * sp_session_clone drops the registration (:792-799);
  * handle / table readback, a NULL table unregisters, a NULL session -> SP_EBADARG
    (:909-925).

The reference's sp_prefill_chunk runs its host forward without touching the
table; this library's returns SP_EUNSUPPORTED there (no host forward in the
product), so prefill is checked on the reference side only: the mock sees no
call, and the next sp_decode_step routes to the table at the advanced position.
"""
import ctypes

import numpy as np
import pytest

import orc
import spkv
from helpers import model_files

c_void_p, c_int, c_size_t = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t

OPEN = ctypes.CFUNCTYPE(c_int, c_void_p, c_int, ctypes.POINTER(c_void_p))
PREFILL = ctypes.CFUNCTYPE(c_int, c_void_p, ctypes.POINTER(ctypes.c_int32), c_int)
STEP = ctypes.CFUNCTYPE(c_int, c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_float))
REWIND = ctypes.CFUNCTYPE(c_int, c_void_p, c_int)
POSN = ctypes.CFUNCTYPE(c_int, c_void_p)
CLOSE = ctypes.CFUNCTYPE(None, c_void_p)

VOCAB = 1000          # qwen3-tiny


class CountingTable:
    """A dispatch table whose decode_step writes a one-hot row at
    (tok + 3 * calls) % V and can be told to fail; it records every call."""

    def __init__(self):
        self.calls, self.fail_next, self.n = [], False, 0
        self._fns = [OPEN(self.open), PREFILL(self.prefill), STEP(self.step), REWIND(self.rewind),
                     POSN(self.position), CLOSE(self.close)]
        self.table = spkv.DispatchTable(*[ctypes.cast(f, c_void_p) for f in self._fns])

    def open(self, qm, p, out):
        self.calls.append(("open",)); return 0

    def prefill(self, h, toks, n):
        self.calls.append(("prefill", n)); return 0

    def step(self, h, tok, logits):
        self.calls.append(("step", h, tok))
        if self.fail_next:
            self.fail_next = False
            return 1
        hot = (tok + 3 * self.n) % VOCAB
        for i in range(VOCAB):
            logits[i] = 1.0 if i == hot else -float(i % 7)
        self.n += 1
        return 0

    def rewind(self, h, n):
        self.calls.append(("rewind", n)); return 0

    def position(self, h):
        self.calls.append(("position",)); return 0

    def close(self, h):
        self.calls.append(("close",))


class L1:
    """The session verbs of one L1 implementation (same frozen signatures)."""

    def __init__(self, lib, name):
        self.lib, self.name = lib, name
        for fn, res, args in [
            ("sp_model_load", c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(c_void_p)]),
            ("sp_model_unload", None, [c_void_p]),
            ("sp_session_create", c_int, [c_void_p, ctypes.POINTER(spkv.SessionConfig), c_void_p,
                                          ctypes.POINTER(c_void_p)]),
            ("sp_session_destroy", None, [c_void_p]),
            ("sp_session_clone", c_int, [c_void_p, c_void_p, ctypes.POINTER(c_void_p)]),
            ("sp_prefill_chunk", c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_size_t]),
            ("sp_decode_step", c_int, [c_void_p, ctypes.c_int32, c_void_p, c_size_t]),
            ("sp_session_rewind", c_int, [c_void_p, c_size_t]),
            ("sp_session_position", c_int, [c_void_p, ctypes.POINTER(c_size_t)]),
            ("sp_session_register_kvdecode_backend", c_int, [c_void_p, c_void_p, c_void_p]),
            ("sp_session_kvdecode_backend_handle", c_void_p, [c_void_p]),
            ("sp_session_kvdecode_backend_dt", c_void_p, [c_void_p]),
        ]:
            f = getattr(lib, fn); f.restype = res; f.argtypes = args

    def pos(self, s):
        p = c_size_t(12345)
        rc = self.lib.sp_session_position(s, ctypes.byref(p))
        return rc, p.value


def ref_l1():
    R = orc.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref (the compiled reference) is not built")
    return L1(R, "reference")


def transcript(l1, spm, spt):
    """Run the script on one L1; returns the list of observations."""
    lib = l1.lib
    out = []
    m = c_void_p()
    assert lib.sp_model_load(spm.encode(), spt.encode(), ctypes.byref(m)) == 0
    cancel = ctypes.c_int(0)
    cfg = spkv.SessionConfig(8, 1, 0, 0, 0, 0)          # max_context 8
    s = c_void_p()
    assert lib.sp_session_create(m, ctypes.byref(cfg), ctypes.byref(cancel), ctypes.byref(s)) == 0
    tab = CountingTable()
    lg = np.full(VOCAB, 7.0, np.float32)

    def obs(tag, rc):
        out.append((tag, rc, l1.pos(s), list(tab.calls), lg.tobytes()))
        tab.calls.clear()

    obs("register-null-session", lib.sp_session_register_kvdecode_backend(None, c_void_p(0x77),
                                                                          ctypes.byref(tab.table)))
    obs("register", lib.sp_session_register_kvdecode_backend(s, c_void_p(0x1234), ctypes.byref(tab.table)))
    out.append(("readback", lib.sp_session_kvdecode_backend_handle(s),
                lib.sp_session_kvdecode_backend_dt(s) == ctypes.addressof(tab.table)))
    for t in (5, 6, 7):
        obs(f"step {t}", lib.sp_decode_step(s, t, spkv.ptr(lg), VOCAB))
    obs("small-capacity", lib.sp_decode_step(s, 1, spkv.ptr(lg), VOCAB - 1))
    obs("null-logits", lib.sp_decode_step(s, 1, None, VOCAB))
    tab.fail_next = True
    obs("backend-fails", lib.sp_decode_step(s, 9, spkv.ptr(lg), VOCAB))
    obs("after-failure", lib.sp_decode_step(s, 9, spkv.ptr(lg), VOCAB))
    cancel.value = 1
    obs("cancelled", lib.sp_decode_step(s, 2, spkv.ptr(lg), VOCAB))
    cancel.value = 0
    obs("rewind-too-far", lib.sp_session_rewind(s, 99))
    obs("rewind 2", lib.sp_session_rewind(s, 2))
    obs("step after rewind", lib.sp_decode_step(s, 11, spkv.ptr(lg), VOCAB))
    for t in range(20):                                   # run into the context limit
        rc = lib.sp_decode_step(s, t, spkv.ptr(lg), VOCAB)
        obs(f"fill {t}", rc)
        if rc != 0:
            break
    c = c_void_p()
    obs("clone", lib.sp_session_clone(s, None, ctypes.byref(c)))
    out.append(("clone-registration", lib.sp_session_kvdecode_backend_handle(c),
                lib.sp_session_kvdecode_backend_dt(c)))
    out.append(("clone-position", l1.pos(c)))
    lib.sp_session_destroy(c)
    obs("unregister", lib.sp_session_register_kvdecode_backend(s, c_void_p(0x1234), None))
    out.append(("after-unregister", lib.sp_session_kvdecode_backend_handle(s),
                lib.sp_session_kvdecode_backend_dt(s)))
    lib.sp_session_destroy(s)
    lib.sp_model_unload(m)
    assert tab.calls == [], "the L1 must never call the table's other entries"
    return out


def test_dispatch_contract_identical_under_both_l1s(tmpdir_models):
    R = ref_l1()
    spm, spt = model_files(tmpdir_models, "qwen3-tiny", max_context=32)
    ref = transcript(R, spm, spt)
    ours = transcript(L1(spkv.l1(), "this library"), spm, spt)
    assert len(ref) == len(ours)
    for a, b in zip(ref, ours):
        assert a == b, f"reference {a[:4]} != this library {b[:4]}"
    # the script exercised what it claims: routed steps, the failure, the limit
    tags = {o[0]: o for o in ref}
    assert tags["step 5"][1] == spkv.SP_OK and tags["step 5"][3] == [("step", 0x1234, 5)]
    assert tags["backend-fails"][1] == spkv.SP_EBADSTATE
    assert tags["backend-fails"][2] == tags["small-capacity"][2]          # position unchanged
    assert tags["small-capacity"][3] == [] and tags["cancelled"][3] == []
    assert tags["cancelled"][1] == spkv.SP_ECANCEL
    assert any(o[1] == spkv.SP_ECONTEXT_FULL for o in ref if o[0].startswith("fill"))
    assert tags["clone-registration"][1:] == (None, None)


def test_reference_prefill_leaves_the_table_alone(tmpdir_models):
    """The reference's sp_prefill_chunk forwards on the host and never calls the
    table (the registrant feeds dt->prefill itself, sp_l1.h:396-399); the next
    sp_decode_step routes to dt->decode_step at the advanced position."""
    R = ref_l1()
    lib = R.lib
    spm, spt = model_files(tmpdir_models, "qwen3-tiny", max_context=32)
    m = c_void_p()
    assert lib.sp_model_load(spm.encode(), spt.encode(), ctypes.byref(m)) == 0
    cfg = spkv.SessionConfig(32, 1, 0, 0, 0, 0)
    s = c_void_p()
    assert lib.sp_session_create(m, ctypes.byref(cfg), None, ctypes.byref(s)) == 0
    tab = CountingTable()
    assert lib.sp_session_register_kvdecode_backend(s, c_void_p(0x55), ctypes.byref(tab.table)) == 0
    lg = np.zeros(VOCAB, np.float32)
    toks = np.array([3, 1, 4, 1, 5], np.int32)
    assert lib.sp_prefill_chunk(s, spkv.ptr(toks), len(toks), spkv.ptr(lg), VOCAB) == spkv.SP_OK
    assert tab.calls == [] and R.pos(s) == (spkv.SP_OK, 5)
    assert lib.sp_decode_step(s, 9, spkv.ptr(lg), VOCAB) == spkv.SP_OK
    assert tab.calls == [("step", 0x55, 9)] and R.pos(s) == (spkv.SP_OK, 6)
    assert int(lg.argmax()) == 9
    lib.sp_session_destroy(s)
    lib.sp_model_unload(m)
