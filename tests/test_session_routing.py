"""Section-6b routing and the session verbs' control semantics, on the CPU with a
counting mock dispatch table (the pattern of core/session/arm_genkv_gate.c:200-233).

Pins the reference's guards and commit points (core/session/sp_session.c
:154-212, :725-770, :773-824, :909-925): argument errors, context full, cancel
before any mutation, backend failure -> SP_EBADSTATE with the position unchanged,
rewind > position -> SP_EBADARG.  Default routing is the reference's contract
(include/sp/sp_l1.h:396-399: only sp_decode_step reaches the table); with
lifecycle routing switched on (spx_session_route_kv_lifecycle, what
sp_hipkv_attach does) prefill = dt->prefill(n-1) + dt->decode_step(last),
rewind -> dt->rewind, and clone without a registered fork drops the
registration as the reference does."""
import ctypes
import os
import re

import numpy as np
import pytest

import spkv
from helpers import model_files

OPEN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p))
PREFILL = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32), ctypes.c_int)
STEP = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_float))
REWIND = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int)
POSN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)
CLOSE = ctypes.CFUNCTYPE(None, ctypes.c_void_p)


class Mock:
    def __init__(self, vocab, fail_step=False):
        self.calls = []
        self.dpos = 0
        self.vocab = vocab
        self.fail_step = fail_step
        self.closed = 0
        self._fns = [OPEN(lambda qm, p, out: 0), PREFILL(self.prefill), STEP(self.step),
                     REWIND(self.rewind), POSN(lambda h: self.dpos), CLOSE(self.close)]
        self.table = spkv.DispatchTable(*[ctypes.cast(f, ctypes.c_void_p) for f in self._fns])

    def prefill(self, h, toks, n):
        self.calls.append(("prefill", [toks[i] for i in range(n)]))
        self.dpos += n
        return 0

    def step(self, h, tok, logits):
        self.calls.append(("step", tok))
        if self.fail_step:
            return 1
        for i in range(self.vocab):
            logits[i] = float(i == (tok + self.dpos) % self.vocab)
        self.dpos += 1
        return 0

    def rewind(self, h, n):
        self.calls.append(("rewind", n))
        self.dpos -= n
        return 0

    def close(self, h):
        self.closed += 1


@pytest.fixture
def session(tmpdir_models):
    spm, spt = model_files(tmpdir_models, "qwen3-tiny", max_context=32)
    m = spkv.Model(spm, spt)
    flag = ctypes.c_int(0)
    s = spkv.Session(m, 0, cancel=flag)          # max_context 0 -> arch default (32)
    yield s, flag
    s.close(); m.close()


def register(s, mock, route=True):
    L = spkv.l1()
    assert L.sp_session_register_kvdecode_backend(s.h, ctypes.c_void_p(0x1234), ctypes.byref(mock.table)) == 0
    assert L.sp_session_kvdecode_backend_handle(s.h) == 0x1234
    if route:
        assert L.spx_session_route_kv_lifecycle(s.h, 1) == 0


def test_default_routing_is_the_reference_contract(session):
    """Registered without lifecycle routing: sp_decode_step is the only verb that
    reaches the table (sp_l1.h:396-399).  The registrant feeds dt->prefill
    itself (here: once, directly), sp_session_rewind moves only the host
    position, sp_prefill_chunk does not call the table (this library has no host
    prefill), and the table sees every token exactly once."""
    s, _ = session
    mock = Mock(1000); register(s, mock, route=False)
    lg = np.zeros(1000, np.float32)
    toks = (ctypes.c_int32 * 3)(5, 6, 7)
    assert mock._fns[1](None, toks, 3) == 0                             # the registrant's own dt->prefill
    assert s.prefill([5, 6, 7], lg) == spkv.SP_EUNSUPPORTED
    assert "no host prefill" in spkv.last_error()
    assert s.decode(8, lg) == 0 and s.decode(9, lg) == 0
    assert mock.calls == [("prefill", [5, 6, 7]), ("step", 8), ("step", 9)]
    assert s.rewind(1) == 0 and s.position() == 1
    assert mock.calls[-1] == ("step", 9) and mock.dpos == 5              # no dt->rewind from the session
    c = s.clone()
    assert spkv.l1().sp_session_kvdecode_backend_dt(c.h) is None        # reference :792-799
    c.close()


def test_lifecycle_routing_switch(session):
    s, _ = session
    L = spkv.l1()
    assert L.spx_session_route_kv_lifecycle(s.h, 1) == spkv.SP_EBADSTATE   # nothing registered
    assert L.spx_session_route_kv_lifecycle(None, 1) == spkv.SP_EBADARG
    mock = Mock(1000); register(s, mock)
    lg = np.zeros(1000, np.float32)
    assert s.prefill([1, 2], lg) == 0 and mock.calls == [("prefill", [1]), ("step", 2)]
    # a new registration (another handle) starts on the default routing again
    assert L.sp_session_register_kvdecode_backend(s.h, ctypes.c_void_p(0x99), ctypes.byref(mock.table)) == 0
    assert s.prefill([3], lg) == spkv.SP_EUNSUPPORTED
    assert L.spx_session_route_kv_lifecycle(s.h, 0) == 0


def test_unregistered_session_has_no_host_decode(session):
    s, _ = session
    lg = np.zeros(1000, np.float32)
    assert s.decode(1, lg) == spkv.SP_EUNSUPPORTED
    assert "no kvdecode backend" in spkv.last_error()
    assert s.prefill([1, 2], lg) == spkv.SP_EUNSUPPORTED
    assert s.position() == 0


def test_decode_routes_and_advances(session):
    s, _ = session
    mock = Mock(1000); register(s, mock)
    lg = np.zeros(1000, np.float32)
    assert s.prefill([5, 6, 7], lg) == 0
    assert mock.calls == [("prefill", [5, 6]), ("step", 7)]
    assert lg.argmax() == (7 + 2) % 1000 and s.position() == 3
    assert s.decode(9, lg) == 0 and s.position() == 4 and mock.calls[-1] == ("step", 9)


def test_guards(session):
    s, flag = session
    mock = Mock(1000); register(s, mock)
    lg = np.zeros(1000, np.float32)
    small = np.zeros(999, np.float32)
    assert s.decode(1, small) == spkv.SP_EBADARG                         # capacity < vocab
    assert spkv.l1().sp_decode_step(s.h, 1, None, 1000) == spkv.SP_EBADARG
    assert s.prefill([], lg) == spkv.SP_EBADARG                          # n_tokens == 0
    assert s.prefill(list(range(33)), lg) == spkv.SP_ECONTEXT_FULL      # > hist_cap
    flag.value = 1
    assert s.decode(1, lg) == spkv.SP_ECANCEL and s.prefill([1], lg) == spkv.SP_ECANCEL
    assert mock.calls == [] and s.position() == 0                        # no mutation on cancel
    flag.value = 0
    for t in range(32):
        assert s.decode(t, lg) == 0
    assert s.decode(0, lg) == spkv.SP_ECONTEXT_FULL and s.position() == 32


def test_backend_failure_keeps_position(session):
    s, _ = session
    mock = Mock(1000, fail_step=True); register(s, mock)
    lg = np.zeros(1000, np.float32)
    assert s.decode(3, lg) == spkv.SP_EBADSTATE
    assert s.position() == 0 and "backend step failed" in spkv.last_error()
    assert s.prefill([1, 2, 3], lg) == spkv.SP_EBADSTATE
    assert s.position() == 0
    assert mock.calls[-1] == ("rewind", 2) and mock.dpos == 0          # backend brought back in step


def test_rewind_routes(session):
    s, _ = session
    mock = Mock(1000); register(s, mock)
    lg = np.zeros(1000, np.float32)
    for t in range(9):
        s.decode(t, lg)
    assert s.rewind(2) == 0 and s.position() == 7 and mock.calls[-1] == ("rewind", 2) and mock.dpos == 7
    assert s.rewind(9999) == spkv.SP_EBADARG and s.position() == 7
    assert s.rewind(0) == 0 and s.position() == 7


def test_clone_without_fork_drops_registration(session):
    s, _ = session
    mock = Mock(1000); register(s, mock)
    lg = np.zeros(1000, np.float32)
    for t in range(4):
        s.decode(t, lg)
    c = s.clone()
    assert c.position() == 4
    assert spkv.l1().sp_session_kvdecode_backend_dt(c.h) is None        # reference :792-799
    assert c.decode(1, lg) == spkv.SP_EUNSUPPORTED
    c.close()


def test_unregister_and_owned_close(session):
    s, _ = session
    mock = Mock(1000); register(s, mock)
    L = spkv.l1()
    assert L.spx_session_own_kvdecode(s.h, 1) == 0
    assert L.sp_session_register_kvdecode_backend(s.h, None, None) == 0      # NULL dt unregisters
    assert mock.closed == 1                                                  # owned handle closed
    assert L.sp_session_kvdecode_backend_dt(s.h) is None
    assert L.sp_session_register_kvdecode_backend(None, None, None) == spkv.SP_EBADARG


def test_hipkv_library_exports_every_declared_symbol():
    """libsp_hipkv.so loads on a host without a GPU and exports each symbol of
    include/sp_hipkv.h; libsp_l1.so exports the session/model ABI headers' symbols."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    lib = spkv.kv()
    hdr = open(os.path.join(root, "include", "sp_hipkv.h")).read()
    names = set(re.findall(r"\b(sp_hipkv_\w+)\s*\(", hdr)) | {"sp_hipkv_dispatch"}
    assert len(names) >= 14
    for n in sorted(names):
        assert hasattr(lib, n), n
    l1 = spkv.l1()
    for h in ("sp_l1_abi.h", "sp_model_abi.h"):
        txt = open(os.path.join(root, "include", h)).read()
        for n in set(re.findall(r"^\s*(?:[\w\s\*]+?)\b((?:sp|spx|qwen3)_\w+)\s*\(", txt, re.M)):
            assert hasattr(l1, n), n
    # the dispatch table points at the named entry points
    tab = spkv.DispatchTable.in_dll(lib, "sp_hipkv_dispatch")
    assert tab.open == ctypes.cast(lib.sp_hipkv_open, ctypes.c_void_p).value
    assert tab.close == ctypes.cast(lib.sp_hipkv_close, ctypes.c_void_p).value


def test_hipkv_open_without_gpu_fails_loudly(session):
    """No silent fallback: opening the HIP backend without a device is an error."""
    import subprocess, sys, json
    s, _ = session
    if os.environ.get("HIP_VISIBLE_DEVICES") is None:
        try:
            import torch
            if torch.cuda.is_available():
                pytest.skip("a GPU is visible")
        except Exception:
            pass
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    h = ctypes.c_void_p()
    rc = spkv.kv().sp_hipkv_open(qm, 16, ctypes.byref(h))
    assert rc != 0 and "no HIP device" in spkv.last_error()


class SharedMock:
    """One dispatch table serving several handles (per-handle positions), as a
    backend serving many sessions does; no batch hook is registered for it."""

    def __init__(self, vocab, fail_handle=None):
        self.calls, self.dpos, self.vocab, self.fail_handle = [], {}, vocab, fail_handle
        self._fns = [OPEN(lambda qm, p, out: 0), PREFILL(lambda h, t, n: 0), STEP(self.step),
                     REWIND(lambda h, n: 0), POSN(lambda h: self.dpos.get(h, 0)), CLOSE(lambda h: None)]
        self.table = spkv.DispatchTable(*[ctypes.cast(f, ctypes.c_void_p) for f in self._fns])

    def step(self, h, tok, logits):
        self.calls.append((h, tok))
        if h == self.fail_handle:
            return 1
        for i in range(self.vocab):
            logits[i] = float(i == (tok + 3) % self.vocab)
        self.dpos[h] = self.dpos.get(h, 0) + 1
        return 0


@pytest.fixture
def sessions(tmpdir_models):
    spm, spt = model_files(tmpdir_models, "qwen3-tiny", max_context=32)
    m = spkv.Model(spm, spt)
    flag = ctypes.c_int(0)
    ss = [spkv.Session(m, 0, cancel=flag) for _ in range(3)]
    yield ss, flag, m
    for s in ss:
        s.close()
    m.close()


def test_decode_batch_without_hook_steps_each_session(sessions):
    """spx_decode_batch on a table with no batch hook: one decode_step per
    session in order, logits rows and greedy tokens returned, every session
    advanced by one."""
    ss, _, _ = sessions
    mock = SharedMock(1000)
    for i, s in enumerate(ss):
        assert spkv.l1().sp_session_register_kvdecode_backend(s.h, ctypes.c_void_p(0x100 + i),
                                                              ctypes.byref(mock.table)) == 0
    rc, lg, nxt = spkv.Session.decode_batch(ss, [7, 8, 9], 1000)
    assert rc == 0
    assert mock.calls == [(0x100, 7), (0x101, 8), (0x102, 9)]
    assert nxt.tolist() == [10, 11, 12] and [int(r.argmax()) for r in lg] == [10, 11, 12]
    assert [s.position() for s in ss] == [1, 1, 1]
    rc, lg, nxt = spkv.Session.decode_batch(ss, [1, 2, 3], 1000, want_logits=False)
    assert rc == 0 and lg is None and nxt.tolist() == [4, 5, 6] and [s.position() for s in ss] == [2, 2, 2]


def test_decode_batch_guards(sessions, tmpdir_models):
    """Every guard is checked for every session before any decode: duplicates,
    mixed tables, no backend, short logits buffer, cancel, context full."""
    ss, flag, m = sessions
    L = spkv.l1()
    mock, other = SharedMock(1000), SharedMock(1000)
    assert spkv.Session.decode_batch(ss, [1, 2, 3], 1000)[0] == spkv.SP_EUNSUPPORTED
    for i, s in enumerate(ss):
        L.sp_session_register_kvdecode_backend(s.h, ctypes.c_void_p(0x100 + i), ctypes.byref(mock.table))
    assert spkv.Session.decode_batch([ss[0], ss[1], ss[0]], [1, 2, 3], 1000)[0] == spkv.SP_EBADARG
    assert "twice" in spkv.last_error()
    L.sp_session_register_kvdecode_backend(ss[2].h, ctypes.c_void_p(0x102), ctypes.byref(other.table))
    assert spkv.Session.decode_batch(ss, [1, 2, 3], 1000)[0] == spkv.SP_EBADARG
    L.sp_session_register_kvdecode_backend(ss[2].h, ctypes.c_void_p(0x102), ctypes.byref(mock.table))
    lg = np.zeros((3, 999), np.float32)
    n = (ctypes.c_void_p * 3)(*[s.h.value for s in ss])
    t = np.array([1, 2, 3], np.int32)
    assert L.spx_decode_batch(n, 3, spkv.ptr(t), spkv.ptr(lg), lg.size, None) == spkv.SP_EBADARG
    assert L.spx_decode_batch(None, 3, spkv.ptr(t), None, 0, None) == spkv.SP_EBADARG
    flag.value = 1
    assert spkv.Session.decode_batch(ss, [1, 2, 3], 1000)[0] == spkv.SP_ECANCEL
    flag.value = 0
    assert mock.calls == [] and [s.position() for s in ss] == [0, 0, 0]
    # context full on the last session: nothing decodes
    for _ in range(32):
        assert ss[2].decode(1, np.zeros(1000, np.float32)) == 0
    mock.calls.clear()
    assert spkv.Session.decode_batch(ss, [1, 2, 3], 1000)[0] == spkv.SP_ECONTEXT_FULL
    assert mock.calls == [] and [s.position() for s in ss] == [0, 0, 32]


def test_decode_batch_failure_commits_only_advanced_sessions(sessions):
    """A backend failure at the second session: SP_EBADSTATE, the first session
    (advanced by its backend) is committed, the others keep their position."""
    ss, _, _ = sessions
    mock = SharedMock(1000, fail_handle=0x101)
    for i, s in enumerate(ss):
        spkv.l1().sp_session_register_kvdecode_backend(s.h, ctypes.c_void_p(0x100 + i), ctypes.byref(mock.table))
    rc, _, _ = spkv.Session.decode_batch(ss, [4, 5, 6], 1000)
    assert rc == spkv.SP_EBADSTATE
    assert [s.position() for s in ss] == [1, 0, 0]
