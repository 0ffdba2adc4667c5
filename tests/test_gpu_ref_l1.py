"""The drop-in under the reference's own L1: the session verbs of the compiled
reference (oracle/_ref/libspref.so, built from core/session/sp_session.c and its
dependencies) with sp_hipkv_dispatch registered through the reference's
sp_session_register_kvdecode_backend, driven by a registrant that follows the
include/sp/sp_l1.h:386-402 contract exactly:

  * sp_prefill_chunk runs the reference's host forward (positions advance on the
    host) and the registrant feeds the same tokens through dt->prefill;
  * every sp_decode_step of the reference routes to dt->decode_step
    (core/session/sp_session.c:737-746): HIP logits, compared with the oracle
    (exact mode bit for bit, float mode rel <= 1e-3 with the same argmax);
  * sp_session_rewind moves only the host position (:818-824), so the registrant
    also calls dt->rewind; decoding then continues in step with the oracle.

The model handle the backend opens is the reference bridge's qwen3_model
(sp_session_qwen3_model of the reference session).
"""
import ctypes

import numpy as np
import pytest

import orc
import spkv
from helpers import model_files

pytestmark = pytest.mark.gpu
c_void_p, c_int, c_size_t = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t


def ref_l1():
    R = orc.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref (the compiled reference) not built")
    for name, res, args in [
        ("sp_model_load", c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(c_void_p)]),
        ("sp_model_unload", None, [c_void_p]),
        ("sp_session_create", c_int, [c_void_p, ctypes.POINTER(spkv.SessionConfig), c_void_p, ctypes.POINTER(c_void_p)]),
        ("sp_session_destroy", None, [c_void_p]),
        ("sp_prefill_chunk", c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_size_t]),
        ("sp_decode_step", c_int, [c_void_p, ctypes.c_int32, c_void_p, c_size_t]),
        ("sp_session_rewind", c_int, [c_void_p, c_size_t]),
        ("sp_session_position", c_int, [c_void_p, ctypes.POINTER(c_size_t)]),
        ("sp_session_qwen3_model", c_void_p, [c_void_p]),
        ("sp_session_register_kvdecode_backend", c_int, [c_void_p, c_void_p, c_void_p]),
        ("sp_last_error", ctypes.c_char_p, []),
    ]:
        f = getattr(R, name); f.restype = res; f.argtypes = args
    return R


@pytest.mark.parametrize("name", ["qwen3-tiny", "gemma3-tiny"])
@pytest.mark.parametrize("exact", [True, False])
def test_dispatch_table_under_reference_l1(tmpdir_models, name, exact):
    R = ref_l1()
    K = spkv.kv()
    spm, spt = model_files(tmpdir_models, name)
    pmax = 128
    m = c_void_p()
    assert R.sp_model_load(spm.encode(), spt.encode(), ctypes.byref(m)) == 0, R.sp_last_error()
    cfg = spkv.SessionConfig(pmax, 1, 0, 0, 0, 0)
    s = c_void_p()
    assert R.sp_session_create(m, ctypes.byref(cfg), None, ctypes.byref(s)) == 0, R.sp_last_error()
    qm = R.sp_session_qwen3_model(s)
    h = c_void_p()
    spkv.check(K.sp_hipkv_open(c_void_p(qm), pmax, ctypes.byref(h)), "sp_hipkv_open (reference qwen3_model)")
    if exact:
        spkv.check(K.sp_hipkv_set_mode(h, 1), "sp_hipkv_set_mode")
    dt = spkv.DispatchTable.in_dll(K, "sp_hipkv_dispatch")
    assert R.sp_session_register_kvdecode_backend(s, h, ctypes.byref(dt)) == 0
    o = orc.Oracle(spm, pmax, orc.EXACT if exact else orc.FLOAT)
    V = o.V
    pr = spkv.splitmix_tokens(40, V, seed=1)
    lg = np.zeros(V, np.float32)
    # the registrant: the reference's host prefill, and the same tokens through dt->prefill
    assert R.sp_prefill_chunk(s, spkv.ptr(pr), len(pr), spkv.ptr(lg), V) == 0, R.sp_last_error()
    spkv.check(K.sp_hipkv_prefill(h, spkv.ptr(pr), len(pr)), "dt->prefill")
    for t in pr:
        ol = o.step(int(t))

    def decode(tok):
        assert R.sp_decode_step(s, int(tok), spkv.ptr(lg), V) == 0, R.sp_last_error()
        want = o.step(int(tok))
        if exact:
            assert np.array_equal(lg.view(np.uint32), want.view(np.uint32))
        else:
            assert np.abs(lg - want).max() / np.abs(want).max() < 1e-3 and int(lg.argmax()) == int(want.argmax())
        return int(want.argmax())

    t = int(ol.argmax())
    for _ in range(10):
        t = decode(t)
    # rewind: the reference moves only its host position, the registrant rewinds the backend
    assert R.sp_session_rewind(s, 3) == 0
    spkv.check(K.sp_hipkv_rewind(h, 3), "dt->rewind")
    assert o.rewind(3) == 0
    for tok in (5, 6, 7, 8):
        decode(tok)
    p = c_size_t()
    assert R.sp_session_position(s, ctypes.byref(p)) == 0 and p.value == K.sp_hipkv_position(h) == o.pos()
    assert R.sp_session_register_kvdecode_backend(s, None, None) == 0
    K.sp_hipkv_close(h)
    R.sp_session_destroy(s)
    R.sp_model_unload(m)
    o.close()
