"""sp_hipkv_decode_step_noalloc -- the decode step that allocates nothing (its
step scratch is the library's static device buffer) -- against
sp_hipkv_decode_step on a copy-on-write twin of the same handle, through the C
ABI.  Two calls in a row on different handles, the second on a smaller model
and context (the shared buffer keeps the first call's contents), in both
arithmetic modes; exact mode bit for bit, float mode too (the same kernels run
in the same order).  A handle whose step scratch exceeds the static buffer is
refused with a clear error and its position is unchanged."""
import numpy as np
import pytest

import spkv
from helpers import SMALL, model_files, prompt

pytestmark = pytest.mark.gpu


def noalloc(be, tok, lg):
    return spkv.kv().sp_hipkv_decode_step_noalloc(be.h, int(tok), spkv.ptr(lg))


@pytest.mark.parametrize("exact", [True, False])
def test_noalloc_step_matches_decode_step(tmpdir_models, exact):
    for name, n_prompt, pmax in (("gemma3-wide", 300, 512), ("qwen3-tiny", 12, 64)):
        spm, spt = model_files(tmpdir_models, name)
        m = spkv.Model(spm, spt); s = spkv.Session(m, pmax)
        qm = spkv.l1().sp_session_qwen3_model(s.h)
        a = spkv.Backend(qm, pmax, exact=exact)
        V = SMALL[name]["vocab"]
        pr = prompt(n_prompt, V, seed=9)
        a.prefill(pr[:-1])
        b = a.fork()
        la, lb = np.zeros(V, np.float32), np.zeros(V, np.float32)
        tok = int(pr[-1])
        for k in range(3):
            a.decode(tok, la)
            assert noalloc(b, tok, lb) == 0, spkv.last_error()
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), (name, k)
            assert a.position() == b.position() == n_prompt + k
            tok = int(la.argmax())
        a.close(); b.close(); s.close(); m.close()


def test_noalloc_refuses_oversized_scratch(tmpdir_models):
    """Float mode keeps per-chunk attention partials: at head_dim 256 and a
    context of 100000 positions they exceed the static buffer."""
    spm, spt = model_files(tmpdir_models, "gemma3-hd256")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 64)
    be = spkv.Backend(spkv.l1().sp_session_qwen3_model(s.h), 100000, exact=False)
    lg = np.zeros(2048, np.float32)
    assert noalloc(be, 1, lg) != 0
    assert "static buffer" in spkv.last_error()
    assert be.position() == 0
    be.decode(1, lg)                                    # the allocating entry point still works
    assert be.position() == 1
    be.close(); s.close(); m.close()
