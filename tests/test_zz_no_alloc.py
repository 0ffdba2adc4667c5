"""sp_hipkv_decode_step_noalloc -- the decode step that allocates nothing (its
step scratch is the library's static device buffer) -- against
sp_hipkv_decode_step on a copy-on-write twin of the same handle, through the C
ABI.  Two calls in a row on different handles, the second on a smaller model
and context (the shared buffer keeps the first call's contents), in both
arithmetic modes; exact mode bit for bit, float mode too (the same kernels run
in the same order).  A handle whose step scratch exceeds the static buffer is
refused with a clear error and its position is unchanged.  A step that needs
more KV pages than the pool has free is refused with nothing changed (the
page tables stay consistent, the fork parent's pages untouched), and calls
from two threads on two handles run one after another (a per-device lock)."""
import threading

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


def test_noalloc_refusal_changes_nothing(tmpdir_models):
    """A pool grown 9 pages at a time holds 7 layers' first pages and 2 free.
    A fork rewound into the shared page needs 7 copy-on-write pages: the
    allocation-free step must refuse before touching any table.  The allocating
    step then copies every layer's page, writes its own position there (the
    parent's K/V at that position stays the parent's), and its logits equal a
    fresh handle's that decoded the same tokens (exact mode, bit for bit)."""
    name, pmax = "gemma3-tiny", 128
    spm, spt = model_files(tmpdir_models, name)
    m = spkv.Model(spm, spt); s = spkv.Session(m, pmax)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    V, NL = SMALL[name]["vocab"], SMALL[name]["n_layers"]
    kvd = SMALL[name]["n_kv_heads"] * SMALL[name]["head_dim"]
    pr = prompt(40, V, seed=5)
    a = spkv.Backend(qm, pmax, exact=True)
    assert spkv.kv().sp_hipkv_set_pool_growth(a.h, 9) == 0
    a.prefill(pr)
    before = [a.read_kv(l, 0, 40, kvd) for l in range(NL)]
    b = a.fork()
    assert b.rewind(5) == 0
    tok = (int(pr[35]) + 1) % V                        # not the parent's token at position 35
    lg = np.zeros(V, np.float32)
    assert noalloc(b, tok, lg) != 0
    assert "free KV pages" in spkv.last_error() and "nothing changed" in spkv.last_error()
    assert b.position() == 35
    b.decode(tok, lg)                                  # grows the pool, copies all 7 pages
    for l in range(NL):
        k, v = a.read_kv(l, 0, 40, kvd)
        assert np.array_equal(k.view(np.uint32), before[l][0].view(np.uint32)), f"parent K, layer {l}"
        assert np.array_equal(v.view(np.uint32), before[l][1].view(np.uint32)), f"parent V, layer {l}"
    c = spkv.Backend(qm, pmax, exact=True)
    c.prefill(pr[:35])
    lc = np.zeros(V, np.float32)
    c.decode(tok, lc)
    assert np.array_equal(lg.view(np.uint32), lc.view(np.uint32))
    for l in range(NL):                                # the fork's own position 35
        kb, vb = b.read_kv(l, 35, 1, kvd); kc, vc = c.read_kv(l, 35, 1, kvd)
        assert np.array_equal(kb.view(np.uint32), kc.view(np.uint32)) and np.array_equal(vb.view(np.uint32), vc.view(np.uint32))
    # the parent goes on from its own position 40 as a fresh twin would
    la = np.zeros(V, np.float32); a.decode(7, la)
    d = spkv.Backend(qm, pmax, exact=True); d.prefill(pr)
    ld = np.zeros(V, np.float32); d.decode(7, ld)
    assert np.array_equal(la.view(np.uint32), ld.view(np.uint32))
    for x in (a, b, c, d):
        x.close()
    s.close(); m.close()


def test_noalloc_two_threads_two_handles(tmpdir_models):
    """Two handles (each on its own stream) step through the allocation-free
    entry point from two threads at once, 6 steps each; every step equals the
    allocating step of a copy-on-write twin fed the same tokens."""
    name, pmax = "gemma3-wide", 512
    spm, spt = model_files(tmpdir_models, name)
    m = spkv.Model(spm, spt); s = spkv.Session(m, pmax)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    V = SMALL[name]["vocab"]
    hs, twins, feeds = [], [], []
    for i, n in enumerate((200, 90)):
        h = spkv.Backend(qm, pmax, exact=True)
        pr = prompt(n, V, seed=20 + i)
        h.prefill(pr)
        hs.append(h); twins.append(h.fork())
        feeds.append(prompt(6, V, seed=30 + i))
    out = [[None] * 6, [None] * 6]
    errs = []

    def run(i):
        for k in range(6):
            lg = np.zeros(V, np.float32)
            if noalloc(hs[i], int(feeds[i][k]), lg) != 0:
                errs.append((i, k, spkv.last_error()))
                return
            out[i][k] = lg

    th = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errs, errs
    for i in range(2):
        for k in range(6):
            lg = np.zeros(V, np.float32)
            twins[i].decode(int(feeds[i][k]), lg)
            assert np.array_equal(out[i][k].view(np.uint32), lg.view(np.uint32)), (i, k)
    for x in hs + twins:
        x.close()
    s.close(); m.close()
