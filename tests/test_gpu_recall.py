"""ARM recall on the device (sp_hipkv_set_recall) against the oracle's recall
decode, through the C ABI.

The oracle's recall decode is pinned against the compiled reference (golden
perplexities of qwen3_ppl_decode and greedy sequences of qwen3_generate_kv with
SP_RECALL_B/W/SINK/R, with and without SP_RECALL_DECODE_ONLY=1).  The device
prefill attends densely and writes the sidecar; decode steps route.  The oracle
runs the prompt's prefilled part with dense recall steps (the effective budget
0 of decode-only), then routes.

Bars:
  exact mode -- logits of every routed step, every resident K/V element and
                every sidecar row BIT-EXACT to the oracle's exact mode;
  float mode -- logits within rel 1e-3, same greedy token.
Identity budget (B >= context): recall on gives the plain path's logits bit for
bit (the reference's T_ARM_GENKV identity gate, core/session/arm_genkv_gate.c).
Cases: head_dim 64/128/256, GQA groups 2 and 4, Gemma's global layer among
window layers, no sinks, a budget below sinks + window (no top-k), budgets
whose candidate scan spans several 1024-position passes, forks (copy-on-write
pages carry the sidecar), rewinds, the device greedy loop and the
allocation-free step.
"""
import numpy as np
import pytest

import orc
import spkv
from helpers import model_files, prompt

pytestmark = pytest.mark.gpu
FLOAT_TOL = 1e-3


def rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def same_bits(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def global_layers(o):
    return [l for l in range(o.NL) if o.arch != spkv.ARCH_GEMMA3 or l % 6 == 5]


class Pair:
    """A device handle and an oracle session with the same recall settings:
    n_pre prompt tokens prefilled (dense), then routed decode steps."""

    def __init__(self, spm, spt, exact, pmax, rec, batch_prefill=True, graph=True):
        self.m = spkv.Model(spm, spt)
        self.s = spkv.Session(self.m, pmax)
        qm = spkv.l1().sp_session_qwen3_model(self.s.h)
        self.be = spkv.Backend(qm, pmax, exact=exact, graph=graph, batch_prefill=batch_prefill)
        self.o = orc.Oracle(spm, pmax, orc.EXACT if exact else orc.FLOAT)
        self.exact = exact
        if rec:
            self.be.set_recall(*rec)
            self.o.set_recall(*rec)
        self.V = self.o.V
        self.lg = np.zeros(self.V, np.float32)

    def prefill(self, toks):
        print(f"[recall] prefill {len(toks)} tokens at {self.be.position()}", flush=True)
        self.be.prefill(toks)
        self.o.set_recall_dense(1)
        for t in toks:
            self.o.step(int(t), False)
        self.o.set_recall_dense(0)

    def step(self, t):
        self.be.decode(int(t), self.lg)
        ol = self.o.step(int(t))
        return self.lg.copy(), ol

    def close(self):
        for x in (self.be, self.o, self.s, self.m):
            x.close()


def check_step(g, c, exact, what):
    if exact:
        assert same_bits(g, c), f"{what}: max rel {rel(g, c):.3e}"
    else:
        assert rel(g, c) < FLOAT_TOL, f"{what}: rel {rel(g, c):.3e}"
        assert int(g.argmax()) == int(c.argmax()), f"{what}: argmax"


def check_resident(p, n):
    """K/V and the global layers' sidecar rows [0, n) against the oracle."""
    o = p.o
    for l in range(o.NL):
        k, v = p.be.read_kv(l, 0, n, o.NKV * o.HD)
        ok, ov = o.kv(l, 0, n)
        assert same_bits(k, ok) and same_bits(v, ov), f"layer {l}: K/V"
    r = o.rec_r
    for l in global_layers(o):
        assert same_bits(p.be.recall_sidecar(l, 0, n, o.NKV, r), o.recall_sidecar(l, 0, n)), f"layer {l}: sidecar"


CASES = [
    # model, (B, W, sink, r), prompt, decode steps
    ("qwen3-tiny", (48, 16, 4, 16), 150, 40),
    ("qwen3-hd128", (100, 8, 0, 64), 180, 40),
    ("qwen3-g4", (40, 12, 3, 8), 170, 40),
    ("qwen3-g4", (33, 40, 2, 16), 120, 24),         # B < W + sink: sinks + window only
    ("gemma3-tiny", (40, 16, 4, 16), 150, 40),       # the global layer among window layers
    ("gemma3-hd256", (64, 16, 4, 32), 180, 40),
]


@pytest.mark.parametrize("name,rec,n_pre,n_gen", CASES, ids=[f"{c[0]}-B{c[1][0]}" for c in CASES])
def test_recall_exact_bitexact(tmpdir_models, name, rec, n_pre, n_gen):
    spm, spt = model_files(tmpdir_models, name, 256)
    p = Pair(spm, spt, True, 256, rec)
    plain = orc.Oracle(spm, 256, orc.EXACT)             # the same steps without recall
    pr = prompt(n_pre + 1, p.V)
    p.prefill(pr[:-1])
    for t in pr[:-1]:
        plain.step(int(t), False)
    g, c = p.step(pr[-1])
    check_step(g, c, True, "first routed step")
    t = int(pr[-1])
    differs = not same_bits(c, plain.step(t))
    for k in range(n_gen):
        t = int(c.argmax())
        g, c = p.step(t)
        check_step(g, c, True, f"step {k}")
        differs |= not same_bits(c, plain.step(t))
    assert differs, "the router changed no logits: the case does not exercise recall"
    check_resident(p, p.be.position())
    plain.close()
    p.close()


KVSEL_CASES = [
    ("qwen3-tiny", (48, 16, 4, 16), 150, 30, True),
    ("qwen3-g4", (40, 12, 3, 8), 170, 30, True),        # GQA 4: one selection serves four q heads
    ("gemma3-hd256", (64, 16, 4, 32), 180, 30, True),
    ("qwen3-hd128", (100, 8, 0, 64), 180, 20, True),
    ("qwen3-g4", (40, 12, 3, 8), 170, 20, False),
]


@pytest.mark.parametrize("name,rec,n_pre,n_gen,exact", KVSEL_CASES,
                         ids=[f"{c[0]}-B{c[1][0]}-{'exact' if c[4] else 'float'}" for c in KVSEL_CASES])
def test_recall_kvsel(tmpdir_models, name, rec, n_pre, n_gen, exact):
    """SP_RECALL_KVSEL on the device (sp_hipkv_set_recall_kvsel) against the
    oracle's KVSEL decode, which reproduces the compiled reference's KVSEL
    perplexities and greedy sequences (committed goldens): exact mode bit for
    bit, float mode within 1e-3; a fork inherits the setting; the shared sets
    change the logits against per-q-head selection."""
    spm, spt = model_files(tmpdir_models, name, 256)
    p = Pair(spm, spt, exact, 256, rec)
    p.be.set_recall_kvsel(True)
    p.o.set_recall_kvsel(True)
    per_head = orc.Oracle(spm, 256, orc.EXACT if exact else orc.FLOAT)   # the same steps, per-q-head sets
    per_head.set_recall(*rec)
    pr = prompt(n_pre + 1, p.V, seed=3)
    p.prefill(pr[:-1])
    per_head.set_recall_dense(1)
    for t in pr[:-1]:
        per_head.step(int(t), False)
    per_head.set_recall_dense(0)
    g, c = p.step(pr[-1])
    check_step(g, c, exact, "first routed step")
    t = int(pr[-1])
    differs = not same_bits(c, per_head.step(t))
    for k in range(n_gen):
        t = int(c.argmax())
        if k == n_gen // 2:                                 # continue on a fork
            f = p.be.fork(); p.be.close(); p.be = f
        g, c = p.step(t)
        check_step(g, c, exact, f"step {k}")
        differs |= not same_bits(c, per_head.step(t))
    assert differs, "KVSEL changed no logits: the case does not exercise the shared selection"
    if exact:
        check_resident(p, p.be.position())
    per_head.close()
    p.close()


RING2_CASES = [
    ("qwen3-tiny", (48, 16, 4, 16), True),
    ("gemma3-tiny", (40, 16, 4, 16), True),             # the global layer among window layers
    ("qwen3-g4", (40, 70, 0, 8), True),                 # no sinks, a window over two pages
    ("qwen3-hd128", (64, 16, 4, 16), False),
]


@pytest.mark.parametrize("name,rec,exact", RING2_CASES,
                         ids=[f"{c[0]}-B{c[1][0]}-{'exact' if c[2] else 'float'}" for c in RING2_CASES])
def test_recall_ring2_is_bit_identical(tmpdir_models, name, rec, exact):
    """Ring-2 (sp_hipkv_set_ring2): the full-context layers' pages outside the
    sinks and the recall window move to host memory before each decode step.
    Against a twin without Ring-2 fed the same tokens: every step's logits bit
    for bit (both modes: the same bytes reach the same kernels), every resident
    K/V row read back identical, pages actually spilled, a rewind into spilled
    pages (they come back to HBM when written), a fork and the device greedy
    loop."""
    pmax, n_pre = 1024, 600
    spm, spt = model_files(tmpdir_models, name, pmax)
    m = spkv.Model(spm, spt); s = spkv.Session(m, pmax)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    o = orc.Oracle(spm, 64, orc.EXACT)
    V, NL, kvd = o.V, o.NL, o.NKV * o.HD
    glob = global_layers(o)
    o.close()
    a = spkv.Backend(qm, pmax, exact=exact); a.set_recall(*rec)
    b = spkv.Backend(qm, pmax, exact=exact); b.set_recall(*rec); b.set_ring2(True)
    pr = prompt(n_pre, V, seed=11)
    a.prefill(pr); b.prefill(pr)
    la, lb = np.zeros(V, np.float32), np.zeros(V, np.float32)

    def both(tok, what):
        a.decode(int(tok), la); b.decode(int(tok), lb)
        assert same_bits(la, lb), what
        return int(la.argmax())

    t = int(pr[-1])
    for k in range(24):
        t = both(t, f"step {k}")
    host, dev, spills, _ = b.ring2_stats()
    W, sink = rec[1], rec[2]
    lo = b.position() - W
    expect = len(glob) * max(0, lo // 64 - (sink + 63) // 64)
    assert spills >= expect > 0 and host >= expect, (host, dev, spills, expect)
    for l in range(NL):
        ka, va = a.read_kv(l, 0, a.position(), kvd); kb, vb = b.read_kv(l, 0, b.position(), kvd)
        assert same_bits(ka, kb) and same_bits(va, vb), f"layer {l}: K/V read back"
    # rewind into spilled pages: the next writes bring them back
    assert a.rewind(300) == 0 and b.rewind(300) == 0
    for k in range(12):
        t = both(t, f"after the rewind, step {k}")
    assert b.ring2_stats()[3] > 0, "no page came back from host memory"
    # a fork reads the shared (host) history and writes its own pages
    fa, fb = a.fork(), b.fork()
    for k in range(6):
        fa.decode(t, la); fb.decode(t, lb)
        assert same_bits(la, lb), f"fork step {k}"
        t = int(la.argmax())
    # the device greedy loop
    ga, _ = a.greedy(t, 20)
    gb, _ = b.greedy(t, 20)
    assert list(ga) == list(gb)
    for x in (fa, fb, a, b):
        x.close()
    s.close(); m.close()


def test_recall_float_within_tolerance(tmpdir_models):
    spm, spt = model_files(tmpdir_models, "qwen3-hd128", 256)
    p = Pair(spm, spt, False, 256, (64, 16, 4, 16))
    pr = prompt(161, p.V)
    p.prefill(pr[:-1])
    g, c = p.step(pr[-1])
    check_step(g, c, False, "first routed step")
    for k in range(40):
        g, c = p.step(int(c.argmax()))
        check_step(g, c, False, f"step {k}")
    p.close()


@pytest.mark.parametrize("exact", [True, False])
def test_identity_budget_is_the_plain_path(tmpdir_models, exact):
    """B >= every position: the recall lists are 0..pos and the logits are the
    plain attention's (bit for bit in exact mode, float within the list-sum
    rounding)."""
    spm, spt = model_files(tmpdir_models, "qwen3-g4", 256)
    a = Pair(spm, spt, exact, 256, (256, 8, 2, 16))
    b = Pair(spm, spt, exact, 256, None)
    pr = prompt(121, a.V)
    a.prefill(pr[:-1]); b.prefill(pr[:-1])
    t = int(pr[-1])
    for k in range(24):
        ga, _ = a.step(t)
        gb, c = b.step(t)
        check_step(ga, gb, exact, f"step {k}")
        t = int(c.argmax())
    a.close(); b.close()


def test_recall_long_candidate_scan(tmpdir_models):
    """3000 resident positions: the router scores and selects over several
    1024-position passes and the attention over 8 list chunks."""
    spm, spt = model_files(tmpdir_models, "qwen3-hd128", 4096)
    p = Pair(spm, spt, True, 4096, (512, 64, 4, 16))
    pr = prompt(3001, p.V)
    p.prefill(pr[:-1])
    g, c = p.step(pr[-1])
    check_step(g, c, True, "first routed step")
    for k in range(12):
        g, c = p.step(int(c.argmax()))
        check_step(g, c, True, f"step {k}")
    p.close()


def test_recall_batch_prefill_off(tmpdir_models):
    """Prefill one step per token (dense, graph-captured) leaves the same
    sidecar and K/V as the batched prefill."""
    spm, spt = model_files(tmpdir_models, "qwen3-tiny", 256)
    p = Pair(spm, spt, True, 256, (48, 16, 4, 16), batch_prefill=False)
    pr = prompt(101, p.V)
    p.prefill(pr[:-1])
    g, c = p.step(pr[-1])
    check_step(g, c, True, "first routed step")
    for k in range(16):
        g, c = p.step(int(c.argmax()))
        check_step(g, c, True, f"step {k}")
    check_resident(p, p.be.position())
    p.close()


@pytest.mark.parametrize("graph", [True, False])
def test_recall_fork_and_rewind(tmpdir_models, graph):
    spm, spt = model_files(tmpdir_models, "qwen3-g4", 256)
    p = Pair(spm, spt, True, 256, (40, 12, 3, 16), graph=graph)
    pr = prompt(140, p.V)
    p.prefill(pr[:-1])
    g, c = p.step(pr[-1])
    check_step(g, c, True, "first routed step")
    child = p.be.fork()
    oc = p.o.clone()
    lg = np.zeros(p.V, np.float32)
    t_child = (int(c.argmax()) + 7) % p.V
    t = int(c.argmax())
    for k in range(12):
        child.decode(t_child, lg)
        cl = oc.step(t_child)
        check_step(lg, cl, True, f"child step {k}")
        t_child = int(cl.argmax())
        g, c = p.step(t)
        check_step(g, c, True, f"parent step {k}")
        t = int(c.argmax())
    assert p.be.rewind(5) == 0
    p.o.rewind(5)
    for k in range(10):
        g, c = p.step(t)
        check_step(g, c, True, f"after rewind, step {k}")
        t = int(c.argmax())
    check_resident(p, p.be.position())
    child.close(); oc.close()
    p.close()


def test_recall_device_greedy_and_noalloc(tmpdir_models):
    spm, spt = model_files(tmpdir_models, "qwen3-hd128", 256)
    p = Pair(spm, spt, True, 256, (64, 16, 4, 16))
    pr = prompt(150, p.V)
    p.prefill(pr[:-1])
    toks, _ = p.be.greedy(int(pr[-1]), 20)
    want = []
    t = int(pr[-1])
    for _ in range(20):
        t = int(p.o.step(t).argmax())
        want.append(t)
    assert [int(x) for x in toks] == want
    # the allocation-free step routes the same way
    lg = np.zeros(p.V, np.float32)
    spkv.check(spkv.kv().sp_hipkv_decode_step_noalloc(p.be.h, int(toks[-1]), spkv.ptr(lg)), "noalloc step")
    check_step(lg, p.o.step(int(toks[-1])), True, "noalloc step")
    p.close()


def test_recall_argument_checks(tmpdir_models):
    spm, spt = model_files(tmpdir_models, "qwen3-tiny", 256)
    m = spkv.Model(spm, spt)
    s = spkv.Session(m, 256)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    be = spkv.Backend(qm, 256, exact=True)
    k = spkv.kv()
    assert k.sp_hipkv_set_recall(be.h, 16, 4, 2, 0) != 0           # r out of range
    assert k.sp_hipkv_set_recall(be.h, 16, 4, 2, 65) != 0
    assert k.sp_hipkv_set_recall(be.h, -1, 4, 2, 16) != 0
    be.set_recall(16, 4, 2, 16)
    be.prefill(prompt(8, 1000))
    assert k.sp_hipkv_set_recall(be.h, 32, 4, 2, 16) != 0          # tokens resident
    assert k.sp_hipkv_read_recall_sidecar(be.h, 0, 0, 9, spkv.ptr(np.zeros(9 * 2 * 16, np.float32))) != 0
    be.close()
    fb = spkv.Backend(qm, 256, exact=False, kv_codec=spkv.KV_SPINOR)
    assert k.sp_hipkv_set_recall(fb.h, 16, 4, 2, 16) != 0          # float Spinor code rows
    fb.close()
    s.close(); m.close()
