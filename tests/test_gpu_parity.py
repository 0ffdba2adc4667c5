"""GPU parity of the HIP section-6b backend against the oracle, through the C ABI.

Bars:
  exact mode  -- logits and every resident K/V element BIT-EXACT to the oracle's
                 exact mode (integer islands, CORDIC RoPE, integer GEMV/attention);
  float mode  -- logits within rel 1e-3 of the oracle's float mode (which is
                 bit-identical to the compiled reference), same greedy trajectory.
Cases cover both architectures, head_dim 64/128/256, GQA groups 2 and 4, an
untied head, GEMVs whose columns are split over workgroups (ragged last split), clipping sliding windows, prefill through sp_prefill_chunk, the
dispatch table driven directly, HIP-graph and plain launches, copy-on-write
forks through sp_session_clone, O(1) rewind (full table and window ring), and
the C1 configuration (Qwen3-0.6B single layer, vocab 151936).
"""
import ctypes

import numpy as np
import pytest

import orc
import spkv
from helpers import SMALL, model_files, prompt

pytestmark = pytest.mark.gpu
FLOAT_TOL = 1e-3


def rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def same_bits(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def run_pair(spm, spt, exact, n_prompt, n_gen, graph=True, pmax=256, via_session=True):
    m = spkv.Model(spm, spt)
    s = spkv.Session(m, pmax)
    o = orc.Oracle(spm, pmax, orc.EXACT if exact else orc.FLOAT)
    V = o.V
    pr = prompt(n_prompt, V)
    lg = np.zeros(V, np.float32)
    if via_session:
        s.attach(pmax, exact=exact)
        if not graph:
            spkv.check(spkv.kv().sp_hipkv_set_graph(s.backend_handle(), 0), "set_graph")
        spkv.check(s.prefill(pr, lg), "sp_prefill_chunk")
        step = lambda t: spkv.check(s.decode(t, lg), "sp_decode_step")
        be = spkv.Backend.wrap(s.backend_handle())
    else:
        be = spkv.Backend(spkv.l1().sp_session_qwen3_model(s.h), pmax, exact=exact, graph=graph)
        be.prefill(pr[:-1])
        be.decode(int(pr[-1]), lg)
        step = lambda t: be.decode(t, lg)
    for t in pr:
        ol = o.step(int(t))
    results = [(lg.copy(), ol)]
    t = int(ol.argmax())
    for k in range(n_gen):
        step(t)
        ol = o.step(t)
        results.append((lg.copy(), ol))
        t = int(ol.argmax())
    return m, s, o, be, results


def check(results, exact):
    for i, (g, c) in enumerate(results):
        if exact:
            assert same_bits(g, c), f"step {i}: max rel {rel(g, c):.3e}"
        else:
            assert rel(g, c) < FLOAT_TOL, f"step {i}: rel {rel(g, c):.3e}"
            assert int(g.argmax()) == int(c.argmax()), f"step {i}: argmax"


def close_all(*objs):
    for o in objs:
        o.close()


@pytest.mark.parametrize("name", ["qwen3-tiny", "gemma3-tiny", "qwen3-hd128", "gemma3-hd256", "qwen3-g4",
                                  "qwen3-wide", "gemma3-wide"])
@pytest.mark.parametrize("exact", [True, False])
def test_decode_parity(tmpdir_models, name, exact):
    spm, spt = model_files(tmpdir_models, name)
    wide = name.endswith("-wide")
    m, s, o, be, res = run_pair(spm, spt, exact, n_prompt=24 if wide else 40, n_gen=12 if wide else 24)
    check(res, exact)
    # resident K/V equals the oracle's slab (exact: bit for bit)
    kvd = o.NKV * o.HD
    pos = be.position()
    assert pos == o.pos()
    for layer in (0, o.NL - 1):
        kg, vg = be.read_kv(layer, 0, pos, kvd)
        kc, vc = o.kv(layer, 0, pos)
        if exact:
            assert same_bits(kg, kc) and same_bits(vg, vc), f"layer {layer}"
        else:
            assert rel(kg, kc) < 1e-4 and rel(vg, vc) < 1e-4
    close_all(s, o, m)


@pytest.mark.parametrize("name,exact", [("qwen3-spread", False),
                                        ("qwen3-spread-x", True), ("qwen3-spread-x", False),
                                        ("gemma3-spread-x", True), ("gemma3-spread-x", False)])
def test_decode_parity_int128_rows(tmpdir_models, name, exact):
    """Rows whose block scales span about 2^20 (their exact sums need more than
    64 bits): every GEMV of the model runs its int128 instance, prefill goes
    token by token.  Spread in every matrix (Qwen3, float mode: the
    activations outgrow exact mode's 64-bit sums of squares, as in the
    reference's islands, and through Gemma-3's seven layers the reference's
    float sums drift past 1e-3 of the exact ones); spread in the embedding/LM
    head, q, k, v and gate: both modes, both architectures."""
    spm, spt = model_files(tmpdir_models, name)
    m, s, o, be, res = run_pair(spm, spt, exact, n_prompt=24, n_gen=12)
    check(res, exact)
    close_all(s, o, m)


@pytest.mark.parametrize("exact", [True, False])
def test_plain_launches_and_direct_table(tmpdir_models, exact):
    spm, spt = model_files(tmpdir_models, "gemma3-tiny")
    m, s, o, be, res = run_pair(spm, spt, exact, n_prompt=30, n_gen=10, graph=False, via_session=False)
    check(res, exact)
    be.close(); close_all(s, o, m)


@pytest.mark.parametrize("exact", [True, False])
def test_batched_prefill_matches_stepwise(tmpdir_models, exact):
    """Prefill through the batched path (int8-MFMA GEMMs, token-batched attention,
    3 batches of up to 128 tokens, window and global layers, split GEMV columns)
    leaves the K/V that one decode step per token leaves, and the same logits
    for the next position (exact: bit for bit)."""
    spm, spt = model_files(tmpdir_models, "gemma3-wide")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 512)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    V = 3000
    pr = prompt(300, V, seed=7)
    lg1, lg2 = np.zeros(V, np.float32), np.zeros(V, np.float32)
    b1 = spkv.Backend(qm, 512, exact=exact)
    b2 = spkv.Backend(qm, 512, exact=exact, batch_prefill=False)
    b1.prefill(pr[:-1]); b1.decode(int(pr[-1]), lg1)
    b2.prefill(pr[:-1]); b2.decode(int(pr[-1]), lg2)
    if exact:
        assert same_bits(lg1, lg2)
    else:
        assert rel(lg1, lg2) < 1e-4 and int(lg1.argmax()) == int(lg2.argmax())
    kvd = 4 * 256
    for layer in range(6):
        k1, v1 = b1.read_kv(layer, 0, 300, kvd)
        k2, v2 = b2.read_kv(layer, 0, 300, kvd)
        if exact:
            assert same_bits(k1, k2) and same_bits(v1, v2), f"layer {layer}"
        else:
            assert rel(k1, k2) < 1e-4 and rel(v1, v2) < 1e-4, f"layer {layer}"
    b1.close(); b2.close(); close_all(s, m)


@pytest.mark.parametrize("anchor", [False, True])
def test_fresh_handles_prefill_identically(tmpdir_models, anchor):
    """Handles opened, forked and closed in a row leave bit-identical K/V and
    logits after the same prefill.  Without an anchor every close frees the
    device model, so each handle allocates and clears fresh buffers (reusing
    memory earlier handles freed): the clears are ordered before the handles'
    kernels.  With an anchor handle open, closed handles are kept as shells and
    the next open / fork takes one (tables, scratch, graphs reused, also across
    a float-mode user in between)."""
    spm, spt = model_files(tmpdir_models, "qwen3-hd128")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 512)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    pr = prompt(200, 2048, seed=21)
    keep = spkv.Backend(qm, 512, exact=True) if anchor else None
    ref = None
    lg = np.zeros(2048, np.float32)
    for it in range(12):
        if it % 4 == 3:                              # a float-mode user of the same shells
            fb = spkv.Backend(qm, 512, exact=False); fb.prefill(pr[:50]); fb.decode(1, lg); fb.close()
        b = spkv.Backend(qm, 512, exact=True)
        if it % 2:                                   # a fork brings its own buffers (or a shell)
            f = b.fork(); b.close(); b = f
        b.prefill(pr[:-1])
        b.decode(int(pr[-1]), lg)
        kv = [b.read_kv(layer, 0, 200, 4 * 128) for layer in range(2)] + [lg.copy()]
        b.close()
        if ref is None:
            ref = kv
            continue
        for layer in range(2):
            assert same_bits(kv[layer][0], ref[layer][0]) and same_bits(kv[layer][1], ref[layer][1]), \
                f"handle {it} layer {layer}"
        assert same_bits(kv[2], ref[2]), f"handle {it} logits"
    if keep:
        keep.close()
    close_all(s, m)


@pytest.mark.parametrize("exact", [True, False])
def test_session_decode_batch_with_clone_and_rewind(tmpdir_models, exact):
    """The batched configuration through the session layer: every step each
    session is cloned (sp_session_clone, the parent closed), the clone rewound
    0-4 tokens (sp_session_rewind) and all clones decoded by one
    spx_decode_batch; the same sequence with sp_decode_step on a second set of
    sessions gives the same logits (exact: bit for bit) and positions."""
    spm, spt = model_files(tmpdir_models, "qwen3-g4")
    m = spkv.Model(spm, spt)
    V = 2048
    lens = [20, 64, 65, 150, 7]
    A, B = [], []
    lg = np.zeros(V, np.float32)
    toks = []
    for i, n in enumerate(lens):
        pr = prompt(n, V, seed=30 + i)
        for group in (A, B):
            s = spkv.Session(m, 512)
            s.attach(512, exact=exact)
            assert s.prefill(pr, lg) == 0
            group.append(s)
        toks.append(int(lg.argmax()))
    rng = np.random.default_rng(5)
    for step in range(6):
        r = rng.integers(0, 5, size=len(lens))
        for group in (A, B):
            for i in range(len(lens)):
                c = group[i].clone(); group[i].close(); group[i] = c
                if r[i]:
                    assert c.rewind(int(r[i])) == 0
        rc, lga, nxt = spkv.Session.decode_batch(A, toks, V)
        assert rc == 0, spkv.last_error()
        for i in range(len(lens)):
            assert B[i].decode(toks[i], lg) == 0
            if exact:
                assert same_bits(lga[i], lg), f"step {step} session {i}"
            else:
                assert rel(lga[i], lg) < FLOAT_TOL, f"step {step} session {i}"
            assert int(nxt[i]) == int(lga[i].argmax())
            assert A[i].position() == B[i].position()
        toks = [int(t) for t in nxt]
    for x in A + B:
        x.close()
    m.close()


@pytest.mark.parametrize("name", ["qwen3-hd128", "gemma3-hd256"])
@pytest.mark.parametrize("exact", [True, False])
def test_decode_batch_matches_per_session(tmpdir_models, name, exact):
    """Batched multi-session decode (the 64-session configuration's pattern at a
    small scale): 6 sessions with ragged contexts; every step forks each session
    copy-on-write, rewinds the fork 0-4 tokens and decodes all forks in one
    sp_hipkv_decode_batch call.  The same sequence on independent handles with
    sp_hipkv_decode_step gives the same logits (exact mode: bit for bit)."""
    spm, spt = model_files(tmpdir_models, name)
    m = spkv.Model(spm, spt); s = spkv.Session(m, 512)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    V = 2048
    rng = np.random.default_rng(3)
    lens = [10, 33, 64, 65, 100, 130]
    A = [spkv.Backend(qm, 512, exact=exact) for _ in lens]
    B = [spkv.Backend(qm, 512, exact=exact) for _ in lens]
    toks = []
    lg = np.zeros(V, np.float32)
    for i, n in enumerate(lens):
        pr = prompt(n, V, seed=10 + i)
        A[i].prefill(pr[:-1]); B[i].prefill(pr[:-1])
        toks.append(int(pr[-1]))
    for step in range(5):
        r = rng.integers(0, 5, size=len(lens))
        A2, B2 = [], []
        for i in range(len(lens)):
            a, b = A[i].fork(), B[i].fork()
            A[i].close(); B[i].close()
            if step and r[i]:
                assert a.rewind(int(r[i])) == 0 and b.rewind(int(r[i])) == 0
            A2.append(a); B2.append(b)
        A, B = A2, B2
        lga, nxt = spkv.Backend.decode_batch(A, toks, V)
        for i in range(len(lens)):
            B[i].decode(toks[i], lg)
            if exact:
                assert same_bits(lga[i], lg), f"step {step} session {i}"
            else:
                assert rel(lga[i], lg) < FLOAT_TOL and int(lga[i].argmax()) == int(lg.argmax()), f"step {step} session {i}"
            assert int(nxt[i]) == int(lga[i].argmax())
            assert A[i].position() == B[i].position()
        toks = [int(t) for t in nxt]
    for x in A + B:
        x.close()
    close_all(s, m)


def oracle_from_device(spm, pmax, exact, be, pos, window):
    """An oracle session whose K/V of positions [0, pos) are the device's (window
    layers: only the positions the next step attends to), at position pos."""
    o = orc.Oracle(spm, pmax, orc.EXACT if exact else orc.FLOAT)
    kvd = o.NKV * o.HD
    for layer in range(o.NL):
        w = window(o, layer)
        a = max(0, pos - w) if w else 0
        if pos > a:
            k, v = be.read_kv(layer, a, pos - a, kvd)
            assert o.set_kv(layer, a, k, v) == 0
    assert o.set_pos(pos) == 0
    return o


@pytest.mark.parametrize("name", ["qwen3-hd128", "gemma3-hd256"])
@pytest.mark.parametrize("exact", [True, False])
def test_decode_batch_across_chunks(tmpdir_models, name, exact):
    """The batched decode's full-context layers split each session into
    512-position chunks, one (session, chunk) work item per workgroup and kv
    head, merged per session by its last arriving workgroup.  Ragged contexts
    around and across the chunk boundaries (100 .. 1700 positions: one to four
    chunks, a session ending on a boundary, one past it); three steps, each a
    copy-on-write fork of every session rewound 0-4 tokens.  Every row equals an
    independent handle's sp_hipkv_decode_step (exact mode bit for bit, float
    mode rel <= 1e-3, same argmax), and the longest and a one-chunk session
    equal the oracle given the device K/V."""
    pmax = 2048
    spm, spt = model_files(tmpdir_models, name, max_context=pmax)
    m = spkv.Model(spm, spt); s = spkv.Session(m, pmax)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    V = 2048
    lens = [100, 511, 512, 513, 600, 1100, 1536, 1700]
    rew = [[0] * len(lens), [4, 1, 0, 2, 3, 0, 1, 4], [1, 0, 4, 1, 0, 2, 3, 0]]
    A, B, toks = [], [], []
    for i, n in enumerate(lens):
        pr = prompt(n, V, seed=40 + i)
        a = spkv.Backend(qm, pmax, exact=exact)
        a.prefill(pr[:-1])
        A.append(a); B.append(a.fork())
        toks.append(int(pr[-1]))
    lg = np.zeros(V, np.float32)
    for step in range(3):
        A2, B2 = [], []
        for i in range(len(lens)):
            a, b = A[i].fork(), B[i].fork()
            A[i].close(); B[i].close()
            if rew[step][i]:
                assert a.rewind(rew[step][i]) == 0 and b.rewind(rew[step][i]) == 0
            A2.append(a); B2.append(b)
        A, B = A2, B2
        lga, nxt = spkv.Backend.decode_batch(A, toks, V)
        for i in range(len(lens)):
            B[i].decode(toks[i], lg)
            if exact:
                assert same_bits(lga[i], lg), f"step {step} session {i} (ctx {lens[i]})"
            else:
                assert rel(lga[i], lg) < FLOAT_TOL and int(lga[i].argmax()) == int(lg.argmax()), \
                    f"step {step} session {i}: rel {rel(lga[i], lg):.3e}"
            assert int(nxt[i]) == int(lga[i].argmax())
            assert A[i].position() == B[i].position()
        last = toks
        toks = [int(t) for t in nxt]
    window = lambda o, layer: o.SW if (o.arch == spkv.ARCH_GEMMA3 and layer % 6 != 5) else 0
    for i in (len(lens) - 1, 0):
        pos = A[i].position() - 1                      # the last batched step's position
        o = oracle_from_device(spm, pmax, exact, A[i], pos, window)
        ol = o.step(last[i])
        if exact:
            assert same_bits(lga[i], ol), f"session {i} vs the oracle"
        else:
            assert rel(lga[i], ol) < FLOAT_TOL and int(lga[i].argmax()) == int(ol.argmax())
        o.close()
    for x in A + B:
        x.close()
    close_all(s, m)


@pytest.mark.parametrize("name", ["qwen3-hd128", "gemma3-hd256"])
@pytest.mark.parametrize("exact", [True, False])
def test_write_kv_restores_a_session(tmpdir_models, name, exact):
    """sp_hipkv_write_kv, the inverse of read_kv: the K/V of a prefilled handle,
    written layer by layer into a fresh handle in uneven pieces, read back
    identical, the position follows, and the next decode step equals the
    original handle's bit for bit (same kernels, same K/V) and the oracle's
    given the same K/V (exact mode bit for bit, float mode within 1e-3).
    Writes past the resident position are refused."""
    pmax, n = 512, 300
    spm, spt = model_files(tmpdir_models, name)
    m = spkv.Model(spm, spt); s = spkv.Session(m, pmax)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    o = orc.Oracle(spm, pmax, orc.EXACT if exact else orc.FLOAT)
    kvd = o.NKV * o.HD
    pr = prompt(n + 1, o.V, seed=17)
    a = spkv.Backend(qm, pmax, exact=exact)
    a.prefill(pr[:n])
    b = spkv.Backend(qm, pmax, exact=exact)
    with pytest.raises(RuntimeError):
        b.write_kv(0, 1, *a.read_kv(0, 0, 1, kvd))          # p0 beyond the resident position
    kv_all = [a.read_kv(layer, 0, n, kvd) for layer in range(o.NL)]
    for lo, hi in ((0, 37), (37, 200), (200, n)):
        for layer in range(o.NL):
            k, v = kv_all[layer]
            b.write_kv(layer, lo, k[lo:hi], v[lo:hi])
    assert b.position() == n
    for layer in range(o.NL):
        kb, vb = b.read_kv(layer, 0, n, kvd)
        assert same_bits(kb, kv_all[layer][0]) and same_bits(vb, kv_all[layer][1]), f"layer {layer}"
        assert o.set_kv(layer, 0, kv_all[layer][0], kv_all[layer][1]) == 0
    assert o.set_pos(n) == 0
    la, lb = np.zeros(o.V, np.float32), np.zeros(o.V, np.float32)
    a.decode(int(pr[n]), la)
    b.decode(int(pr[n]), lb)
    ol = o.step(int(pr[n]))
    assert same_bits(la, lb)
    if exact:
        assert same_bits(lb, ol)
    else:
        assert rel(lb, ol) < FLOAT_TOL and int(lb.argmax()) == int(ol.argmax())
    close_all(a, b, o, s, m)


def test_decode_batch_errors(tmpdir_models):
    spm, spt = model_files(tmpdir_models, "qwen3-hd128")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 64)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    a, b = spkv.Backend(qm, 64, exact=True), spkv.Backend(qm, 64, exact=False)
    with pytest.raises(RuntimeError, match="differ in mode"):
        spkv.Backend.decode_batch([a, b], [1, 2], 2048)
    with pytest.raises(RuntimeError, match="appears twice"):
        spkv.Backend.decode_batch([a, a], [1, 2], 2048)
    with pytest.raises(RuntimeError, match="out of vocabulary"):
        spkv.Backend.decode_batch([a], [5000], 2048)
    assert a.position() == 0
    a.close(); b.close(); close_all(s, m)


def test_long_prefill_vs_oracle(tmpdir_models):
    """A 300-token prompt (three prefill batches) then decode: exact mode == oracle."""
    spm, spt = model_files(tmpdir_models, "gemma3-tiny")
    m, s, o, be, res = run_pair(spm, spt, True, n_prompt=300, n_gen=8, pmax=512)
    check(res, True)
    close_all(s, o, m)


def test_clone_fork_and_rewind(tmpdir_models):
    """sp_session_clone forks the device KV copy-on-write; both sessions then
    decode independently and bit-identically to independent oracle sessions;
    rewind + re-decode reproduces the same logits (exact mode)."""
    spm, spt = model_files(tmpdir_models, "gemma3-tiny")
    m, s, o, be, res = run_pair(spm, spt, True, n_prompt=70, n_gen=3)   # crosses a 64-position page
    lg = np.zeros(o.V, np.float32)
    c = s.clone()
    assert c.backend_handle() and c.backend_handle() != s.backend_handle()
    oc = o.clone()
    for t in (11, 12, 13):                     # diverge the two
        assert s.decode(t, lg) == 0; a = lg.copy(); assert same_bits(a, o.step(t))
        assert c.decode(t + 100, lg) == 0; b = lg.copy(); assert same_bits(b, oc.step(t + 100))
    assert s.rewind(2) == 0 and o.rewind(2) == 0
    assert s.decode(12, lg) == 0 and same_bits(lg, o.step(12))
    assert c.position() == oc.pos() and s.position() == o.pos()
    c.close(); oc.close(); close_all(s, o, m)


def test_window_ring_rewind(tmpdir_models):
    """Window layers on a ring of window + max_rewind positions: decode through
    several ring wraps, rewind within the bound (exact == oracle), beyond it fails."""
    spm, spt = model_files(tmpdir_models, "gemma3-tiny")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 512)
    be = spkv.Backend(spkv.l1().sp_session_qwen3_model(s.h), 512, exact=True)
    spkv.check(spkv.kv().sp_hipkv_set_max_rewind(be.h, 8), "set_max_rewind")
    o = orc.Oracle(spm, 512, orc.EXACT)
    lg = np.zeros(o.V, np.float32)
    toks = prompt(300, o.V, seed=5)
    be.prefill(toks[:200])
    for t in toks[:200]:
        o.step(int(t), False)
    for t in toks[200:260]:
        be.decode(int(t), lg); assert same_bits(lg, o.step(int(t)))
    assert be.rewind(8) == 0 and o.rewind(8) == 0
    for t in toks[260:270]:
        be.decode(int(t), lg); assert same_bits(lg, o.step(int(t)))
    assert be.rewind(400) != 0                          # beyond the resident position
    be.close(); close_all(s, o, m)


@pytest.mark.parametrize("name", ["gemma3-w200", "gemma3-g4w130", "gemma3-hd128w100", "gemma3-g4hd256w150",
                                  "gemma3-g4hd64w150"])
@pytest.mark.parametrize("ring", [False, True])
def test_window_layers_one_launch(tmpdir_models, name, ring):
    """Exact decode on window layers scores and sums V in one launch whose
    workgroups hand off through tagged slots.  Windows of 100 to 200 positions
    span 2 to 5 64-position chunks (the first and last ragged), at every
    head_dim x group instance (256/128/64 x 2/4); decoding from position 179 to
    399 crosses the point where the window starts to slide and, on a ring of
    window + 8 positions (plain launches), wraps it.  Logits every step and the
    last 100 positions' K/V of every layer bit-exact."""
    spm, spt = model_files(tmpdir_models, name)
    m = spkv.Model(spm, spt); s = spkv.Session(m, 512)
    be = spkv.Backend(spkv.l1().sp_session_qwen3_model(s.h), 512, exact=True, graph=not ring)
    if ring:
        spkv.check(spkv.kv().sp_hipkv_set_max_rewind(be.h, 8), "set_max_rewind")
    o = orc.Oracle(spm, 512, orc.EXACT)
    lg = np.zeros(o.V, np.float32)
    toks = prompt(180, o.V, seed=11)
    be.prefill(toks[:-1])
    for t in toks[:-1]:
        o.step(int(t), False)
    t = int(toks[-1])
    for k in range(220):
        be.decode(t, lg)
        ol = o.step(t)
        assert same_bits(lg, ol), f"step {k}: max rel {rel(lg, ol):.3e}"
        t = int(ol.argmax())
    pos, kvd = be.position(), o.NKV * o.HD
    for layer in range(o.NL):
        kg, vg = be.read_kv(layer, pos - 100, 100, kvd)
        kc, vc = o.kv(layer, pos - 100, 100)
        assert same_bits(kg, kc) and same_bits(vg, vc), f"layer {layer}"
    be.close(); close_all(s, o, m)


def test_window_one_launch_switch(tmpdir_models):
    """sp_hipkv_set_window_one_launch(0) sends exact window layers through the
    score + V-sum launches: the same bits as the one-launch kernel, step by
    step, on a fork of the same handle (graphs recaptured at each switch)."""
    name = "gemma3-w200"
    spm, spt = model_files(tmpdir_models, name)
    m = spkv.Model(spm, spt); s = spkv.Session(m, 512)
    a = spkv.Backend(spkv.l1().sp_session_qwen3_model(s.h), 512, exact=True)
    V = SMALL[name]["vocab"]
    a.prefill(prompt(230, V, seed=17))
    b = a.fork()
    b.set_window_one_launch(False)
    la, lb = np.zeros(V, np.float32), np.zeros(V, np.float32)
    t = 5
    for k in range(40):
        if k == 20:
            b.set_window_one_launch(True); a.set_window_one_launch(False)
        a.decode(t, la); b.decode(t, lb)
        assert same_bits(la, lb), f"step {k}"
        t = int(la.argmax())
    a.close(); b.close(); s.close(); m.close()


@pytest.mark.parametrize("name,n_prompt,pmax", [("gemma3-w1", 70, 256), ("gemma3-w2100", 2150, 2304)])
def test_window_edges(tmpdir_models, name, n_prompt, pmax):
    """Window edge cases, exact mode, bit for bit every step: a one-position
    window (one chunk: one workgroup finishes the whole head) and a window of
    2 100 positions (over 32 chunks: the two-kernel path), decoding across a
    64-position boundary and, for 2 100, past the point where the window starts
    to slide."""
    spm, spt = model_files(tmpdir_models, name, max_context=pmax)
    m = spkv.Model(spm, spt); s = spkv.Session(m, pmax)
    be = spkv.Backend(spkv.l1().sp_session_qwen3_model(s.h), pmax, exact=True)
    o = orc.Oracle(spm, pmax, orc.EXACT)
    lg = np.zeros(o.V, np.float32)
    toks = prompt(n_prompt, o.V, seed=13)
    be.prefill(toks[:-1])
    for t in toks[:-1]:
        o.step(int(t), False)
    t = int(toks[-1])
    for k in range(pmax - n_prompt - 8):
        be.decode(t, lg)
        ol = o.step(t)
        assert same_bits(lg, ol), f"step {k}: max rel {rel(lg, ol):.3e}"
        t = int(ol.argmax())
    be.close(); close_all(s, o, m)


def test_greedy_device_loop_matches_abi(tmpdir_models):
    """The device-resident greedy loop (argmax on the GPU) generates the same tokens
    as host-driven sp_decode_step + argmax, and as the oracle (exact mode)."""
    spm, spt = model_files(tmpdir_models, "qwen3-hd128")
    m, s, o, be, res = run_pair(spm, spt, True, n_prompt=20, n_gen=0)
    first = int(res[-1][1].argmax())
    f = be.fork()
    toks, ms = f.greedy(first, 12)
    t = first
    for k in range(12):
        ol = o.step(t); t = int(ol.argmax())
        assert toks[k] == t, f"step {k}"
    f.close(); close_all(s, o, m)


def test_errors_are_reported(tmpdir_models):
    spm, spt = model_files(tmpdir_models, "qwen3-tiny")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 64)
    be = spkv.Backend(spkv.l1().sp_session_qwen3_model(s.h), 4)
    lg = np.zeros(1000, np.float32)
    with pytest.raises(RuntimeError, match="out of vocabulary"):
        be.decode(1000, lg)
    assert be.position() == 0
    for t in range(4):
        be.decode(t, lg)
    with pytest.raises(RuntimeError, match="context full"):
        be.decode(1, lg)
    assert be.rewind(5) != 0 and be.position() == 4
    assert spkv.kv().sp_hipkv_set_mode(be.h, 1) != 0          # mode fixed once tokens are resident
    be.close(); close_all(s, m)


@pytest.mark.slow
@pytest.mark.parametrize("exact", [True, False])
def test_config1_qwen3_single_layer(tmpdir_models, exact):
    """Config 1: one Qwen3-0.6B layer, vocab 151936, a 512-token SplitMix64 (seed
    1) prompt, then 64 greedy decode steps -- the GPU logits and trajectory vs the
    oracle (exact: bit for bit; float: rel 1e-3, same argmax)."""
    spm, spt = model_files(tmpdir_models, "qwen3-0.6b-1layer", max_context=1024)
    m, s, o, be, res = run_pair(spm, spt, exact, n_prompt=512, n_gen=64, pmax=1024)
    check(res, exact)
    close_all(s, o, m)


def _set_norm(spm, name, value):
    """Rewrite one f32 norm tensor of a .sp-model file in place (the loader checks
    the header CRC and the tokenizer hash; the tensor bytes are data)."""
    import struct
    b = bytearray(open(spm, "rb").read())
    n = struct.unpack_from("<I", b, 316)[0]
    data_off = struct.unpack_from("<Q", b, 328)[0]
    for i in range(n):
        off = 512 + 256 * i
        if b[off:off + 80].rstrip(b"\0") == name.encode():
            toff, size = struct.unpack_from("<QQ", b, off + 152)
            b[data_off + toff:data_off + toff + size] = np.full(size // 4, value, np.float32).tobytes()
            open(spm, "wb").write(bytes(b))
            return
    raise KeyError(name)


def test_exact_v_clamp_is_counted(tmp_path):
    """V beyond the exact grid's bound (|v| >= 128, here from a large attn_norm
    weight): the device clamps exactly as the oracle does (logits bit-exact) and
    counts the clamped V heads as the oracle does; a normal model counts none."""
    import shutil
    spm, spt = model_files(tmp_path, "qwen3-tiny")
    big = str(tmp_path / "bigv.spm"); shutil.copy(spm, big)
    for layer in range(2):
        _set_norm(big, f"blk.{layer}.attn_norm.weight", 3000.0)
    for path, want_clamps in ((spm, False), (big, True)):
        m, s, o, be, res = run_pair(path, spt, True, n_prompt=12, n_gen=6, pmax=64)
        check(res, True)
        assert be.v_clamps() == o.v_clamps()
        assert (o.v_clamps() > 0) == want_clamps
        close_all(s, o, m)


def test_concurrent_handles_window_layers(tmpdir_models):
    """Three handles of one model decode from three threads at once (each on
    its own stream, graph replay), windows of 200 positions over 4-5 chunks:
    every step's logits equal those of a fresh handle fed the same tokens
    afterwards, alone (exact mode, bit for bit).  The one-launch window kernel
    polls for its sibling workgroups; concurrent launches from the other
    handles' streams must not change that."""
    import threading
    name, pmax = "gemma3-w200", 512
    spm, spt = model_files(tmpdir_models, name)
    m = spkv.Model(spm, spt); s = spkv.Session(m, pmax)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    V = SMALL[name]["vocab"]
    prompts = [prompt(n, V, seed=40 + i) for i, n in enumerate((230, 260, 300))]
    feeds = [prompt(40, V, seed=50 + i) for i in range(3)]
    hs = []
    for pr in prompts:
        b = spkv.Backend(qm, pmax, exact=True)
        b.prefill(pr)
        hs.append(b)
    out = [[None] * 40 for _ in range(3)]
    errs = []

    def run(i):
        try:
            for k in range(40):
                lg = np.zeros(V, np.float32)
                hs[i].decode(int(feeds[i][k]), lg)
                out[i][k] = lg
        except Exception as e:                       # reported below
            errs.append((i, repr(e)))

    th = [threading.Thread(target=run, args=(i,)) for i in range(3)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errs, errs
    for i in range(3):
        c = spkv.Backend(qm, pmax, exact=True)
        c.prefill(prompts[i])
        lg = np.zeros(V, np.float32)
        for k in range(40):
            c.decode(int(feeds[i][k]), lg)
            assert same_bits(out[i][k], lg), (i, k)
        c.close()
    for b in hs:
        b.close()
    s.close(); m.close()


def test_kernel_times_are_greedy_steps(tmpdir_models):
    """sp_hipkv_kernel_times runs n greedy steps with every kernel class timed:
    the GEMV classes by events their launches record at the kernel's start and
    end, the attention classes by events on the stream; every class of the
    model gets launches and positive time, and the handle goes on bit-identically
    to a fork that ran the same steps untimed through the device greedy loop."""
    name = "gemma3-w200"
    spm, spt = model_files(tmpdir_models, name)
    m = spkv.Model(spm, spt); s = spkv.Session(m, 512)
    a = spkv.Backend(spkv.l1().sp_session_qwen3_model(s.h), 512, exact=True)
    V = SMALL[name]["vocab"]
    a.prefill(prompt(240, V, seed=19))
    b = a.fork()
    ms, nl, by = a.kernel_times(7, 4)
    for c in range(7):                          # QKV, O, gate/up, down, LM head, global, window attention
        assert nl[c] > 0 and ms[c] > 0 and by[c] > 0, (c, nl[c], ms[c], by[c])
    toks, _ = b.greedy(7, 4)
    assert a.position() == b.position()
    la, lb = np.zeros(V, np.float32), np.zeros(V, np.float32)
    a.decode(int(toks[-1]), la); b.decode(int(toks[-1]), lb)
    assert same_bits(la, lb)
    a.close(); b.close(); s.close(); m.close()
