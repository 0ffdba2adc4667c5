"""GPU parity of the Spinor-63 KV codec (SP_KV_SPINOR sessions) against the oracle.

The oracle's Spinor sessions are pinned to the compiled reference (codec bytes
and decode logits, tests/test_oracle.py).  Bars here, through the C ABI:
  exact mode -- logits and every resident K/V element BIT-EXACT to the oracle's
                exact mode with the codec (the int32 grid of the decoded values);
  float mode -- every resident value is code * multiplier of its chunk and lies
                within one quantization step of the oracle's decoded value (the
                codec is discontinuous: a float difference of one ulp can move
                a value across a rounding boundary); logits within rel 1e-3 of
                an oracle that attends over the device's own decoded rows (its
                K/V rows forced from the device after each step).
Cases: head_dim 64/128/256, GQA 2 and 4, clipping windows, prefill through
sp_prefill_chunk (batched) and step by step, forks, batched multi-session
decode, the codec knob's guards.
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
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def chunks(hd):
    nb = 1 if hd <= 55 else (hd + 54) // 55
    base, extra = hd // nb, hd % nb
    out, off = [], 0
    for b in range(nb):
        n = base + (1 if b < extra else 0)
        out.append((off, n)); off += n
    return out


def check_float_rows(dev, ref, hd, steps=1):
    """dev, ref: [n][NKV*HD] decoded K or V rows (device, oracle); at most
    `steps` quantization steps apart (1: the layer's inputs agree to float
    rounding, a code may flip at a rounding boundary; later layers inherit the
    earlier layers' flips through their inputs)."""
    rows_d = dev.reshape(-1, hd); rows_r = ref.reshape(-1, hd)
    for lo, n in chunks(hd):
        d, r = rows_d[:, lo:lo + n], rows_r[:, lo:lo + n]
        amax = np.abs(d).max(axis=1, keepdims=True)
        mul = np.where(amax > 0, amax, 1.0).astype(np.float32) / np.float32(127)
        code = np.rint(d / mul)
        assert np.abs(code).max() <= 127
        assert np.allclose(code * mul, d, rtol=1e-6, atol=0), "not code * chunk multiplier"
        step = np.abs(r).max(axis=1, keepdims=True) / 127
        assert (np.abs(d - r) <= 1.01 * steps * step + 1e-6).all(), f"beyond {steps} quantization step(s)"
        if steps == 1:
            assert np.mean(np.abs(d - r) > 0.5 * step) < 0.01, "more than 1% of the codes differ"


def run_spinor(tmpdir_models, name, exact, n_prompt, n_gen, flags=spkv.SP_KV_SPINOR, pmax=256):
    """Device session vs oracle, step by step.  Exact: pairs (device, oracle)
    logits.  Float: pairs (device, forced oracle) -- the forced oracle gets the
    device's decoded K/V rows of every layer up to the step's position before
    it steps, so both attend over the same codes."""
    spm, spt = model_files(tmpdir_models, name)
    m = spkv.Model(spm, spt)
    s = spkv.Session(m, pmax, flags=flags)
    o = orc.Oracle(spm, pmax, orc.EXACT if exact else orc.FLOAT, kv_flags=orc.KV_SPINOR)
    of = None if exact else orc.Oracle(spm, pmax, orc.FLOAT, kv_flags=orc.KV_SPINOR)
    if of:
        of.set_kv_forced(True)
    V = o.V
    pr = prompt(n_prompt, V)
    lg = np.zeros(V, np.float32)
    s.attach(pmax, exact=exact)
    be = spkv.Backend.wrap(s.backend_handle())
    kvd = o.NKV * o.HD

    def oracle_logits(tok, ol):
        if not of:
            return ol
        p = be.position()
        for layer in range(o.NL):
            k, v = be.read_kv(layer, 0, p, kvd)
            assert of.set_kv(layer, 0, k, v) == 0
        assert of.set_pos(p - 1) == 0
        return of.step(int(tok))

    spkv.check(s.prefill(pr, lg), "sp_prefill_chunk")
    for t in pr:
        ol = o.step(int(t))
    res = [(lg.copy(), oracle_logits(pr[-1], ol))]
    t = int(ol.argmax())
    for _ in range(n_gen):
        spkv.check(s.decode(t, lg), "sp_decode_step")
        ol = o.step(t)
        res.append((lg.copy(), oracle_logits(t, ol)))
        t = int(lg.argmax())
    if of:
        of.close()
    return m, s, o, be, res


@pytest.mark.parametrize("name", ["qwen3-tiny", "gemma3-tiny", "qwen3-hd128", "gemma3-hd256", "qwen3-g4"])
@pytest.mark.parametrize("exact", [True, False])
def test_spinor_decode_parity(tmpdir_models, name, exact):
    m, s, o, be, res = run_spinor(tmpdir_models, name, exact, n_prompt=40, n_gen=12)
    for i, (g, c) in enumerate(res):
        if exact:
            assert same_bits(g, c), f"step {i}: max rel {rel(g, c):.3e}"
        else:
            assert rel(g, c) < FLOAT_TOL, f"step {i}: rel {rel(g, c):.3e}"
            assert int(g.argmax()) == int(c.argmax()), f"step {i}: argmax"
    kvd, hd = o.NKV * o.HD, o.HD
    n = be.position()
    for layer in range(o.NL):
        kd, vd = be.read_kv(layer, 0, n, kvd)
        ko, vo = o.kv(layer, 0, n)
        if exact:
            assert same_bits(kd, ko) and same_bits(vd, vo), f"layer {layer}"
        else:
            st = 1 if layer == 0 else 3
            check_float_rows(kd, ko, hd, st); check_float_rows(vd, vo, hd, st)
    info = np.zeros(8, np.int64)
    spkv.check(spkv.kv().sp_hipkv_info(be.h, spkv.ptr(info)), "info")
    rb = hd * 4 if exact else (hd + 4 * len(chunks(hd)) + 15) // 16 * 16
    assert info[2] == 2 * o.NKV * rb
    s.close(); o.close(); m.close()


def test_spinor_ref_flag_and_codec_in_path(tmpdir_models):
    """SP_KV_SPINOR_REF sessions decode exactly as SP_KV_SPINOR ones (the
    reference's codec identity); both differ from the plain cache."""
    m1, s1, o1, _, r1 = run_spinor(tmpdir_models, "qwen3-hd128", True, 20, 4, flags=spkv.SP_KV_SPINOR)
    m2, s2, o2, _, r2 = run_spinor(tmpdir_models, "qwen3-hd128", True, 20, 4, flags=spkv.SP_KV_SPINOR_REF)
    for (a, _), (b, _) in zip(r1, r2):
        assert same_bits(a, b)
    spm, spt = model_files(tmpdir_models, "qwen3-hd128")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 256)
    s.attach(256, exact=True)
    lg = np.zeros(o1.V, np.float32)
    spkv.check(s.prefill(prompt(20, o1.V), lg), "sp_prefill_chunk")
    assert not same_bits(lg, r1[0][0])
    for x in (s, s1, s2, o1, o2, m, m1, m2):
        x.close()


@pytest.mark.parametrize("exact", [True, False])
def test_spinor_batched_prefill_matches_stepwise(tmpdir_models, exact):
    """Batched prefill (MFMA GEMMs, token-batched attention over code rows)
    leaves the K/V and next logits of one decode step per token."""
    spm, spt = model_files(tmpdir_models, "gemma3-hd256")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 512)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    V = 2048
    pr = prompt(200, V, seed=7)
    lg1, lg2 = np.zeros(V, np.float32), np.zeros(V, np.float32)
    b1 = spkv.Backend(qm, 512, exact=exact, kv_codec=spkv.KV_SPINOR)
    b2 = spkv.Backend(qm, 512, exact=exact, batch_prefill=False, kv_codec=spkv.KV_SPINOR)
    b1.prefill(pr[:-1]); b1.decode(int(pr[-1]), lg1)
    b2.prefill(pr[:-1]); b2.decode(int(pr[-1]), lg2)
    if exact:
        assert same_bits(lg1, lg2)
    else:
        assert rel(lg1, lg2) < 1e-4 and int(lg1.argmax()) == int(lg2.argmax())
    kvd = 2 * 256
    for layer in range(6):
        k1, v1 = b1.read_kv(layer, 0, 200, kvd)
        k2, v2 = b2.read_kv(layer, 0, 200, kvd)
        if exact:
            assert same_bits(k1, k2) and same_bits(v1, v2), f"layer {layer}"
        else:
            st = 1 if layer == 0 else 3
            check_float_rows(k1, k2, 256, st); check_float_rows(v1, v2, 256, st)
    b1.close(); b2.close(); s.close(); m.close()


@pytest.mark.parametrize("exact", [True, False])
def test_spinor_fork_and_decode_batch(tmpdir_models, exact):
    """Copy-on-write forks of code-row pages and batched multi-session decode
    give what independent handles give (exact: bit for bit)."""
    spm, spt = model_files(tmpdir_models, "qwen3-hd128")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 256)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    V = 2048
    lens = [9, 64, 70]
    A = [spkv.Backend(qm, 256, exact=exact, kv_codec=spkv.KV_SPINOR) for _ in lens]
    B = [spkv.Backend(qm, 256, exact=exact, kv_codec=spkv.KV_SPINOR) for _ in lens]
    toks = []
    for i, n in enumerate(lens):
        pr = prompt(n, V, seed=20 + i)
        A[i].prefill(pr[:-1]); B[i].prefill(pr[:-1]); toks.append(int(pr[-1]))
    lg = np.zeros(V, np.float32)
    for step in range(4):
        F = [a.fork() for a in A]
        lga, nxt = spkv.Backend.decode_batch(F, toks, V)
        for i in range(len(lens)):
            B[i].decode(toks[i], lg)
            if exact:
                assert same_bits(lga[i], lg), f"step {step} session {i}"
            else:
                assert rel(lga[i], lg) < FLOAT_TOL and int(lga[i].argmax()) == int(lg.argmax())
        for a in A:
            a.close()
        A = F
        toks = [int(t) for t in nxt]
    for x in A + B:
        x.close()
    s.close(); m.close()


def test_spinor_codec_guards(tmpdir_models):
    spm, spt = model_files(tmpdir_models, "qwen3-hd128")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 64)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    a = spkv.Backend(qm, 64, exact=True)
    b = spkv.Backend(qm, 64, exact=True, kv_codec=spkv.KV_SPINOR)
    assert spkv.kv().sp_hipkv_set_kv_codec(a.h, 7) != 0
    with pytest.raises(RuntimeError, match="differ in mode, KV codec"):
        spkv.Backend.decode_batch([a, b], [1, 2], 2048)
    lg = np.zeros(2048, np.float32)
    b.decode(1, lg)
    assert spkv.kv().sp_hipkv_set_kv_codec(b.h, 0) != 0
    assert "fixed once tokens are resident" in spkv.last_error()
    # codec then mode switches before the first token re-page the cache
    c = spkv.Backend(qm, 64, kv_codec=spkv.KV_SPINOR)
    spkv.check(spkv.kv().sp_hipkv_set_mode(c.h, 1), "set_mode")
    lc = np.zeros(2048, np.float32)
    c.decode(1, lc)
    assert same_bits(lc, lg)
    for x in (a, b, c):
        x.close()
    s.close(); m.close()


@pytest.mark.parametrize("exact", [True, False])
def test_recycled_handle_drops_codec_graphs(tmpdir_models, exact):
    """A closed handle is kept as a shell with its captured step graphs; a
    plain handle (or fork) that reuses a Spinor handle's shell decodes as a
    fresh plain handle does, and the other way round (exact mode: bit for bit;
    its step graphs bake the codec into the fused score pass)."""
    spm, spt = model_files(tmpdir_models, "qwen3-hd128")
    m = spkv.Model(spm, spt); s = spkv.Session(m, 128)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    V = 2048
    pr = prompt(30, V, seed=5)
    keep = spkv.Backend(qm, 128, exact=exact)     # keeps the model referenced: closed handles become shells
    ref = {}
    for codec in (spkv.KV_PLAIN, spkv.KV_SPINOR):
        b = spkv.Backend(qm, 128, exact=exact, kv_codec=codec)
        lg = np.zeros(V, np.float32)
        b.prefill(pr[:-1]); b.decode(int(pr[-1]), lg); b.decode(7, lg)
        ref[codec] = lg.copy()
        b.close()
    assert not same_bits(ref[spkv.KV_PLAIN], ref[spkv.KV_SPINOR])
    for codec in (spkv.KV_PLAIN, spkv.KV_SPINOR, spkv.KV_PLAIN):
        b = spkv.Backend(qm, 128, exact=exact, kv_codec=codec)
        lg = np.zeros(V, np.float32)
        b.prefill(pr[:-1]); b.decode(int(pr[-1]), lg)
        f = b.fork(); b.close()
        f.decode(7, lg)
        if exact:
            assert same_bits(lg, ref[codec]), codec
        else:
            assert rel(lg, ref[codec]) < 1e-6, codec
        f.close()
    keep.close(); s.close(); m.close()
