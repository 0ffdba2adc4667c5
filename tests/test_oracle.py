"""Pinning the oracle (the CPU restatement that the GPU path is checked against).

Float mode:  bit-identical to the compiled reference (oracle/_ref, built from the
             reference's own C sources) on Qwen3 and Gemma3 models with a
             clipping sliding window -- prefill logits and every decode step.
Islands:     bit-identical to the reference's exact islands on the inputs of
             core/exact_islands/exact_islands_test.c:32-97, plus that test's own
             properties (fidelity, order immunity, determinism) and the closed
             forms of every integer constant.
Build-defined exact primitives (CORDIC RoPE, integer GEMV, SiLU, V-sum
rounding) are pinned by closed forms and exact rational arithmetic in Python.
"""
import ctypes
import math
from decimal import Decimal, getcontext
from fractions import Fraction

import numpy as np
import pytest

import orc
import spkv
from helpers import island_inputs, model_files, prompt, spinor_vectors

P = orc.ptr


def _ref():
    R = orc.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref (the compiled reference) not built")
    return R


# ---------------------------------------------------------------- float mode vs reference
@pytest.mark.parametrize("name", ["qwen3-tiny", "gemma3-tiny", "qwen3-g4"])
def test_float_decode_bitexact_vs_reference(tmpdir_models, name):
    R = _ref()
    spm, spt = model_files(tmpdir_models, name)
    o = orc.Oracle(spm, 64, orc.FLOAT)
    V = o.V
    n_prompt, n_gen = 24, 16
    pr = prompt(n_prompt, V)
    pre = np.zeros(V, np.float32); lg = np.zeros((n_gen, V), np.float32); fed = np.zeros(n_gen, np.int32)
    assert R.refh_decode(spm.encode(), spt.encode(), P(pr), n_prompt, n_gen, None, P(pre), P(lg), P(fed)) == 0
    for i, t in enumerate(pr):
        ol = o.step(int(t), i == n_prompt - 1)
    assert np.array_equal(ol.view(np.uint32), pre.view(np.uint32)), "prefill logits"
    for k in range(n_gen):
        ol = o.step(int(fed[k]))
        assert np.array_equal(ol.view(np.uint32), lg[k].view(np.uint32)), f"decode step {k}"
    o.close()


def test_float_clone_rewind_semantics(tmpdir_models):
    """core/session/session_test.c:171-206 semantics on the oracle: clone decodes
    bit-identically; rewind then re-decode reproduces the original logits."""
    spm, _ = model_files(tmpdir_models, "qwen3-tiny")
    o = orc.Oracle(spm, 64)
    for t in prompt(9, o.V):
        last = o.step(int(t))
    c = o.clone()
    a = o.step(7); b = c.step(7)
    assert np.array_equal(a, b)
    assert o.rewind(2) == 0 and o.pos() == 8
    assert o.rewind(999) != 0
    o.step(int(prompt(9, o.V)[-1]))          # re-decode position 8 with the same token
    again = o.step(7)
    assert np.array_equal(again, a)
    c.close(); o.close()


# ---------------------------------------------------------------- islands
def _island_inputs():
    return island_inputs()


def test_islands_bitexact_vs_reference():
    R = _ref()
    L = orc.lib()
    x, w, z, g = _island_inputs()
    a = np.zeros_like(x); b = np.zeros_like(x)
    L.orc_rmsnorm_exact(P(x), P(w), x.size, P(a)); R.sp_rmsnorm_exact(P(x), P(w), x.size, P(b))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    pa = np.zeros(z.size); pb = np.zeros(z.size)
    L.orc_softmax_exact(P(z), z.size, P(pa)); R.sp_softmax_exact(P(z), z.size, P(pb))
    assert np.array_equal(pa.view(np.uint64), pb.view(np.uint64))
    ga = np.zeros_like(g); gb = np.zeros_like(g)
    L.orc_gelu_exact(P(g), g.size, P(ga)); R.sp_gelu_exact(P(g), g.size, P(gb))
    assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32))


def test_islands_properties():
    """exact_islands_test.c:32-97 gates, run on the oracle without the reference."""
    L = orc.lib()
    x, w, z, g = _island_inputs()
    out = np.zeros_like(x)
    L.orc_rmsnorm_exact(P(x), P(w), x.size, P(out))
    yf = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2)) * w
    assert np.linalg.norm(out - yf) / np.linalg.norm(yf) < 1e-4
    one = np.ones_like(x); oa = np.zeros_like(x); orr = np.zeros_like(x)
    L.orc_rmsnorm_exact(P(x), P(one), x.size, P(oa))
    xr = np.ascontiguousarray(x[::-1])
    L.orc_rmsnorm_exact(P(xr), P(one), x.size, P(orr))
    assert np.array_equal(orr, oa[::-1])                      # order immunity
    p = np.zeros(z.size); pr = np.zeros(z.size)
    L.orc_softmax_exact(P(z), z.size, P(p))
    e = np.exp(z.astype(np.float64) - z.max()); e /= e.sum()
    assert np.abs(p - e).max() < 1e-5
    zr = np.ascontiguousarray(z[::-1])
    L.orc_softmax_exact(P(zr), z.size, P(pr))
    assert np.array_equal(pr, p[::-1])
    go = np.zeros_like(g); go2 = np.zeros_like(g)
    L.orc_gelu_exact(P(g), g.size, P(go)); L.orc_gelu_exact(P(g), g.size, P(go2))
    gd = g.astype(np.float64)
    gf = 0.5 * gd * (1 + np.tanh(math.sqrt(2 / math.pi) * (gd + 0.044715 * gd ** 3)))
    assert np.linalg.norm(go - gf) / np.linalg.norm(gf) < 1e-4
    assert np.array_equal(go, go2)


def test_island_constants_closed_form():
    """Every integer constant of the islands equals round(closed form * 2^30)."""
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    S = Decimal(2) ** 30
    assert int((Decimal(1) / ln2 * S).to_integral_value()) == 1549082005        # log2(e)
    fact = 1
    expc = [1073741824, 744261118, 257941248, 59597083, 10327387, 1431680, 165394]
    for k in range(7):
        fact *= max(k, 1)
        assert int((ln2 ** k / fact * S).to_integral_value()) == expc[k]
    pi = Decimal("3.14159265358979323846264338327950288419716939937510582097494459")
    assert int(((2 / pi).sqrt() * S).to_integral_value()) == 856722024
    assert int((Decimal("0.044715") * S).to_integral_value()) == 48012366


# ---------------------------------------------------------------- build-defined exact primitives
PI = Fraction(314159265358979323846264338327950288419716939937510582097494459, 10 ** 62)


def test_cordic_sincos():
    L = orc.lib()
    co = ctypes.c_int32(); si = ctypes.c_int32()
    two_pi_q60 = 7244019458077122842
    assert two_pi_q60 == round(2 * PI * 2 ** 60) and 1811004864519280711 == round(PI / 2 * 2 ** 60)
    rng = np.random.default_rng(0)
    worst = 0.0
    for th in list(rng.integers(0, two_pi_q60, 400)) + [0, two_pi_q60 // 4, two_pi_q60 // 2, two_pi_q60 - 1]:
        L.orc_cordic_sincos(int(th), ctypes.byref(co), ctypes.byref(si))
        t = int(th) / 2 ** 60
        worst = max(worst, abs(co.value / 2 ** 30 - math.cos(t)), abs(si.value / 2 ** 30 - math.sin(t)))
    assert worst < 4e-9                      # Q30 output resolution is ~1e-9


def test_rope_freq_table():
    L = orc.lib()
    for base in (1e6, 1e4):
        for d in (64, 128, 256):
            for i in range(0, d // 2, 7):
                f = L.orc_rope_freq_q60(base, i, d) / 2 ** 60
                exact = float(base) ** (-2.0 * i / d)
                assert abs(f - exact) <= 1e-15 + 2e-14 * exact, (base, d, i)


def test_rope_exact_vs_libm():
    """CORDIC RoPE agrees with the mathematically exact rotation (angle computed in
    double) to float rounding, and preserves pair norms (forward_kernels_test.c)."""
    L = orc.lib()
    rng = np.random.default_rng(2)
    for p in (0, 1, 17, 1000, 32768, 131071):
        v = rng.standard_normal(256).astype(np.float32)
        out = v.copy()
        L.orc_rope_exact(P(out), 256, p, 1e6)
        half = 128
        i = np.arange(half)
        th = p * np.power(1e6, -2.0 * i / 256)
        c, s = np.cos(th), np.sin(th)
        a, b = v[:half].astype(np.float64), v[half:].astype(np.float64)
        ref = np.concatenate([a * c - b * s, a * s + b * c])
        assert np.abs(out - ref).max() < 1e-5 * max(1.0, np.abs(ref).max())
        n0 = a * a + b * b; n1 = out[:half].astype(np.float64) ** 2 + out[half:].astype(np.float64) ** 2
        assert np.abs(n0 - n1).max() < 1e-5 * n0.max()


def _q4b_tensor(rows, cols, seed, spread=False):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if spread:   # odd blocks x 2^13, even blocks x 2^-7, as the synthetic writer's spread rows
        w *= np.repeat(np.ldexp(1.0, np.where(np.arange(cols // 32) & 1, 13, -7)), 32).astype(np.float32)
    codes = np.zeros((rows, cols // 2), np.uint8); bs = np.zeros((rows, cols // 32), np.uint16)
    for r in range(rows):
        spkv.l1().sp_q4b_quantize_row(P(w[r]), cols, P(codes[r]), P(bs[r]))
    return codes, bs


def _codes_int(codes):
    q = np.empty((codes.shape[0], codes.shape[1] * 2), np.int64)
    q[:, 0::2] = codes & 15; q[:, 1::2] = codes >> 4
    return np.where(q >= 8, q - 16, q)


def _f16_frac(h):
    h = int(h); E5 = (h >> 10) & 31; m = h & 1023
    v = Fraction(1024 + m, 1) * Fraction(2) ** (E5 - 25) if E5 else Fraction(m) * Fraction(2) ** -24
    return -v if h & 0x8000 else v


@pytest.mark.parametrize("cols,spread", [(64, False), (256, False), (1024, False), (256, True), (1024, True)])
def test_exact_gemv_is_rne_of_rational(cols, spread):
    """y = RNE( sum_b f16(s_b) sum_i code_i * xq_i / 2^sh ) exactly, with xq the
    per-vector power-of-two grid of x (max |xq| < 2^22); also for rows whose
    block scales span about 20 binary exponents (sums beyond 64 bits)."""
    rows = 24
    codes, bs = _q4b_tensor(rows, cols, cols, spread)
    if spread:   # every row past the int64 bound: exponent spread > 21 - ceil(log2 nblk)
        e = ((bs.astype(np.int64) >> 10) & 31)
        assert (e.max(axis=1) - e.min(axis=1)).min() > 21 - math.ceil(math.log2(cols // 32))
    x = (np.random.default_rng(9).standard_normal(cols) * np.float32(0.7)).astype(np.float32)
    x[3] = 0.0
    y = np.zeros(rows, np.float32)
    orc.lib().orc_q4b_gemv_exact(P(codes), P(bs), rows, cols, P(x), P(y))
    e = math.frexp(float(np.abs(x).max()))[1]
    sh = 22 - e
    xq = [int(np.rint(math.ldexp(float(v), sh))) for v in x]
    assert max(abs(v) for v in xq) < 2 ** 22
    q = _codes_int(codes)
    for r in range(rows):
        acc = Fraction(0)
        for b in range(cols // 32):
            acc += _f16_frac(bs[r, b]) * sum(int(q[r, i]) * xq[i] for i in range(b * 32, b * 32 + 32))
        exact = acc / 2 ** sh
        assert y[r] == np.float32(float(exact)) or abs(Fraction(float(y[r])) - exact) <= abs(exact) * Fraction(1, 2 ** 24)
    yf = np.zeros(rows, np.float32)
    orc.lib().orc_q4b_gemv(P(codes), P(bs), rows, cols, P(x), P(yf))
    assert np.abs(y - yf).max() <= 1e-5 * np.abs(yf).max()


def test_exact_silu_fidelity():
    g = np.linspace(-12, 12, 2001).astype(np.float32)
    out = np.zeros_like(g)
    orc.lib().orc_silu_exact(P(g), g.size, P(out))
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    assert np.abs(out - ref).max() < 2e-5 * 12


# ---------------------------------------------------------------- Spinor-63 KV codec
def test_spinor_crc8_check_value():
    """CRC-8/SMBus (poly 0x07, init 0, no reflection): the catalogued check value
    of the ASCII string "123456789" is 0xF4; a single flipped bit anywhere in a
    62-byte payload changes it (core/vht2/spinor_test.c:89-111)."""
    L = orc.lib()
    s = np.frombuffer(b"123456789", np.uint8).copy()
    assert L.orc_crc8(P(s), 9) == 0xF4
    rng = np.random.default_rng(3)
    pay = rng.integers(0, 256, 62, dtype=np.uint8)
    good = L.orc_crc8(P(pay), 62)
    for bit in range(62 * 8):
        c = pay.copy(); c[bit // 8] ^= np.uint8(1 << (bit % 8))
        assert L.orc_crc8(P(c), 62) != good


def test_spinor_block_layout_and_split():
    """The byte image of include/sp/spinor_block.h:29-72: little-endian float
    scale (the largest magnitude: 0.15625 -> 00 00 20 3E), exponent/basis/reserved
    bytes 0, coefficient i at body byte 17 i mod 55, the CRC over bytes 0..61;
    the balanced split of spinor_test.c:201-238 (128 -> 43/43/42)."""
    L = orc.lib()
    v = np.zeros(40, np.float32); v[5] = -0.15625; v[9] = 0.078125
    blk = np.zeros(63, np.uint8)
    L.orc_spinor_encode(P(v), 40, P(blk))
    assert list(blk[:7]) == [0x00, 0x00, 0x20, 0x3E, 0, 0, 0]
    assert blk[7 + (17 * 5) % 55].view(np.int8) == -127
    assert blk[7 + (17 * 9) % 55].view(np.int8) == 64          # 0.5 * 127 = 63.5 rounds away from zero
    assert np.count_nonzero(blk[7:62]) == 2
    assert blk[62] == L.orc_crc8(P(blk), 62)
    # every body byte is hit exactly once: 17 is a unit mod 55
    assert sorted((17 * i) % 55 for i in range(55)) == list(range(55))
    assert [L.orc_spinor_blocks_for(k) for k in (1, 55, 56, 110, 111, 128, 256)] == [1, 1, 2, 2, 3, 3, 5]
    x = np.arange(128, dtype=np.float32) + 1.0
    blks = np.zeros(3 * 63, np.uint8)
    L.orc_spinor_encode_vec(P(x), 128, P(blks))
    for b, (lo, n) in enumerate([(0, 43), (43, 43), (86, 42)]):
        one = np.zeros(63, np.uint8)
        L.orc_spinor_encode(P(np.ascontiguousarray(x[lo:lo + n])), n, P(one))
        assert np.array_equal(one, blks[63 * b:63 * b + 63])
    # decode: within half a quantization step of each block's scale, corruption rejected
    y = np.zeros(128, np.float32)
    assert L.orc_spinor_decode_vec(P(blks), 128, P(y)) == 0
    for lo, n in [(0, 43), (43, 43), (86, 42)]:
        sc = float(np.max(np.abs(x[lo:lo + n])))
        assert np.max(np.abs(y[lo:lo + n] - x[lo:lo + n])) <= sc / 254 * (1 + 1e-6)
    bad = blks.copy(); bad[70] ^= 1
    assert L.orc_spinor_decode_vec(P(bad), 128, P(y)) != 0


@pytest.mark.parametrize("k", [1, 7, 43, 55, 56, 64, 128, 200, 256, 512])
def test_spinor_codec_bitexact_vs_reference(k):
    """Byte images and decoded floats identical to the compiled reference's
    sp_spinor_encode_vec / sp_spinor_decode_vec (core/vht2/spinor_block.c:128-149)
    on vectors with zeros, ties at half a step, tiny and large magnitudes."""
    R = _ref(); L = orc.lib()
    for trial, x in enumerate(spinor_vectors(k)):
        nb = L.orc_spinor_blocks_for(k)
        a = np.zeros(63 * nb, np.uint8); b = np.zeros(63 * nb, np.uint8)
        L.orc_spinor_encode_vec(P(x), k, P(a)); R.sp_spinor_encode_vec(P(x), k, P(b))
        assert np.array_equal(a, b), (k, trial)
        ya = np.zeros(k, np.float32); yb = np.zeros(k, np.float32)
        assert L.orc_spinor_decode_vec(P(a), k, P(ya)) == R.sp_spinor_decode_vec(P(b), k, P(yb)) == 0
        assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))


@pytest.mark.parametrize("name", ["qwen3-tiny", "gemma3-tiny"])
@pytest.mark.parametrize("flags", [orc.KV_SPINOR, orc.KV_SPINOR_REF])
def test_float_decode_spinor_kv_bitexact_vs_reference(tmpdir_models, name, flags):
    """Sessions created with SP_KV_SPINOR (the block cache) and SP_KV_SPINOR_REF
    (the in-place round trip), core/session/sp_session.c:298-323 and :410-432:
    every decode step's logits bit-identical to the compiled reference's, and
    different from the f32 cache's (the codec is in the path).  The reference's
    prefill logits come from a full forward that keeps no K/V (sp_session.c:
    154-212, the cache is backfilled by the next decode step), so they carry no
    codec; the oracle prefills step by step and its prompt logits are not compared."""
    R = _ref()
    spm, spt = model_files(tmpdir_models, name)
    o = orc.Oracle(spm, 64, orc.FLOAT, kv_flags=flags)
    V = o.V
    n_prompt, n_gen = 20, 8
    pr = prompt(n_prompt, V)
    pre = np.zeros(V, np.float32); lg = np.zeros((n_gen, V), np.float32); fed = np.zeros(n_gen, np.int32)
    assert R.refh_decode_flags(spm.encode(), spt.encode(), P(pr), n_prompt, n_gen, None, P(pre), P(lg), P(fed), flags) == 0
    pre0 = np.zeros(V, np.float32); lg0 = np.zeros((n_gen, V), np.float32); fed0 = np.zeros(n_gen, np.int32)
    assert R.refh_decode(spm.encode(), spt.encode(), P(pr), n_prompt, n_gen, P(fed), P(pre0), P(lg0), P(fed0)) == 0
    assert np.array_equal(pre0, pre) and not np.array_equal(lg0[0], lg[0])
    for t in pr:
        o.step(int(t), False)
    for k in range(n_gen):
        ol = o.step(int(fed[k]))
        assert np.array_equal(ol.view(np.uint32), lg[k].view(np.uint32)), f"decode step {k}"
    o.close()


# ---------------------------------------------------------------- ARM recall router
def test_recall_projection_matrix_matches_reference():
    R = _ref(); L = orc.lib()
    for r, hd in ((16, 128), (8, 64), (32, 256)):
        a = np.zeros(r * hd, np.int8); b = np.zeros(r * hd, np.int8)
        L.orc_arm_build_R(P(a), r, hd); R.sp_arm_build_R(P(b), r, hd)
        assert np.array_equal(a, b) and set(np.unique(a)) == {-1, 1}


def _sel_geom(B, W, sink, pos):
    """sp_arm_select's clamps (core/arm/arm.c:110-160): identity?, sinks, candidate end, top-k."""
    if B <= 0 or pos + 1 <= B:
        return True, 0, 0, 0
    W = min(W, pos + 1); sink = min(sink, pos + 1)
    hi = min(max(pos + 1 - W, sink), pos + 1)
    return False, sink, hi, min(max(B - W - sink, 0), hi - sink)


def _check_selection(ri_a, ma, ri_b, mb, cand_a, B, W, sink, pos):
    """The oracle's list against the reference's: identical, or -- only when
    candidates equal to the k-th projected score straddle the cut, where the
    reference's quickselect keeps whichever its partitions leave in front --
    the same sinks, window and above-threshold positions, the tied slots filled
    with the lowest tied positions.  Returns True when the tie rule applied."""
    assert ma == mb
    if np.array_equal(ri_a[:ma], ri_b[:mb]):
        return False
    ident, sk, hi, topk = _sel_geom(B, W, sink, pos)
    assert not ident and 0 < topk < hi - sk
    nc = hi - sk
    pairs = cand_a[:2 * nc].reshape(nc, 2)
    score = {int(p): float(v) for v, p in zip(pairs[:, 0].view(np.float32), pairs[:, 1])}
    th = sorted(score.values(), reverse=True)[topk - 1]
    above = {p for p, v in score.items() if v > th}
    tied = sorted(p for p, v in score.items() if v == th)
    mine, ref = ri_a[sk:sk + topk], ri_b[sk:sk + topk]
    assert np.array_equal(ri_a[:sk], ri_b[:sk]) and np.array_equal(ri_a[sk + topk:ma], ri_b[sk + topk:mb])
    assert above <= set(mine.tolist()) and above <= set(ref.tolist())
    assert set(mine.tolist()) - above == set(tied[:topk - len(above)])
    assert (set(ref.tolist()) - above) <= set(tied)
    return True


@pytest.mark.parametrize("ties", [False, True])
def test_recall_selection_matches_reference(ties):
    """orc_arm_select against the reference's sp_arm_select (core/arm/arm.c:
    110-160): the same positions in the same order for budgets below and above
    the context, windows and sinks.  With duplicated sidecar rows (tied
    projected scores) the lists are identical unless the tie straddles the
    k-th score; there the oracle (like the device) keeps the lowest tied
    positions, where the reference keeps its quickselect's arrangement."""
    R = _ref(); L = orc.lib()
    rng = np.random.default_rng(8 + ties)
    straddled = 0
    for trial in range(40):
        hd, r, nkv = (64, 16, 2) if trial % 2 else (128, 8, 4)
        P_, layer = 300, int(rng.integers(0, 3))
        Rm = np.zeros(r * hd, np.int8); L.orc_arm_build_R(P(Rm), r, hd)
        projk = rng.standard_normal((3, P_, nkv, r)).astype(np.float32)
        if ties:
            src = rng.integers(0, P_, 40)
            projk[layer, rng.integers(0, P_, 40)] = projk[layer, src]
        q = rng.standard_normal(hd).astype(np.float32)
        pos = int(rng.integers(1, P_))
        B, W, sink, kvh = int(rng.integers(0, 120)), int(rng.integers(0, 40)), int(rng.integers(0, 6)), int(rng.integers(0, nkv))
        cand_a = np.zeros(2 * P_, np.int32); ri_a = np.zeros(P_, np.int32)
        cand_b = np.zeros(2 * P_, np.int32); ri_b = np.zeros(P_, np.int32)
        flat = np.ascontiguousarray(projk)
        pk = flat[layer, :, kvh, :]                         # this head's rows, stride nkv*r
        base = flat.ctypes.data + ((layer * P_ * nkv + kvh) * r) * 4
        ma = L.orc_arm_select(P(Rm), r, hd, P(q), ctypes.c_void_p(base), nkv, B, W, sink, pos, P(cand_a), P(ri_a))
        mb = R.sp_arm_select(P(Rm), r, hd, P(q), P(flat), layer, P_, nkv, kvh, B, W, sink, pos, P(cand_b), P(ri_b))
        straddled += _check_selection(ri_a, ma, ri_b, mb, cand_a, B, W, sink, pos)
        assert pk.shape == (P_, r)
    if not ties:
        assert straddled == 0


def test_recall_selection_tie_rule_on_zero_scores():
    """A zero query projects every candidate to the score +0.0 (and a score of
    -0.0 equals it): the top-k slots take the lowest candidate positions, the
    sinks and the window stay where they are."""
    R = _ref(); L = orc.lib()
    hd, r, nkv, P_ = 64, 16, 2, 200
    Rm = np.zeros(r * hd, np.int8); L.orc_arm_build_R(P(Rm), r, hd)
    rng = np.random.default_rng(3)
    flat = np.ascontiguousarray(rng.standard_normal((1, P_, nkv, r)).astype(np.float32))
    q = np.zeros(hd, np.float32)
    for B, W, sink, pos in ((40, 8, 4, 150), (64, 16, 0, 199), (20, 4, 2, 60)):
        cand_a = np.zeros(2 * P_, np.int32); ri_a = np.zeros(P_, np.int32)
        cand_b = np.zeros(2 * P_, np.int32); ri_b = np.zeros(P_, np.int32)
        ma = L.orc_arm_select(P(Rm), r, hd, P(q), P(flat), nkv, B, W, sink, pos, P(cand_a), P(ri_a))
        mb = R.sp_arm_select(P(Rm), r, hd, P(q), P(flat), 0, P_, nkv, 0, B, W, sink, pos, P(cand_b), P(ri_b))
        _, sk, hi, topk = _sel_geom(B, W, sink, pos)
        want = list(range(sk)) + list(range(sk, sk + topk)) + list(range(hi, pos + 1))
        assert ri_a[:ma].tolist() == want, (B, W, sink, pos)
        _check_selection(ri_a, ma, ri_b, mb, cand_a, B, W, sink, pos)
    # -0.0 and +0.0 are one score: a sidecar of negative zeros ties with positive ones
    z = np.zeros((1, P_, nkv, r), np.float32)
    z[0, ::2] = -0.0
    q1 = rng.standard_normal(hd).astype(np.float32)
    cand_a = np.zeros(2 * P_, np.int32); ri_a = np.zeros(P_, np.int32)
    ma = L.orc_arm_select(P(Rm), r, hd, P(q1), P(z), nkv, 40, 8, 4, 150, P(cand_a), P(ri_a))
    assert ri_a[:ma].tolist() == list(range(4)) + list(range(4, 32)) + list(range(143, 151))


@pytest.mark.parametrize("cfg", [(0, 64, 4, 16), (16, 8, 2, 16), (24, 4, 3, 8), (12, 4, 0, 32)])
def test_recall_decode_matches_reference_ppl(tmpdir_models, cfg):
    """Teacher-forced decode with the ARM recall router (the reference's
    qwen3_ppl_decode with SP_RECALL_B/W/SINK/R, core/forward/decode.c:740-790,
    :859-874): the oracle's float decode with the same recall settings gives
    the same perplexity to the last bit of the double -- every scored logit,
    every selected set and the order of every float sum agree."""
    from helpers import oracle_ppl
    R = _ref()
    B, W, sink, r = cfg
    for name in ("qwen3-tiny", "qwen3-g4"):
        spm, spt = model_files(tmpdir_models, name)
        o = orc.Oracle(spm, 64)
        toks = prompt(48, o.V)
        if B:
            o.set_recall(B, W, sink, r)
        mine = oracle_ppl(o, toks, 4)
        o.close()
        ref = ctypes.c_double()
        assert R.refh_ppl_recall(spm.encode(), spt.encode(), P(toks), len(toks), 4, B, W, sink, r, ctypes.byref(ref)) == 0
        assert mine.hex() == ref.value.hex(), (name, mine, ref.value)
