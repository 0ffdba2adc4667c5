"""Pinning the oracle's exact-mode attention and its rounding primitives.

The reference has no integer attention, so the exact-mode attention is a
build-defined spec (oracle/sp_oracle.c attn_head_exact):
  qi = rne(q 2^16); ip = <qi, ki> exact; score = (float)((double)ip / 2^32) * ascale
  (core/forward/decode.c:141-152 form); z = llround(score 2^14) (the softmax
  island's grid, core/exact_islands/exact_islands.c:82-97); e = exp_fixed((z - M)
  2^16) >> 8 (Q22); out = RNE(sum e vq / (S 2^16)) with an int128 V-sum.
What pins it here:
  * the island exp restated in Python is checked bit for bit against the softmax
    island (which tests/test_oracle.py pins to the compiled reference), so the
    weights below are the reference island's weights;
  * an exact-rational brute force of the spec (Python integers and Fractions,
    no int128 helper, no float division) equals the oracle bit for bit on random
    tiny heads, windowed and not, with V at the clamp bound;
  * closed forms independent of the spec's constants: one position gives V on
    the Q16 grid exactly; equal scores give the RNE of the mean V; a window of
    w positions equals the same attention over a slab holding only those rows;
  * RNE of an exact rational, including exact ties and subnormals, for the
    division primitive;
  * the V clamp at its bound and its count;
  * exact-mode logits against float mode (bit-identical to the compiled
    reference) on three architectures / head sizes for 40 steps: the same greedy
    argmax at every step and rel <= 5e-3 (the islands' Q16 input grid on the
    synthetic models' residual stream, rms ~0.02: 2^-17 / 0.02 ~ 4e-4 per norm;
    measured 1.2e-3 at most).
"""
import math
from fractions import Fraction

import numpy as np
import pytest

import orc
from helpers import model_files, prompt

P = orc.ptr

FB, ONE = 30, 1 << 30
LOG2E = 1549082005
EXPC = [1073741824, 744261118, 257941248, 59597083, 10327387, 1431680, 165394]


def exp2_frac(r):
    acc = EXPC[6]
    for k in range(5, -1, -1):
        acc = ((acc * r) >> FB) + EXPC[k]
    return acc


def exp_fixed(d):
    """e^(d / 2^30) in Q30 for d <= 0, the softmax island's exp."""
    g = -((d * LOG2E) >> FB)
    n = g >> FB
    r = g - (n << FB)
    if n >= 32:
        return 0
    return exp2_frac(ONE - r) >> (n + 1) if r else ONE >> n


def llround(x):
    """C llround of a double: round half away from zero."""
    x = float(x)
    a = math.floor(abs(x) + 0.5) if abs(x) < 2 ** 52 else abs(x)
    return int(a) if x >= 0 else -int(a)


def rne_f32(x):
    """The float32 nearest to the rational x, ties to even (subnormals, overflow)."""
    x = Fraction(x)
    if x == 0:
        return np.float32(0.0)
    sgn, a = (-1 if x < 0 else 1), abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = max(e - 23, -149)
    q = a / Fraction(2) ** ulp
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = Fraction(n) * Fraction(2) ** ulp
    if val >= Fraction(2) ** 128:
        return np.float32(sgn * np.inf)
    return np.float32(sgn * float(val))


def test_python_island_exp_is_the_reference_island():
    """p_i = e_i / S from the Python exp equals the softmax island bit for bit
    (the oracle's island is bit-identical to the compiled reference's)."""
    L = orc.lib()
    rng = np.random.default_rng(4)
    for trial in range(30):
        m = int(rng.integers(1, 300))
        z = (rng.standard_normal(m) * (0.5 + 6 * rng.random())).astype(np.float32)
        if trial % 3 == 0:
            z[rng.integers(0, m, max(1, m // 4))] = z[0]          # ties at the max
        p = np.zeros(m)
        L.orc_softmax_exact(P(z), m, P(p))
        zi = [llround(float(v) * 16384.0) for v in z]
        mx = max(zi)
        e = [exp_fixed(((v - mx) * ONE) >> 14) for v in zi]
        S = sum(e)
        ref = np.array([float(v) / float(S) for v in e])
        assert np.array_equal(p.view(np.uint64), ref.view(np.uint64)), trial


def attn_exact_py(q, K, V, pos, win, ascale):
    """The exact-mode attention of one head, evaluated with Python integers and
    one exact rational per output (K, V: int32 rows of this head)."""
    s0 = max(0, pos - win + 1) if win >= 0 else 0
    qi = [int(v) for v in np.rint(q.astype(np.float32) * np.float32(65536.0)).astype(np.int64)]
    z = {}
    for s in range(s0, pos + 1):
        ip = sum(a * int(b) for a, b in zip(qi, K[s]))
        sc = np.float32(np.float64(ip) / 4294967296.0) * np.float32(ascale)
        z[s] = llround(np.float64(sc) * 16384.0)
    M = max(z.values())
    e = {s: exp_fixed(((z[s] - M) * ONE) >> 14) >> 8 for s in z}
    S = sum(e.values())
    HD = len(qi)
    return np.array([rne_f32(Fraction(sum(e[s] * int(V[s][i]) for s in z), S * 65536)) for i in range(HD)],
                    np.float32)


def orc_attn(q, K, V, pos, win, ascale, kvh=0, nkv=1):
    HD = q.size
    out = np.zeros(HD, np.float32)
    Kc = np.ascontiguousarray(K, np.int32); Vc = np.ascontiguousarray(V, np.int32)
    orc.lib().orc_attn_head_exact(P(np.ascontiguousarray(q, np.float32)), P(Kc), P(Vc), pos, nkv * HD, kvh, HD,
                                  float(ascale), win, P(out))
    return out


def _head(rng, n, HD, kscale=3.0, vscale=2.0):
    q = (rng.standard_normal(HD) * 1.5).astype(np.float32)
    K = np.rint(rng.standard_normal((n, HD)) * kscale * 65536).astype(np.int32)
    V = np.rint(rng.standard_normal((n, HD)) * vscale * 65536).astype(np.int32)
    return q, K, V


@pytest.mark.parametrize("HD", [64, 128])
@pytest.mark.parametrize("win", [-1, 1, 7, 16])
def test_attn_exact_vs_rational_brute_force(HD, win):
    rng = np.random.default_rng(HD * 100 + win + 7)
    ascale = np.float32(1.0) / np.sqrt(np.float32(HD))
    for pos in (0, 1, 5, 23, 40):
        q, K, V = _head(rng, pos + 1, HD)
        if pos == 23:                                    # V at the clamp bound
            V[3, :5] = 8388607; V[7, 5:9] = -8388607
        got = orc_attn(q, K, V, pos, win, ascale)
        want = attn_exact_py(q, K, V, pos, win, ascale)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (HD, win, pos)


def test_attn_exact_reads_its_kv_head_of_a_grouped_slab():
    """kvh selects head kvh's HD columns of each KVD-wide slab row."""
    rng = np.random.default_rng(11)
    HD, nkv, pos = 64, 3, 12
    q = (rng.standard_normal(HD)).astype(np.float32)
    K = np.rint(rng.standard_normal((pos + 1, nkv * HD)) * 2 * 65536).astype(np.int32)
    V = np.rint(rng.standard_normal((pos + 1, nkv * HD)) * 65536).astype(np.int32)
    for kvh in range(nkv):
        got = orc_attn(q, K, V, pos, -1, 0.125, kvh=kvh, nkv=nkv)
        want = attn_exact_py(q, K[:, kvh * HD:(kvh + 1) * HD], V[:, kvh * HD:(kvh + 1) * HD], pos, -1, 0.125)
        assert np.array_equal(got, want), kvh


def test_attn_exact_closed_forms():
    rng = np.random.default_rng(3)
    HD = 64
    # one position (pos 0, or a window of 1): softmax of one element = V on the Q16 grid
    for pos, win in ((0, -1), (9, 1)):
        q, K, V = _head(rng, pos + 1, HD, vscale=50.0)
        out = orc_attn(q, K, V, pos, win, 0.125)
        assert np.array_equal(out, (V[pos].astype(np.float64) / 65536.0).astype(np.float32))
    # equal scores: every weight equal, out = RNE(mean V / 2^16)
    n = 13
    q, K, V = _head(rng, n, HD)
    K[:] = K[0]
    out = orc_attn(q, K, V, n - 1, -1, 0.125)
    for i in range(HD):
        assert out[i] == rne_f32(Fraction(int(V[:, i].astype(np.int64).sum()), n * 65536))
    # a window of w positions == the same attention over a slab of only those rows
    for w in (3, 8, 17):
        pos = 30
        q, K, V = _head(rng, pos + 1, HD)
        a = orc_attn(q, K, V, pos, w, 0.125)
        b = orc_attn(q, K[pos - w + 1:], V[pos - w + 1:], w - 1, -1, 0.125)
        c = orc_attn(q, K[pos - w + 1:], V[pos - w + 1:], w - 1, w + 5, 0.125)
        assert np.array_equal(a, b) and np.array_equal(a, c)
    # a dominant score: e^-(gap) underflows the Q22 weight, out = that row's V
    q = np.zeros(HD, np.float32); q[0] = 4.0
    K = np.zeros((6, HD), np.int32); V = np.rint(rng.standard_normal((6, HD)) * 65536).astype(np.int32)
    K[2, 0] = 40 * 65536                                  # score 40*4*0.125 = 20 above the rest
    out = orc_attn(q, K, V, 5, -1, 0.125)
    assert np.array_equal(out, (V[2].astype(np.float64) / 65536.0).astype(np.float32))


def _split(num):
    u = num & ((1 << 128) - 1)
    hi = u >> 64
    if hi >= 1 << 63:
        hi -= 1 << 64
    return hi, u & ((1 << 64) - 1)


def test_i128_div_to_float_is_rne_of_the_rational():
    L = orc.lib()
    rng = np.random.default_rng(5)
    cases = []
    for _ in range(3000):
        nb = int(rng.integers(1, 110)); db = int(rng.integers(1, 62))
        num = int(rng.integers(1, 1 << 62)) << max(0, nb - 62) | int(rng.integers(0, 1 << 31))
        num = num % (1 << nb) or 1
        den = int(rng.integers(1, 1 << 62)) % (1 << db) or 1
        cases.append((num if rng.random() < 0.5 else -num, den, int(rng.integers(0, 48))))
    # exact ties between two floats: (2m+1)/2 ulps, normal and subnormal; just above a tie
    for _ in range(400):
        m = int(rng.integers(1 << 23, 1 << 24)); D = int(rng.integers(1, 1 << 20)) | 1
        u = int(rng.integers(-20, 40)); k = int(rng.integers(21, 40))      # value = (2m+1) 2^(u-1)
        cases.append(((2 * m + 1) * D << (u - 1 + k), D, k))
        cases.append((-((2 * m + 1) * D << (u - 1 + k)), D, k))
        cases.append((((2 * m + 1) * D << (u - 1 + k)) + 1, D, k))
        ms = int(rng.integers(0, 1 << 23))                                  # subnormal tie at 2^-150
        cases.append(((2 * ms + 1) * D, D, 150))
    cases += [(1, 1, 150), (1, 1, 149), (3, 1, 151), (1, 3, 150), (-(1 << 100), 1, 0), ((1 << 127) - 1, 1, 0)]
    for num, den, k in cases:
        hi, lo = _split(num)
        got = np.float32(L.orc_i128_div_to_float(hi, lo, den, k))
        want = rne_f32(Fraction(num, den * (1 << k)))
        assert got.view(np.uint32) == want.view(np.uint32), (num, den, k)


def test_v_clamp_bound_and_count(tmpdir_models):
    L = orc.lib()
    import ctypes
    c = ctypes.c_int(0)
    lim = (2 ** 23 - 1) / 65536
    for v, q, cl in [(lim, 8388607, 0), (-lim, -8388607, 0), (128.0, 8388607, 1), (-128.0, -8388607, 1),
                     ((2 ** 23 - 0.5) / 65536, 8388607, 1), ((2 ** 23 - 1.5) / 65536, 8388606, 0),
                     (1e30, 8388607, 1), (0.5 / 65536, 0, 0), (1.5 / 65536, 2, 0)]:
        assert L.orc_vq_of(np.float32(v), ctypes.byref(c)) == q and c.value == cl, v
    spm, _ = model_files(tmpdir_models, "qwen3-tiny")
    o = orc.Oracle(spm, 32, orc.EXACT)
    for t in range(6):
        o.step(t)
    assert o.v_clamps() == 0                           # N(0, 0.02) weights: V far inside the bound
    o.close()


@pytest.mark.parametrize("name", ["qwen3-tiny", "gemma3-tiny", "gemma3-hd256"])
def test_exact_mode_tracks_float_mode(tmpdir_models, name):
    """Exact-mode logits against float-mode logits (float mode is the reference's
    arithmetic bit for bit) on the float mode's greedy trajectory: the same
    argmax at every step and rel <= 5e-3."""
    spm, _ = model_files(tmpdir_models, name)
    of, oe = orc.Oracle(spm, 128, orc.FLOAT), orc.Oracle(spm, 128, orc.EXACT)
    for t in prompt(24, of.V):
        lf, le = of.step(int(t)), oe.step(int(t))
    for k in range(40):
        r = float(np.abs(lf - le).max() / np.abs(lf).max())
        assert r <= 5e-3, (k, r)
        assert int(lf.argmax()) == int(le.argmax()), k
        t = int(lf.argmax())
        lf, le = of.step(t), oe.step(t)
    of.close(); oe.close()


@pytest.mark.parametrize("mode", [orc.FLOAT, orc.EXACT])
def test_oracle_threads_do_not_change_results(tmpdir_models, mode):
    """The row-parallel oracle (GEMV rows and attention heads over threads) gives
    bit-identical logits for any thread count."""
    spm, _ = model_files(tmpdir_models, "gemma3-hd256")
    L = orc.lib()
    saved = L.orc_threads()
    out = []
    for th in (1, 7):
        L.orc_set_threads(th)
        o = orc.Oracle(spm, 400, mode)
        for i, t in enumerate(prompt(300, o.V)):
            lg = o.step(int(t), i >= 297)
        out.append(lg)
        o.close()
    L.orc_set_threads(saved)
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
