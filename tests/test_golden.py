"""The oracle against the compiled reference's known answers, without the
compiled reference: tests/golden/reference_decode.json (written by
tests/golden/make_golden.py from oracle/_ref, the reference built from its own
C sources).

  * the synthetic OK_Q4B writer reproduces the recorded .spm / .spt SHA-256s;
  * oracle float mode reproduces the reference's logits bit for bit (SHA-256 of
    every row) and its greedy tokens: prefill logits and every decode step
    (with the Spinor-63 K/V flags: every decode step; the reference's prefill
    logits come from a full forward that keeps no K/V and carries no codec),
    including config 1 (one Qwen3-0.6B layer, vocab 151936, 512 + 64);
  * the exact islands and the Spinor-63 codec reproduce the reference's output
    hashes on the shared test vectors;
  * the oracle's decode with the ARM recall router reproduces the reference's
    decode-path perplexity (qwen3_ppl_decode with SP_RECALL_B/W/SINK/R) as the
    exact double, and its greedy sequences (qwen3_generate_kv) with the router
    on the whole sequence and with SP_RECALL_DECODE_ONLY=1 (dense prompt steps,
    orc_set_recall_dense); the recall sequences differ from the plain one, so
    the pin sees the router.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import orc
import spkv
from helpers import SMALL, SPINOR_KS, island_inputs, oracle_ppl, spinor_vectors

GOLDEN = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_decode.json")))
P = orc.ptr


def sha(b):
    return hashlib.sha256(b).hexdigest()


def _files(tmp_models, case):
    name, ctx = case["model"], case["max_context"]
    prefix = os.path.join(str(tmp_models), f"golden_{name}_c{ctx}")
    if not os.path.exists(prefix + ".spm"):
        kw = dict(SMALL[name]) if name in SMALL else {}
        spkv.write_model(prefix, shape=None if name in SMALL else name, seed=case["seed"], max_context=ctx, **kw)
    return prefix + ".spm", prefix + ".spt"


def _ids(c):
    return f'{c["model"]}-flags{c["flags"]}'


@pytest.mark.parametrize("case", GOLDEN["cases"], ids=_ids)
def test_oracle_float_decode_matches_reference_golden(tmpdir_models, case):
    spm, spt = _files(tmpdir_models, case)
    assert sha(open(spm, "rb").read()) == case["spm_sha256"], "synthetic writer drifted"
    assert sha(open(spt, "rb").read()) == case["spt_sha256"]
    o = orc.Oracle(spm, case["max_context"], orc.FLOAT, kv_flags=case["flags"])
    pr = spkv.splitmix_tokens(case["prompt"]["n"], o.V, seed=case["prompt"]["seed"])
    for i, t in enumerate(pr):
        lg = o.step(int(t), i == len(pr) - 1)
    if not case["flags"]:
        assert sha(lg.tobytes()) == case["prefill_logits_sha256"], "prefill logits"
    assert int(lg.argmax()) == case["prefill_argmax"] or case["flags"]
    for k, t in enumerate(case["fed"]):
        lg = o.step(t)
        assert sha(lg.tobytes()) == case["logits_sha256"][k], f"decode step {k}"
        assert int(lg.argmax()) == case["argmax"][k]
    assert [float(v).hex() for v in lg[:8]] == case["last_logits_head"]
    o.close()


def test_islands_match_reference_golden():
    L = orc.lib()
    x, w, z, g = island_inputs()
    a = np.zeros_like(x); L.orc_rmsnorm_exact(P(x), P(w), x.size, P(a))
    p = np.zeros(z.size); L.orc_softmax_exact(P(z), z.size, P(p))
    ge = np.zeros_like(g); L.orc_gelu_exact(P(g), g.size, P(ge))
    gi = GOLDEN["islands"]
    assert sha(a.tobytes()) == gi["rmsnorm_sha256"]
    assert sha(p.tobytes()) == gi["softmax_sha256"]
    assert sha(ge.tobytes()) == gi["gelu_sha256"]


@pytest.mark.parametrize("k", SPINOR_KS)
def test_spinor_codec_matches_reference_golden(k):
    L = orc.lib()
    enc, dec = hashlib.sha256(), hashlib.sha256()
    nb = L.orc_spinor_blocks_for(k)
    for x in spinor_vectors(k):
        b = np.zeros(63 * nb, np.uint8); L.orc_spinor_encode_vec(P(x), k, P(b))
        y = np.zeros(k, np.float32)
        assert L.orc_spinor_decode_vec(P(b), k, P(y)) == 0
        enc.update(b.tobytes()); dec.update(y.tobytes())
    want = GOLDEN["spinor"]["k"][str(k)]
    assert enc.hexdigest() == want["blocks_sha256"] and dec.hexdigest() == want["decoded_sha256"]


@pytest.mark.parametrize("case", GOLDEN["recall"], ids=lambda c: f'{c["model"]}-B{c["B"]}-W{c["W"]}-s{c["sink"]}-r{c["r"]}')
def test_oracle_recall_decode_matches_reference_golden(tmpdir_models, case):
    c = dict(case, seed=0, flags=0)
    spm, _ = _files(tmpdir_models, c)
    o = orc.Oracle(spm, case["max_context"])
    if case["B"]:
        o.set_recall(case["B"], case["W"], case["sink"], case["r"])
    toks = spkv.splitmix_tokens(case["n"], o.V, seed=case["prompt_seed"])
    assert oracle_ppl(o, toks, case["n_warm"]).hex() == case["ppl_hex"]
    o.close()


@pytest.mark.parametrize("case", GOLDEN["recall_generate"],
                         ids=lambda c: f'{c["model"]}-B{c["B"]}-W{c["W"]}-s{c["sink"]}-r{c["r"]}-d{c["decode_only"]}')
def test_oracle_recall_generation_matches_reference_golden(tmpdir_models, case):
    c = dict(case, seed=0, flags=0)
    spm, _ = _files(tmpdir_models, c)
    o = orc.Oracle(spm, case["max_context"])
    if case["B"]:
        o.set_recall(case["B"], case["W"], case["sink"], case["r"])
    o.set_recall_dense(case["decode_only"])
    pr = spkv.splitmix_tokens(case["n_prompt"], o.V, seed=case["prompt_seed"])
    for t in pr:
        lg = o.step(int(t))
    o.set_recall_dense(0)
    out = []
    for k in range(len(case["generated"])):
        out.append(int(lg.argmax()))
        if k + 1 < len(case["generated"]):
            lg = o.step(out[-1])
    assert out == case["generated"]
    o.close()


@pytest.mark.parametrize("case", GOLDEN["recall_kvsel"],
                         ids=lambda c: f'{c["model"]}-B{c["B"]}-W{c["W"]}-s{c["sink"]}-r{c["r"]}')
def test_oracle_recall_kvsel_decode_matches_reference_golden(tmpdir_models, case):
    """SP_RECALL_KVSEL: one selection per kv head from the group-centroid query
    (core/forward/decode.c:53-63, :738-757); the reference's perplexity as the
    exact double."""
    c = dict(case, seed=0, flags=0)
    spm, _ = _files(tmpdir_models, c)
    o = orc.Oracle(spm, case["max_context"])
    o.set_recall(case["B"], case["W"], case["sink"], case["r"])
    o.set_recall_kvsel(True)
    toks = spkv.splitmix_tokens(case["n"], o.V, seed=case["prompt_seed"])
    assert oracle_ppl(o, toks, case["n_warm"]).hex() == case["ppl_hex"]
    o.close()


@pytest.mark.parametrize("case", GOLDEN["recall_generate_kvsel"],
                         ids=lambda c: f'{c["model"]}-B{c["B"]}-W{c["W"]}-s{c["sink"]}-r{c["r"]}-d{c["decode_only"]}')
def test_oracle_recall_kvsel_generation_matches_reference_golden(tmpdir_models, case):
    c = dict(case, seed=0, flags=0)
    spm, _ = _files(tmpdir_models, c)
    o = orc.Oracle(spm, case["max_context"])
    o.set_recall(case["B"], case["W"], case["sink"], case["r"])
    o.set_recall_kvsel(True)
    o.set_recall_dense(case["decode_only"])
    pr = spkv.splitmix_tokens(case["n_prompt"], o.V, seed=case["prompt_seed"])
    for t in pr:
        lg = o.step(int(t))
    o.set_recall_dense(0)
    out = []
    for k in range(len(case["generated"])):
        out.append(int(lg.argmax()))
        if k + 1 < len(case["generated"]):
            lg = o.step(out[-1])
    assert out == case["generated"]
    o.close()


def test_kvsel_goldens_differ_from_per_head_selection():
    """KVSEL changes the recalled sets: its perplexities differ from the
    per-q-head selection's for every case."""
    per_head = {(c["model"], c["B"], c["W"], c["sink"], c["r"]): c["ppl_hex"] for c in GOLDEN["recall"]}
    for c in GOLDEN["recall_kvsel"]:
        assert c["ppl_hex"] != per_head[(c["model"], c["B"], c["W"], c["sink"], c["r"])], c


def test_recall_generation_goldens_see_the_router():
    plain = {c["model"]: c["generated"] for c in GOLDEN["recall_generate"] if c["B"] == 0}
    for c in GOLDEN["recall_generate"]:
        if c["B"]:
            assert c["generated"] != plain[c["model"]], c
