"""GPU parity at configuration C5's real shape (exact mode, through the C ABI):

  C5  Gemma-3-12B at 131072 positions: prefill, then greedy runs of 16 steps,
      each followed by a U{1..64} rewind (SplitMix64 seed 4), window layers on
      a ring sized for the drift (sp_hipkv_set_max_rewind); after the last
      rewind the oracle, given the device K/V (window layers read back from the
      ring), reproduces the next step's logits and K/V bit for bit.
"""
import numpy as np
import pytest

import orc
import spkv
from helpers import prompt
from test_gpu_configs import check_kv_at, load_kv, same_bits

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


def test_config5_gemma3_12b_128k_rewinds(tmp_path):
    ctx, runs, every, rmax = 131072, 4, 16, 64
    rw = (1 + spkv.splitmix_u64(runs, 4) % np.uint64(rmax)).astype(np.int64)
    pmax = ctx + runs * every + 64
    spm, spt = spkv.write_model(str(tmp_path / "gemma3-12b"), shape="gemma3-12b", seed=0, max_context=pmax,
                                threads=16)
    m = spkv.Model(spm, spt); s = spkv.Session(m, pmax)
    s.attach(pmax, exact=True)
    be = spkv.Backend.wrap(s.backend_handle())
    # the ring must hold every position a rewind returns to (rewinds count from
    # the highest position written, drifting up to rmax per run)
    spkv.check(spkv.kv().sp_hipkv_set_max_rewind(be.h, (runs + 1) * rmax), "sp_hipkv_set_max_rewind")
    V = 262144
    pr = prompt(ctx, V)
    lg = np.zeros(V, np.float32)
    for c0 in range(0, ctx, 16384):
        spkv.check(s.prefill(pr[c0:c0 + 16384], lg), "sp_prefill_chunk")
        print(f"[C5] prefill {c0 + 16384}/{ctx}", flush=True)
    tok = int(lg.argmax())
    for i in range(runs):
        toks, _ = be.greedy(tok, every)
        assert be.rewind(int(rw[i])) == 0
        tok = int(toks[-1])
    p = be.position()
    o = orc.Oracle(spm, pmax, orc.EXACT)
    load_kv(o, be, 0, p)
    ol = o.step(tok)
    be.decode(tok, lg)
    assert same_bits(lg, ol), "the step after the last rewind"
    check_kv_at(o, be, p)
    o.close(); s.close(); m.close()
