"""Models whose rows have block scales spread over more binary exponents than
the GEMV's int64 accumulation holds: the backend's host validation
(sp_hipkv_check_model, no device call) marks them wide -- their GEMVs take the
int128 path and prefill runs token by token -- and plain random-init models not."""
import ctypes

import numpy as np
import pytest

import spkv
from helpers import model_files


@pytest.mark.parametrize("name,wide", [("qwen3-tiny", 0), ("gemma3-tiny", 0), ("qwen3-spread", 1), ("gemma3-spread", 1),
                                       ("qwen3-spread-x", 1), ("gemma3-spread-x", 1)])
def test_spread_rows_mark_the_model_wide(tmpdir_models, name, wide):
    spm, spt = model_files(tmpdir_models, name)
    m = spkv.Model(spm, spt)
    s = spkv.Session(m, 64)
    out = np.zeros(8, np.int64)
    qm = spkv.l1().sp_session_qwen3_model(s.h)
    assert spkv.kv().sp_hipkv_check_model(ctypes.c_void_p(qm), spkv.ptr(out)) == 0, spkv.last_error()
    assert out[7] == wide
    s.close(); m.close()
