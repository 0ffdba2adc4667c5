"""The drop-in boundary on the CPU: the restated ABI structs against the
reference's own headers, and the backend's model validation on a model built by
the reference's own bridge.

  * every field the backend reads from the model handle (qwen3_model,
    qwen3_config, qwen3_layer, gguf_tensor, sp_arena_tensor,
    sp_frob_packed_tensor) and every field of the section-6b table, the arch
    info and the session config sits at the same offset with the same size in
    include/sp_model_abi.h / include/sp_l1_abi.h as in include/sp/{model,gguf,
    arena,frobenius_lift,sp_l1}.h -- one probe compiled against each side
    (needs the reference headers; skipped without them);
  * a qwen3_model built by the compiled reference (oracle/_ref: its
    sp_model_load + sp_model_to_qwen3 / sp_model_to_gemma3,
    core/session/sp_model_bridge.c) passes sp_hipkv_check_model with the same
    figures as the model this library's bridge builds from the same file, and
    a short norm tensor -- which the reference bridge copies as it is -- is
    rejected by the backend; sp_hipkv_open on that model gets as far as the
    device probe (no GPU here).
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import orc
import spkv
from helpers import model_files

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INC = "/root/reference/include"

FIELDS = {
    "qwen3_model": ["gguf", "cfg", "token_embd", "output_norm", "output", "layers", "arena", "released",
                    "norm_src", "norm_buf", "n_norm"],
    "qwen3_config": ["arch", "n_layers", "n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_vocab",
                     "context_length", "sliding_window", "rope_freq_base", "rms_eps"],
    "qwen3_layer": ["attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "attn_q_norm", "attn_k_norm",
                    "post_attn_norm", "ffn_norm", "ffn_gate", "ffn_up", "ffn_down", "post_ffw_norm"],
    "gguf_tensor": ["name", "n_dims", "dims", "type", "offset", "n_elements", "nbytes"],
    "sp_arena_tensor": ["name", "pt"],
    "sp_frob_packed_tensor": ["rows", "cols", "row_prec", "row_scale", "row_off", "codes", "codes_bytes",
                              "alias_mask", "bscale", "bs_nblk"],
    "sp_kvdecode_dispatch_fn": ["open", "prefill", "decode_step", "rewind", "position", "close"],
    "sp_arch_info": ["arch_id", "vocab_size", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "head_dim",
                     "max_context", "swa_window", "rope_freq_base", "ffn_variant", "tied_embeddings", "n_ff",
                     "rms_eps", "preferred_precision"],
    "sp_session_config": ["max_context", "deterministic", "flags", "precision_override"],
}


def _probe(tmp_path, tag, includes, flags):
    lines = ['#include <stddef.h>', '#include <stdio.h>'] + [f'#include "{h}"' for h in includes]
    lines.append("int main(void) {")
    for st, fs in FIELDS.items():
        lines.append(f'    printf("{st} %zu\\n", sizeof({st}));')
        for f in fs:
            lines.append(f'    printf("{st}.{f} %zu %zu\\n", offsetof({st}, {f}), sizeof((({st} *)0)->{f}));')
    lines.append("    return 0;\n}")
    src = tmp_path / f"probe_{tag}.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / f"probe_{tag}"
    subprocess.run(["gcc", "-std=gnu11", "-w", *flags, "-o", str(exe), str(src)], check=True)
    return subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines()


def test_abi_offsets_match_reference_headers(tmp_path):
    if not os.path.isdir(REF_INC):
        pytest.skip("reference headers not present")
    ref = _probe(tmp_path, "ref", ["sp/sp_l1.h", "sp/model.h", "sp/gguf.h", "sp/arena.h", "sp/frobenius_lift.h"],
                 ["-I", REF_INC])
    ours = _probe(tmp_path, "ours", ["sp_l1_abi.h", "sp_model_abi.h"], ["-I", os.path.join(ROOT, "include")])
    assert len(ref) == len(ours) > 80
    for a, b in zip(ref, ours):
        assert a == b, (a, b)


def _ref_bridge():
    R = orc.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref (the compiled reference) not built")
    R.sp_model_load.restype = ctypes.c_int
    R.sp_model_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]
    R.sp_model_unload.argtypes = [ctypes.c_void_p]
    for f in ("sp_model_to_qwen3", "sp_model_to_gemma3"):
        getattr(R, f).restype = ctypes.c_void_p
        getattr(R, f).argtypes = [ctypes.c_void_p]
    R.qwen3_free.argtypes = [ctypes.c_void_p]
    R.sp_last_error.restype = ctypes.c_char_p
    return R


def _check(qm):
    out = np.zeros(8, np.int64)
    rc = spkv.kv().sp_hipkv_check_model(ctypes.c_void_p(qm), spkv.ptr(out))
    return rc, out


@pytest.mark.parametrize("name", ["qwen3-tiny", "gemma3-hd256", "qwen3-g4"])
def test_reference_bridge_model_passes_backend_validation(tmpdir_models, name):
    R = _ref_bridge()
    spm, spt = model_files(tmpdir_models, name)
    h = ctypes.c_void_p()
    assert R.sp_model_load(spm.encode(), spt.encode(), ctypes.byref(h)) == 0, R.sp_last_error()
    qm_ref = (R.sp_model_to_gemma3 if name.startswith("gemma3") else R.sp_model_to_qwen3)(h)
    assert qm_ref, R.sp_last_error()
    rc, ref_out = _check(qm_ref)
    assert rc == 0, spkv.last_error()
    m = spkv.Model(spm, spt); s = spkv.Session(m, 64)
    rc, our_out = _check(spkv.l1().sp_session_qwen3_model(s.h))
    assert rc == 0 and np.array_equal(ref_out, our_out)
    d = orc.Oracle(spm, 8)
    E, FF, NL, V = d.E, d.FF, d.NL, d.V
    QD, KVD = d.NH * d.HD, d.NKV * d.HD
    per_layer = (QD + 2 * KVD) * E + E * QD + 3 * E * FF
    mats = NL * per_layer + V * E * (1 if name != "qwen3-g4" else 2)
    assert our_out[0] == mats // 2 + mats // 32 * 2              # Q4B codes + f16 block scales
    assert list(our_out[2:7]) == [NL, E, V, FF, d.SW]
    d.close()
    if os.environ.get("HIP_VISIBLE_DEVICES") is None:
        try:
            import torch
            gpu = torch.cuda.is_available()
        except Exception:
            gpu = False
        if not gpu:
            hh = ctypes.c_void_p()
            assert spkv.kv().sp_hipkv_open(ctypes.c_void_p(qm_ref), 16, ctypes.byref(hh)) != 0
            assert "no HIP device" in spkv.last_error()          # validation passed, then the device probe
    R.qwen3_free(ctypes.c_void_p(qm_ref))
    R.sp_model_unload(h)
    s.close(); m.close()


def test_backend_rejects_short_norm_in_q4b_model(tmp_path, tmpdir_models):
    """A well-formed OK_Q4B model whose blk.0.attn_q_norm tensor is cut short
    (its table entry rewritten): the reference bridge copies a norm of any
    length (sp_model_bridge.c:160-170) and builds the model; the backend's
    validation names the tensor before anything reads past the short copy."""
    import struct
    R = _ref_bridge()
    spm, spt = model_files(tmpdir_models, "qwen3-tiny")
    b = bytearray(open(spm, "rb").read())
    n = struct.unpack_from("<I", b, 316)[0]
    for i in range(n):
        off = 512 + 256 * i
        if b[off:off + 80].rstrip(b"\0") == b"blk.0.attn_q_norm.weight":
            struct.pack_into("<Q", b, off + 88, 60)                     # dims[0]
            struct.pack_into("<Q", b, off + 160, 240)                   # size_bytes
            break
    else:
        pytest.fail("tensor not found")
    bad = tmp_path / "shortq.spm"
    bad.write_bytes(bytes(b))
    h = ctypes.c_void_p()
    assert R.sp_model_load(str(bad).encode(), spt.encode(), ctypes.byref(h)) == 0, R.sp_last_error()
    qm = R.sp_model_to_qwen3(h)
    assert qm, R.sp_last_error()
    rc, _ = _check(qm)
    assert rc != 0 and "attn_q_norm" in spkv.last_error() and "wrong length" in spkv.last_error()
    R.qwen3_free(ctypes.c_void_p(qm)); R.sp_model_unload(h)
