"""Writes tests/golden/reference_decode.json: known answers of the compiled
reference (oracle/_ref/libspref.so, built from the reference's own C sources
under /root/reference by oracle/ref.mk) on this repository's synthetic OK_Q4B
models, so that the oracle stays pinned where the compiled reference is absent
(a GPU host, a fresh checkout).

Recorded per decode case (float decode through the reference's own session:
core/session/sp_session.c sp_prefill_chunk :154-212 + sp_decode_step :725-770):
  * SHA-256 of the .spm / .spt files the synthetic writer produces (the writer is
    pinned with the decode);
  * the prompt (SplitMix64 seed 1, uniform in [0, vocab)), the greedy tokens fed
    to every decode step, and SHA-256 + argmax of every logits row (float32
    little-endian), plus the first 8 logits of the last row as exact hex floats;
  * cases: the tiny shapes of the tests (Qwen3, Gemma3 with clipping windows,
    an untied head, head_dim 256), the Spinor-63 K/V codec flags, and config 1
    (one Qwen3-0.6B layer, vocab 151936, 512-token prompt, 64 decode steps).
Recall: the reference's decode-path perplexity (core/forward/decode.c
qwen3_ppl_decode, through oracle/ref_harness.c refh_ppl_recall) with the ARM
recall knobs SP_RECALL_B/W/SINK/R, as the exact double (hex), also with
SP_RECALL_KVSEL=1 (recall_kvsel).
Recall generation: the reference's greedy decode (qwen3_generate_kv through
oracle/ref_harness.c refh_generate_recall) with the recall knobs, with and
without SP_RECALL_DECODE_ONLY=1 (dense prompt, router at the generated
positions), as the generated token sequence; B = 0 is the plain decode.
Also the reference's exact islands (core/exact_islands/exact_islands.c) on the
island test vectors and its Spinor-63 codec (core/vht2/spinor_block.c:128-149)
on seeded vectors, as SHA-256 of the outputs.

Run in the build container after `make -C oracle -f oracle/ref.mk`:
    python tests/golden/make_golden.py
"""
import ctypes
import hashlib
import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "shannon-prime-system_amd"), os.path.join(ROOT, "oracle"),
                os.path.join(ROOT, "tests")]
import orc  # noqa: E402
import spkv  # noqa: E402
from helpers import SMALL, SPINOR_KS, island_inputs, spinor_vectors  # noqa: E402

OUT = os.path.join(HERE, "reference_decode.json")
P = orc.ptr

# (model, max_context, n_prompt, n_gen, sp_session_config.flags)
CASES = [
    ("qwen3-tiny", 64, 24, 16, 0),
    ("gemma3-tiny", 64, 24, 16, 0),
    ("qwen3-g4", 64, 24, 16, 0),
    ("gemma3-hd256", 96, 48, 16, 0),
    ("qwen3-tiny", 64, 20, 8, spkv.SP_KV_SPINOR),
    ("gemma3-tiny", 64, 20, 8, spkv.SP_KV_SPINOR_REF),
    ("qwen3-0.6b-1layer", 1024, 512, 64, 0),
]


# (B, W, sink, r) of the recall cases; B = 0 is the plain decode path
RECALL = [(0, 64, 4, 16), (16, 8, 2, 16), (24, 4, 3, 8), (12, 4, 0, 32)]
# (B, W, sink, r, decode_only) of the recall generation cases (24-token prompt, 32 generated)
RECALL_GEN = [(0, 64, 4, 16, 0), (16, 8, 2, 16, 1), (12, 4, 0, 32, 1), (16, 8, 2, 16, 0), (24, 4, 3, 8, 0)]


def sha(b):
    return hashlib.sha256(b).hexdigest()


def model(d, name, max_context):
    prefix = os.path.join(d, f"{name}_c{max_context}")
    kw = dict(SMALL[name]) if name in SMALL else {}
    return spkv.write_model(prefix, shape=None if name in SMALL else name, seed=0, max_context=max_context, **kw)


def main():
    R = orc.ref_lib()
    if R is None:
        sys.exit("oracle/_ref/libspref.so is not built (make -C oracle -f oracle/ref.mk)")
    out = {"generator": "tests/golden/make_golden.py",
           "reference": "oracle/_ref/libspref.so (oracle/ref.mk over the reference's C sources)",
           "cases": []}
    with tempfile.TemporaryDirectory() as d:
        for name, ctx, n_prompt, n_gen, flags in CASES:
            t0 = time.time()
            spm, spt = model(d, name, ctx)
            V = int(SMALL[name]["vocab"]) if name in SMALL else spkv.SHAPES[name]["vocab"]
            pr = spkv.splitmix_tokens(n_prompt, V, seed=1)
            pre = np.zeros(V, np.float32)
            lg = np.zeros((n_gen, V), np.float32)
            fed = np.zeros(n_gen, np.int32)
            rc = R.refh_decode_flags(spm.encode(), spt.encode(), P(pr), n_prompt, n_gen, None, P(pre), P(lg),
                                     P(fed), flags)
            if rc:
                sys.exit(f"reference decode failed for {name}: {rc}")
            out["cases"].append({
                "model": name, "seed": 0, "max_context": ctx, "flags": flags,
                "spm_sha256": sha(open(spm, "rb").read()), "spt_sha256": sha(open(spt, "rb").read()),
                "prompt": {"generator": "splitmix64", "seed": 1, "n": n_prompt},
                "prefill_logits_sha256": sha(pre.tobytes()), "prefill_argmax": int(pre.argmax()),
                "fed": [int(t) for t in fed],
                "logits_sha256": [sha(r.tobytes()) for r in lg],
                "argmax": [int(r.argmax()) for r in lg],
                "last_logits_head": [float(v).hex() for v in lg[-1][:8]],
            })
            print(f"{name} flags={flags}: {time.time() - t0:.1f}s", file=sys.stderr)

    out["recall"] = []
    with tempfile.TemporaryDirectory() as d:
        for name in ("qwen3-tiny", "qwen3-g4"):
            spm, spt = model(d, name, 64)
            V = int(SMALL[name]["vocab"])
            toks = spkv.splitmix_tokens(48, V, seed=1)
            for B, W, sink, r in RECALL:
                ppl = ctypes.c_double()
                if R.refh_ppl_recall(spm.encode(), spt.encode(), P(toks), len(toks), 4, B, W, sink, r, ctypes.byref(ppl)):
                    sys.exit(f"reference recall decode failed for {name}")
                out["recall"].append({"model": name, "max_context": 64, "n": 48, "n_warm": 4, "prompt_seed": 1,
                                      "B": B, "W": W, "sink": sink, "r": r, "ppl_hex": ppl.value.hex()})

    out["recall_generate"] = []
    with tempfile.TemporaryDirectory() as d:
        for name in ("qwen3-tiny", "qwen3-g4"):
            spm, spt = model(d, name, 64)
            V = int(SMALL[name]["vocab"])
            for B, W, sink, r, dec_only in RECALL_GEN:
                n_prompt, n_gen = 24, 32
                seq = np.zeros(n_prompt + n_gen, np.int32)
                seq[:n_prompt] = spkv.splitmix_tokens(n_prompt, V, seed=1)
                if R.refh_generate_recall(spm.encode(), spt.encode(), P(seq), n_prompt, n_gen, B, W, sink, r,
                                          dec_only) != n_prompt + n_gen:
                    sys.exit(f"reference recall generation failed for {name}")
                out["recall_generate"].append({
                    "model": name, "max_context": 64, "n_prompt": n_prompt, "prompt_seed": 1, "B": B, "W": W,
                    "sink": sink, "r": r, "decode_only": dec_only, "generated": [int(t) for t in seq[n_prompt:]]})

    # SP_RECALL_KVSEL (one selection per kv head, group-centroid query)
    out["recall_kvsel"] = []
    out["recall_generate_kvsel"] = []
    R.refh_set_kvsel(1)
    with tempfile.TemporaryDirectory() as d:
        for name in ("qwen3-tiny", "qwen3-g4"):
            spm, spt = model(d, name, 64)
            V = int(SMALL[name]["vocab"])
            toks = spkv.splitmix_tokens(48, V, seed=1)
            for B, W, sink, r in RECALL[1:]:
                ppl = ctypes.c_double()
                if R.refh_ppl_recall(spm.encode(), spt.encode(), P(toks), len(toks), 4, B, W, sink, r, ctypes.byref(ppl)):
                    sys.exit(f"reference KVSEL recall decode failed for {name}")
                out["recall_kvsel"].append({"model": name, "max_context": 64, "n": 48, "n_warm": 4, "prompt_seed": 1,
                                            "B": B, "W": W, "sink": sink, "r": r, "ppl_hex": ppl.value.hex()})
            for B, W, sink, r, dec_only in RECALL_GEN[1:]:
                n_prompt, n_gen = 24, 32
                seq = np.zeros(n_prompt + n_gen, np.int32)
                seq[:n_prompt] = spkv.splitmix_tokens(n_prompt, V, seed=1)
                if R.refh_generate_recall(spm.encode(), spt.encode(), P(seq), n_prompt, n_gen, B, W, sink, r,
                                          dec_only) != n_prompt + n_gen:
                    sys.exit(f"reference KVSEL recall generation failed for {name}")
                out["recall_generate_kvsel"].append({
                    "model": name, "max_context": 64, "n_prompt": n_prompt, "prompt_seed": 1, "B": B, "W": W,
                    "sink": sink, "r": r, "decode_only": dec_only, "generated": [int(t) for t in seq[n_prompt:]]})
    R.refh_set_kvsel(0)

    x, w, z, g = island_inputs()
    a = np.zeros_like(x); R.sp_rmsnorm_exact(P(x), P(w), x.size, P(a))
    p = np.zeros(z.size); R.sp_softmax_exact(P(z), z.size, P(p))
    ge = np.zeros_like(g); R.sp_gelu_exact(P(g), g.size, P(ge))
    out["islands"] = {"inputs": "tests/helpers.py island_inputs()", "rmsnorm_sha256": sha(a.tobytes()),
                      "softmax_sha256": sha(p.tobytes()), "gelu_sha256": sha(ge.tobytes())}
    sp = {}
    for k in SPINOR_KS:
        enc, dec = hashlib.sha256(), hashlib.sha256()
        nb = orc.lib().orc_spinor_blocks_for(k)
        for x in spinor_vectors(k):
            b = np.zeros(63 * nb, np.uint8); R.sp_spinor_encode_vec(P(x), k, P(b))
            y = np.zeros(k, np.float32)
            if R.sp_spinor_decode_vec(P(b), k, P(y)):
                sys.exit("reference spinor decode failed")
            enc.update(b.tobytes()); dec.update(y.tobytes())
        sp[str(k)] = {"blocks_sha256": enc.hexdigest(), "decoded_sha256": dec.hexdigest()}
    out["spinor"] = {"inputs": "tests/helpers.py spinor_vectors(k)", "k": sp}
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {OUT}", file=sys.stderr)


if __name__ == "__main__":
    main()
