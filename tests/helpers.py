"""Shared test helpers: synthetic models on disk and small decode drivers."""
import os

import numpy as np

import spkv

SMALL = {
    # tiny shapes for fast parity: (qwen3) 2 layers; (gemma3) 7 layers so layer 5
    # is global and the others use a 16-token window that clips
    "qwen3-tiny": dict(arch_id=spkv.ARCH_QWEN3, n_layers=2, hidden=256, n_heads=4, n_kv_heads=2,
                       head_dim=64, n_ff=512, vocab=1000),
    "gemma3-tiny": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=7, hidden=256, n_heads=4, n_kv_heads=2,
                        head_dim=64, n_ff=512, vocab=1000, swa_window=16),
    "qwen3-hd128": dict(arch_id=spkv.ARCH_QWEN3, n_layers=2, hidden=512, n_heads=8, n_kv_heads=4,
                        head_dim=128, n_ff=1024, vocab=2048),
    "gemma3-hd256": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=6, hidden=512, n_heads=4, n_kv_heads=2,
                         head_dim=256, n_ff=1024, vocab=2048, swa_window=32),
    "qwen3-g4": dict(arch_id=spkv.ARCH_QWEN3, n_layers=2, hidden=512, n_heads=8, n_kv_heads=2,
                     head_dim=128, n_ff=1024, vocab=2048, untied=1),
    # wide rows: the GEMVs split their columns over workgroups (2-3 splits, the
    # last one ragged) and combine exact partials atomically
    "qwen3-wide": dict(arch_id=spkv.ARCH_QWEN3, n_layers=2, hidden=2304, n_heads=8, n_kv_heads=4,
                       head_dim=128, n_ff=4352, vocab=3000),
    "gemma3-wide": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=6, hidden=2304, n_heads=8, n_kv_heads=4,
                        head_dim=256, n_ff=4352, vocab=3000, swa_window=16),
    # windows over several 64-position chunks (the one-launch window attention)
    "gemma3-w200": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=6, hidden=512, n_heads=4, n_kv_heads=2,
                        head_dim=256, n_ff=1024, vocab=2048, swa_window=200),
    "gemma3-g4w130": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=6, hidden=512, n_heads=8, n_kv_heads=2,
                          head_dim=128, n_ff=1024, vocab=2048, swa_window=130),
    # the other head_dim x group instances of the one-launch window attention
    "gemma3-hd128w100": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=6, hidden=512, n_heads=4, n_kv_heads=2,
                             head_dim=128, n_ff=1024, vocab=2048, swa_window=100),
    "gemma3-g4hd256w150": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=6, hidden=512, n_heads=8, n_kv_heads=2,
                               head_dim=256, n_ff=1024, vocab=2048, swa_window=150),
    "gemma3-g4hd64w150": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=6, hidden=512, n_heads=8, n_kv_heads=2,
                              head_dim=64, n_ff=1024, vocab=2048, swa_window=150),
    # one-position window (a single chunk); a window over more than 32 chunks (the two-kernel path)
    "gemma3-w1": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=6, hidden=512, n_heads=4, n_kv_heads=2,
                      head_dim=64, n_ff=1024, vocab=2048, swa_window=1),
    "gemma3-w2100": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=6, hidden=512, n_heads=4, n_kv_heads=2,
                         head_dim=64, n_ff=1024, vocab=2048, swa_window=2100),
    # rows whose block scales span about 20 binary exponents: the GEMVs' int128
    # accumulation (and the per-token prefill: no batched GEMM).  Spread in every
    # matrix, the activations outgrow exact mode's 64-bit sums of squares (float
    # mode only); in the embedding/LM head, q, k, v and gate (SPREAD_EXACT) the
    # norms, the V clamp and the activation keep them in range.
    "qwen3-spread": dict(arch_id=spkv.ARCH_QWEN3, n_layers=2, hidden=256, n_heads=4, n_kv_heads=2,
                         head_dim=64, n_ff=512, vocab=1000, spread_rows=8),
    "gemma3-spread": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=7, hidden=256, n_heads=4, n_kv_heads=2,
                          head_dim=64, n_ff=512, vocab=1000, swa_window=16, spread_rows=8),
    "qwen3-spread-x": dict(arch_id=spkv.ARCH_QWEN3, n_layers=2, hidden=256, n_heads=4, n_kv_heads=2,
                           head_dim=64, n_ff=512, vocab=1000, spread_rows=8, spread_mask=0x5D),
    "gemma3-spread-x": dict(arch_id=spkv.ARCH_GEMMA3, n_layers=7, hidden=256, n_heads=4, n_kv_heads=2,
                            head_dim=64, n_ff=512, vocab=1000, swa_window=16, spread_rows=8, spread_mask=0x5D),
}


def model_files(dirpath, name, max_context=512, seed=0):
    prefix = os.path.join(str(dirpath), f"{name}_s{seed}_c{max_context}")
    if not os.path.exists(prefix + ".spm"):
        kw = dict(SMALL[name]) if name in SMALL else {}
        shape = None if name in SMALL else name
        spkv.write_model(prefix, shape=shape, seed=seed, max_context=max_context, **kw)
    return prefix + ".spm", prefix + ".spt"


def prompt(n, vocab, seed=1):
    """Seeded uniform prompt tokens: SplitMix64 (seed) mod vocab, the generator
    of the benchmark configurations' prompts."""
    return spkv.splitmix_tokens(n, vocab, seed=seed)


def lcg_uniform(state, rng):
    """core/exact_islands/exact_islands_test.c:196-201 LCG: uniform in [-rng, rng]."""
    state[0] = (state[0] * 6364136223846793005 + 1442695040888963407) & ((1 << 64) - 1)
    u = (state[0] >> 11) / float(1 << 53)
    return (2.0 * u - 1.0) * rng


def island_inputs():
    """The island test vectors: x, w (RMSNorm, E = 3840), z (softmax, 256), g (GELU, 512)."""
    E, M, G = 3840, 256, 512
    st = [1]
    x = np.zeros(E, np.float32); w = np.zeros(E, np.float32)
    for i in range(E):
        x[i] = lcg_uniform(st, 2.0); w[i] = 1.0 + lcg_uniform(st, 0.1)
    st = [7]; z = np.array([lcg_uniform(st, 8.0) for _ in range(M)], np.float32)
    st = [11]; g = np.array([lcg_uniform(st, 3.0) for _ in range(G)], np.float32)
    return x, w, z, g


SPINOR_KS = [1, 7, 43, 55, 56, 64, 128, 200, 256, 512]


def spinor_vectors(k, trials=40):
    """Seeded Spinor-63 codec inputs of length k: Gaussian at magnitudes 1e-6..1e3,
    some with zeros, all-zero, and exact half-step ties."""
    rng = np.random.default_rng(k)
    out = []
    for trial in range(trials):
        x = (rng.standard_normal(k) * (10.0 ** rng.integers(-6, 4))).astype(np.float32)
        if trial % 5 == 1: x[rng.integers(0, k, max(1, k // 3))] = 0.0
        if trial % 5 == 2: x[:] = 0.0
        if trial % 5 == 3:
            x = (rng.integers(-254, 255, k).astype(np.float32) / 2.0) * np.float32(0.125)
        out.append(x)
    return out


def oracle_ppl(o, toks, n_warm):
    """The decode-path perplexity of core/forward/decode.c qwen3_ppl_decode
    (:859-874) from an oracle session's logits: for positions pos in
    [n_warm, n-2], -log softmax(logits_pos)[toks[pos+1]] with the max taken in
    float, the exp-sum sequential in double (libm exp / log), then
    exp(mean).  n_warm is clamped to [1, n-2] as the reference does."""
    import math
    n = len(toks)
    n_warm = min(max(n_warm, 1), n - 2)
    nll, ns = 0.0, 0
    for pos, t in enumerate(toks):
        want = pos + 1 < n and pos >= n_warm
        lg = o.step(int(t), want)
        if not want:
            continue
        tgt = int(toks[pos + 1])
        m = lg[0]
        for j in range(1, len(lg)):
            if lg[j] > m:
                m = lg[j]
        maxl = float(m)
        se = 0.0
        for v in lg.tolist():
            se += math.exp(v - maxl)
        nll += -(float(lg[tgt]) - maxl - math.log(se))
        ns += 1
    return math.exp(nll / ns)
