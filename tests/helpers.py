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
}


def model_files(dirpath, name, max_context=512, seed=0):
    prefix = os.path.join(str(dirpath), f"{name}_s{seed}_c{max_context}")
    if not os.path.exists(prefix + ".spm"):
        kw = dict(SMALL[name]) if name in SMALL else {}
        shape = None if name in SMALL else name
        spkv.write_model(prefix, shape=shape, seed=seed, max_context=max_context, **kw)
    return prefix + ".spm", prefix + ".spt"


def prompt(n, vocab, seed=1):
    """Seeded uniform prompt tokens (SplitMix-free numpy generator; test-only)."""
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.int32)
