#!/usr/bin/env python3
"""bench.py -- section-6b kvdecode throughput on one MI355X.

Workload (default): Gemma-3-12B shape (48 layers, hidden 3840, 16q/8kv heads,
head_dim 256, FFN 15360, vocab 262144, 5:1 window/global with a 1024 window),
random-init OK_Q4B weights (seed 0), a 32768-token seeded uniform prompt
(seed 1) prefilled through sp_prefill_chunk, then greedy decode steps.  One
"step" = one token through the whole model incl. the LM head and argmax.

`value` is decode tokens/s with weights and KV resident in HBM (device-resident
greedy loop: the argmax feeds the next token on the GPU).  The rate of the full
ABI path (sp_decode_step with the 1 MiB logits row copied to host memory each
step) is reported beside it as `pcie_inclusive_tokens_per_s`.

The CPU baseline is the oracle (scalar C restatement of the reference decode)
timed for one decode step at the same context on the host, with its KV state
loaded from the device.
"""
import argparse
import json
import os
import platform
import shutil
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "shannon-prime-system_amd"))
from spkv import splitmix_tokens, splitmix_u64  # noqa: E402  (seeded synthetic inputs)

METRIC = "kvdecode tokens/s + KV-read HBM GB/s (% of peak), Gemma-12B shape 32k ctx"
PEAK_GBS = 8000.0
GEMV_CLASSES = ("qkv_gemv_q4b", "o_gemv_q4b", "gate_up_gemv_q4b", "down_gemv_q4b", "lm_head_gemv_q4b")
CLASSES = ["qkv_gemv_q4b", "o_gemv_q4b", "gate_up_gemv_q4b", "down_gemv_q4b", "lm_head_gemv_q4b",
           "gqa_decode_attn_global", "gqa_decode_attn_window", "qk_norm_rope_append", "embed_rope_argmax"]
# the rocprofv3 kernel names of each class's launches (exact mode; float mode in brackets)
KERNEL_NAMES = {
    "qkv_gemv_q4b": ["kvd::k_gemv<2, false, false>", "kvd::k_gemv<1, false, false> (layer 0)"],
    "o_gemv_q4b": ["kvd::k_gemv<0, false, false>"],
    "gate_up_gemv_q4b": ["kvd::k_gemv<2, true, false>"],
    "down_gemv_q4b": ["kvd::k_gemv<0, false, false>"],
    "lm_head_gemv_q4b": ["kvd::k_gemv<2, false, false>"],
    "gqa_decode_attn_global": ["kvd::k_attn_exact_scores<EPL, G, false, true, 8> + kvd::k_attn_exact_vsum<EPL, G, false, 12>",
                               "[kvd::k_qk_prep<false> + kvd::k_attn_float<EPL, G, false, SPINOR>]"],
    "gqa_decode_attn_window": ["kvd::k_attn_exact_window<EPL, G>",
                               "[kvd::k_qk_prep<false> + kvd::k_attn_float<EPL, G, false, SPINOR>]"],
    # float mode only: exact-mode decode prepares the heads inside the score pass
    "qk_norm_rope_append": ["[kvd::k_qk_prep<false>]"],
    "embed_rope_argmax": ["kvd::k_embed_rope", "kvd::k_argmax"],
}
# the batched multi-session decode's global attention (Qwen3-8B shape: head_dim
# 128, 4 q heads per kv head), exact and float mode
BATCH_ATTN_NAMES = {True: "kvd::k_attn_exact_scores<2, 4, true, false, 8> + kvd::k_attn_exact_vsum<2, 4, true, 12>",
                    False: "kvd::k_attn_float<2, 4, true, false>"}
# a routed global layer's launches (--recall), exact and float mode
RECALL_NAMES = {True: "kvd::k_recall_score<RT> + kvd::k_recall_select + kvd::k_recall_scores<EPL, true>"
                      " + kvd::k_recall_vsum_exact<EPL>",
                False: "kvd::k_recall_score<RT> + kvd::k_recall_select + kvd::k_recall_scores<EPL, false>"
                       " + kvd::k_recall_vsum_float<EPL>"}
# committed rocprofv3 --pmc summaries (FETCH_SIZE / WRITE_SIZE per dispatch) of the
# decode kernels at this model shape and context, with the 1 GiB calibration copy they hold
PMC_SUMMARY = os.path.join(ROOT, "profiles", "gemma3-12b_32k_decode_pmc_fetch_write.txt")
# committed rocprofv3 --kernel-trace --stats summary of this workload (kernel durations)
KERNEL_STATS = os.path.join(ROOT, "profiles", "gemma3-12b_32k_kernel_stats.csv.txt")


def pmc_traffic(kernel, path=PMC_SUMMARY):
    """HBM bytes per launch of `kernel` from the committed PMC summary: FETCH_SIZE
    and WRITE_SIZE means, each scaled by what the counter reads for the plain
    1 GiB device copy in the same run.  None when the summary lacks it."""
    try:
        lines = open(path).read().splitlines()
    except OSError:
        return None
    sec, val, cal = None, {}, {}
    for ln in lines:
        if ln.startswith("# FETCH_SIZE"):
            sec = "FETCH_SIZE"
        elif ln.startswith("# WRITE_SIZE"):
            sec = "WRITE_SIZE"
        elif sec and not ln.startswith("#") and ln.strip() and not ln.startswith("kernel"):
            parts = ln.split()
            name = " ".join(parts[:-3])
            mean, mx = float(parts[-2]), float(parts[-1])
            if "copyBuffer" in name:                  # the 1 GiB copy: the largest copy dispatch
                cal[sec] = max(cal.get(sec, 0.0), mx)
            if name.startswith("void " + kernel + "(") or name.startswith(kernel + "("):
                val[sec] = mean
    if len(val) < 2 or len(cal) < 2 or not cal["FETCH_SIZE"] or not cal["WRITE_SIZE"]:
        return None
    gib_kib = 1024.0 * 1024.0
    f = val["FETCH_SIZE"] * gib_kib / cal["FETCH_SIZE"]
    w = val["WRITE_SIZE"] * gib_kib / cal["WRITE_SIZE"]
    return {"bytes": (f + w) * 1024.0, "fetch_scale": round(gib_kib / cal["FETCH_SIZE"], 4),
            "write_scale": round(gib_kib / cal["WRITE_SIZE"], 4), "source": os.path.relpath(path, ROOT)}


def rocprof_fields(names, launch_bytes, headline):
    """The dominant kernel's average duration in the committed rocprof summary of
    this workload (the headline workload only) and the roofline fraction it gives."""
    us = rocprof_avg_us(names[0]) if headline and len(names) == 1 else None
    if not us:
        return {"rocprof_avg_us": None}
    gbs = launch_bytes / (us * 1e-6) / 1e9
    return {"rocprof_avg_us": round(us, 3), "rocprof_achieved": round(gbs, 1),
            "rocprof_frac": round(gbs / PEAK_GBS, 4), "rocprof_source": os.path.relpath(KERNEL_STATS, ROOT)}


def rocprof_avg_us(kernel, path=KERNEL_STATS):
    """Average duration (us) of `kernel` in the committed rocprofv3 kernel-stats
    summary, or None."""
    import csv
    try:
        rows = [ln for ln in open(path).read().splitlines() if ln and not ln.startswith("#")]
    except OSError:
        return None
    for r in csv.DictReader(rows):
        if r["Name"].startswith("void " + kernel + "(") or r["Name"].startswith(kernel + "("):
            return float(r["AverageNs"]) / 1e3
    return None


WORKLOADS = {
    "gemma3-12b-32k": dict(shape="gemma3-12b", ctx=32768),
    "qwen3-0.6b-4k": dict(shape="qwen3-0.6b", ctx=4096),
    # 131072-token prefill, then greedy decode with a rewind of 1-64 tokens
    # (seed 4) after every 16 steps; window layers keep a ring of W + 64
    "gemma3-12b-128k": dict(shape="gemma3-12b", ctx=131072, rewind_every=16, rewind_max=64),
    # 64 concurrent sessions, contexts uniform in [1024, 16384] (seed 2); every
    # step clones each session (sp_session_clone), rewinds the clone 0-4 tokens
    # (seed 3) and decodes all 64 in one batched call (spx_decode_batch)
    "qwen3-8b-batch64": dict(shape="qwen3-8b", ctx=16384, sessions=64, ctx_lo=1024),
}
BATCH_METRIC = "batched multi-session kvdecode tokens/s (aggregate over sessions), Qwen3-8B shape, 64 sessions"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="gemma3-12b-32k", choices=sorted(WORKLOADS))
    ap.add_argument("--mode", default="exact", choices=["exact", "float"])
    ap.add_argument("--kv", default="plain", choices=["plain", "spinor"],
                    help="session K/V codec: spinor = SP_KV_SPINOR (int8 chunk codes in float mode)")
    ap.add_argument("--cpu-steps", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-steps", type=int, default=8)
    ap.add_argument("--workdir", default=None)
    ap.add_argument("--ctx", type=int, default=None, help="override the workload's prefill length")
    ap.add_argument("--no-graph", action="store_true", help="plain kernel launches instead of one HIP graph per step")
    ap.add_argument("--no-batch-prefill", action="store_true", help="prefill one decode step per token")
    ap.add_argument("--recall", default=None, metavar="B,W,SINK,R",
                    help="ARM recall on the global layers (sp_hipkv_set_recall): budget, window, sinks, projection rows")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="run one device-to-device copy of this many MiB first (HBM counter calibration)")
    ap.add_argument("--kv-import", action="store_true",
                    help="build the context by writing synthetic K/V rows (sp_hipkv_write_kv) instead of the "
                         "prefill: the decode reads the same bytes, and a counter run sees a few dispatches "
                         "before it instead of the prefill's ~150k")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("CSV", "COUNTER"), default=None,
                    help="summarize a rocprofv3 --pmc counter_collection.csv per kernel and exit")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "sharding the path over several GPUs is designed but not built or measured", file=sys.stderr)
        sys.exit(2)

    import spkv
    wl = WORKLOADS[args.workload]
    if wl.get("sessions"):
        return run_sessions(args, wl)
    shape = dict(spkv.SHAPES[wl["shape"]])
    ctx, V, E = (args.ctx or wl["ctx"]), shape["vocab"], shape["hidden"]
    pmax = ctx + args.warmup + args.steps + args.kernel_steps + 64
    exact = args.mode == "exact"
    work = args.workdir or tempfile.mkdtemp(prefix="spkv_bench_", dir=os.environ.get("TMPDIR", "/tmp"))
    prefix = os.path.join(work, wl["shape"])
    t0 = time.time()
    threads = min(16, os.cpu_count() or 1)
    spm, spt = spkv.write_model(prefix, shape=wl["shape"], seed=0, max_context=pmax, threads=threads)
    log(f"model written {os.path.getsize(spm)/1e9:.2f} GB in {time.time()-t0:.1f}s ({threads} threads)")
    try:
        model = spkv.Model(spm, spt)
        sess = spkv.Session(model, pmax, flags=spkv.SP_KV_SPINOR if args.kv == "spinor" else 0)
        t0 = time.time()
        sess.attach(pmax, exact=exact)
        log(f"backend attached (upload) in {time.time()-t0:.1f}s, mode={args.mode}")
        be = spkv.Backend.wrap(sess.backend_handle())
        if args.no_graph:
            spkv.check(spkv.kv().sp_hipkv_set_graph(be.h, 0), "sp_hipkv_set_graph")
        if args.no_batch_prefill:
            spkv.check(spkv.kv().sp_hipkv_set_batch_prefill(be.h, 0), "sp_hipkv_set_batch_prefill")
        recall = tuple(int(x) for x in args.recall.split(",")) if args.recall else None
        if recall:
            be.set_recall(*recall)
        every = wl.get("rewind_every", 0)
        if every:
            # the window ring must hold every position a rewind can return to:
            # rewinds are measured from the highest position ever written, and
            # 1..rewind_max back every `every` steps can drift that far per run
            max_rewind = (args.steps // every + 1) * wl["rewind_max"]
            spkv.check(spkv.kv().sp_hipkv_set_max_rewind(be.h, max_rewind), "sp_hipkv_set_max_rewind")
        info = be.info()

        if args.calib_copy_mib:
            calib_copy(args.calib_copy_mib << 20)

        prompt = splitmix_tokens(ctx, V, seed=1)
        logits = np.zeros(V, np.float32)
        t0 = time.time()
        if args.kv_import:
            import_kv(be, shape, ctx, exact)
            log(f"synthetic K/V of {ctx} positions written ({time.time()-t0:.1f}s)")
            spkv.check(sess.decode(int(prompt[-1]), logits), "sp_decode_step")
        else:
            chunk = 4096
            for c0 in range(0, ctx, chunk):
                rc = sess.prefill(prompt[c0:c0 + chunk], logits)
                spkv.check(rc, "sp_prefill_chunk")
                log(f"prefill {c0 + min(chunk, ctx - c0)}/{ctx} ({time.time()-t0:.1f}s)")
        prefill_s = time.time() - t0
        tok = int(np.argmax(logits))

        # PCIe-inclusive ABI rate: sp_decode_step with host logits
        n_abi = 8
        t0 = time.time()
        for _ in range(n_abi):
            spkv.check(sess.decode(tok, logits), "sp_decode_step")
            tok = int(np.argmax(logits))
        abi_s = time.time() - t0

        # device-resident greedy loop: warmup, then the timed steps
        toks, _ = be.greedy(tok, args.warmup)
        tok = int(toks[-1]) if args.warmup else tok
        rewinds = []
        if every:
            # greedy runs of `every` steps, each followed by an O(1) rewind of
            # 1..rewind_max tokens (the next run decodes from the rewound position)
            rw = 1 + (splitmix_u64(args.steps // every + 1, 4) % np.uint64(wl["rewind_max"])).astype(np.int64)
            dev_ms = 0.0
            t0 = time.perf_counter()
            for i in range(0, args.steps, every):
                toks, ms_i = be.greedy(tok, min(every, args.steps - i))
                dev_ms += ms_i
                r = int(rw[i // every])
                spkv.check(be.rewind(r), "sp_hipkv_rewind")
                rewinds.append(r)
                tok = int(toks[-1])
            wall = time.perf_counter() - t0
        else:
            t0 = time.perf_counter()
            toks, dev_ms = be.greedy(tok, args.steps)
            wall = time.perf_counter() - t0
            tok = int(toks[-1])
        value = args.steps / wall
        log(f"decode {args.steps} steps: wall {wall*1e3:.1f} ms, device {dev_ms:.1f} ms -> {value:.1f} tok/s"
            + (f" ({len(rewinds)} rewinds, {sum(rewinds)} tokens)" if rewinds else ""))

        # per-kernel-class device times (each launch bracketed by HIP events)
        ms, nl, by = be.kernel_times(tok, args.kernel_steps)
        cls = []
        for i, name in enumerate(CLASSES):
            if nl[i]:
                cls.append(dict(kernel=name, launches=int(nl[i]), avg_us=1e3 * ms[i] / nl[i],
                                total_ms=float(ms[i]), bytes=float(by[i]),
                                gbs=float(by[i] / (ms[i] * 1e-3) / 1e9) if ms[i] > 0 else None))
        dom = max(cls, key=lambda c: c["total_ms"])             # the class with the most device time per step
        dom_names = KERNEL_NAMES.get(dom["kernel"], [])
        if recall and dom["kernel"] == "gqa_decode_attn_global":
            dom_names = [RECALL_NAMES[exact]]
        dom_launch_bytes = dom["bytes"] / dom["launches"]
        traffic = pmc_traffic(dom_names[0]) if len(dom_names) == 1 else None
        kv_gb = sum(c["bytes"] for c in cls if c["kernel"].startswith("gqa")) / 1e9
        kv_ms = sum(c["total_ms"] for c in cls if c["kernel"].startswith("gqa"))
        w_gb = sum(c["bytes"] for c in cls if "gemv" in c["kernel"]) / 1e9
        w_ms = sum(c["total_ms"] for c in cls if "gemv" in c["kernel"])
        step_bytes = sum(c["bytes"] for c in cls) / args.kernel_steps
        for c in cls:
            log(f"  {c['kernel']:26s} launches {c['launches']:6d} avg {c['avg_us']:8.2f} us  {c['gbs'] or 0:8.1f} GB/s")

        headline = (args.workload == "gemma3-12b-32k" and ctx == 32768 and not recall and exact
                    and args.kv == "plain")
        cpu = None
        if not args.no_cpu_baseline and not args.kv_import:
            cpu = cpu_baseline(spm, be, info, shape, exact, args.cpu_steps, tok, sess, args.kv == "spinor", recall)

        rec = {
            "metric": METRIC if args.workload == "gemma3-12b-32k" and ctx == 32768 and not recall else
                      f"kvdecode tokens/s + KV-read HBM GB/s (% of peak), {args.workload} at ctx {ctx}"
                      + (f", ARM recall B={recall[0]} W={recall[1]} sink={recall[2]} r={recall[3]}" if recall else ""),
            "value": round(value, 3), "unit": "tokens/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(1e3 * wall / args.steps, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "int4xint4->int64 GEMV, int32 KV (exact mode)" if exact else
                     ("int4xint4->int64 GEMV, int8 Spinor KV codes, f32 attention" if args.kv == "spinor"
                      else "int4xint4->int64 GEMV, f32 KV/attention"),
            "data": "synthetic: seeded random-init OK_Q4B weights (SplitMix64 seed 0, N(0,0.02)), seeded uniform prompt (seed 1)",
            "config": {"workload": f"{args.workload}: {wl['shape']}-shape kvdecode, prefill {ctx} then {args.steps} greedy steps, batch 1"
                                   + (f", rewind 1-{wl['rewind_max']} tokens every {every} steps" if every else ""),
                       "ctx": ctx, "mode": args.mode, "kv": args.kv,
                       **({"recall": dict(zip(("B", "W", "sink", "r"), recall))} if recall else {}),
                       "b_kv": float(info[2]) / (2 * shape["n_kv_heads"] * shape["head_dim"]), "pmax": pmax,
                       **({"rewinds": rewinds, "max_rewind": max_rewind} if every else {})},
            "roofline": {"bound": "hbm", "kernel": dom["kernel"], "rocprof_kernels": dom_names,
                         "achieved": round(dom["gbs"], 1), "peak": PEAK_GBS, "unit": "GB/s",
                         "frac": round(dom["gbs"] / PEAK_GBS, 4),
                         "algorithmic_bytes_per_launch": round(dom_launch_bytes),
                         "avg_launch_us": round(dom["avg_us"], 3),
                         "timing": ("HIP events recorded by each launch of the class at the kernel's start and end "
                                    "(hipExtLaunchKernelGGL)" if dom["kernel"] in GEMV_CLASSES else
                                    "HIP events around every launch of the class on the backend's stream "
                                    "(the event pair adds about 2 us per launch)"),
                         **rocprof_fields(dom_names, dom_launch_bytes, headline),
                         "traffic": round(traffic["bytes"]) if traffic else None,
                         "traffic_source": traffic},
            "kv_read": {"gbs": round(kv_gb / (kv_ms * 1e-3), 1), "frac": round(kv_gb / (kv_ms * 1e-3) / PEAK_GBS, 4),
                        "bytes_per_step": kv_gb * 1e9 / args.kernel_steps},
            "weight_read": {"gbs": round(w_gb / (w_ms * 1e-3), 1), "frac": round(w_gb / (w_ms * 1e-3) / PEAK_GBS, 4),
                            "bytes_per_step": w_gb * 1e9 / args.kernel_steps},
            "step_algorithmic_bytes": step_bytes,
            "step_hbm_frac": round(step_bytes / (wall / args.steps) / 1e9 / PEAK_GBS, 4),
            "device_ms_per_step": round(dev_ms / args.steps, 4),
            "pcie_inclusive_tokens_per_s": round(n_abi / abi_s, 2),
            "prefill_tokens_per_s": None if args.kv_import else round(ctx / prefill_s, 1),
            "kernels": cls,
            "cpu_baseline": cpu,
        }
        print(json.dumps(rec), flush=True)
        sess.close()
        model.close()
    finally:
        if not args.workdir:
            shutil.rmtree(work, ignore_errors=True)


def import_kv(be, shape, ctx, exact):
    """Synthetic K/V for positions [0, ctx - 1) through sp_hipkv_write_kv: every
    position of the full-attention layers, the last window of the window
    layers (the positions a decode step reads).  Values: exact mode int32 grid
    values below 2^17 (|k|, |v| < 2), float mode N(0, 1); one 64-position block
    of rows reused.  The resident position ends at ctx - 1, so the next decode
    step is position ctx - 1 as after a ctx-token prefill."""
    import spkv
    NL, NKV, HD, SW = shape["n_layers"], shape["n_kv_heads"], shape["head_dim"], shape.get("swa_window", 0)
    gemma = shape["arch_id"] == spkv.ARCH_GEMMA3
    rng = np.random.default_rng(5)
    if exact:
        blk = rng.integers(-(1 << 17), 1 << 17, size=(2, 64, NKV * HD), dtype=np.int32).view(np.float32)
    else:
        blk = rng.standard_normal((2, 64, NKV * HD)).astype(np.float32)
    n = ctx - 1
    glob = [l for l in range(NL) if not (gemma and SW > 0 and l % 6 != 5)]      # Gemma-3: L % 6 == 5 is global
    for p0 in range(0, n, 64):
        m = min(64, n - p0)
        for l in glob:
            be.write_kv(l, p0, blk[0, :m], blk[1, :m])
    for l in range(NL):
        if l in glob:
            continue
        lo = max(0, n - SW)
        for p0 in range(lo, n, 64):
            m = min(64, n - p0)
            be.write_kv(l, p0, blk[0, :m], blk[1, :m])


def run_sessions(args, wl):
    """The batched multi-session workload: S sessions of one model with ragged
    contexts, each step = sp_session_clone of every session (the parent is
    closed, the clone carries on), sp_session_rewind of the clone by 0-4 tokens,
    then one spx_decode_batch over all S sessions (greedy tokens feed the next
    step).  value = S * steps / wall over the timed steps (clone + rewind +
    batched decode), inputs resident in HBM."""
    import spkv
    shape = dict(spkv.SHAPES[wl["shape"]])
    S, hi, lo = wl["sessions"], (args.ctx or wl["ctx"]), wl["ctx_lo"]
    V = shape["vocab"]
    exact = args.mode == "exact"
    ctxs = (lo + splitmix_u64(S, 2) % np.uint64(hi - lo + 1)).astype(np.int64)
    pmax = int(hi) + args.warmup + args.steps + 2 + 64
    rew = (splitmix_u64(S * (args.warmup + args.steps + 2), 3) % np.uint64(5)).astype(np.int64)
    rew = rew.reshape(args.warmup + args.steps + 2, S)
    work = args.workdir or tempfile.mkdtemp(prefix="spkv_bench_", dir=os.environ.get("TMPDIR", "/tmp"))
    prefix = os.path.join(work, wl["shape"])
    t0 = time.time()
    threads = min(16, os.cpu_count() or 1)
    spm, spt = spkv.write_model(prefix, shape=wl["shape"], seed=0, max_context=pmax, threads=threads)
    log(f"model written {os.path.getsize(spm)/1e9:.2f} GB in {time.time()-t0:.1f}s; contexts {ctxs.min()}..{ctxs.max()}, "
        f"mean {ctxs.mean():.0f}, total {int(ctxs.sum())}")
    try:
        model = spkv.Model(spm, spt)
        prompts = splitmix_tokens(int(ctxs.sum()), V, seed=1)
        sess, toks = [], []
        logits = np.zeros(V, np.float32)
        t0 = time.time()
        off = 0
        for i in range(S):
            s = spkv.Session(model, pmax)
            s.attach(pmax, exact=exact)
            pr = prompts[off:off + int(ctxs[i])]
            off += int(ctxs[i])
            for c0 in range(0, len(pr), 4096):
                spkv.check(s.prefill(pr[c0:c0 + 4096], logits), "sp_prefill_chunk")
            toks.append(int(np.argmax(logits)))
            sess.append(s)
            if i % 8 == 7 or i == S - 1:
                log(f"prefilled {i + 1}/{S} sessions ({off} tokens, {time.time()-t0:.1f}s)")
        prefill_s = time.time() - t0
        step_i = [0]

        def fork_and_rewind():
            r = rew[step_i[0]]
            step_i[0] += 1
            for i in range(S):
                c = sess[i].clone()
                sess[i].close()
                sess[i] = c
                if r[i]:
                    spkv.check(c.rewind(int(r[i])), "sp_session_rewind")

        def step(want_logits=False):
            nonlocal toks
            fork_and_rewind()
            rc, lg, nxt = spkv.Session.decode_batch(sess, toks, V, want_logits=want_logits)
            spkv.check(rc, "spx_decode_batch")
            toks = [int(t) for t in nxt]
            return lg

        for _ in range(args.warmup):
            step()
        t0 = time.perf_counter()
        host_s = 0.0
        for _ in range(args.steps):
            h0 = time.perf_counter()
            fork_and_rewind()
            host_s += time.perf_counter() - h0
            rc, _, nxt = spkv.Session.decode_batch(sess, toks, V, want_logits=False)
            spkv.check(rc, "spx_decode_batch")
            toks = [int(t) for t in nxt]
        wall = time.perf_counter() - t0
        value = S * args.steps / wall
        log(f"{args.steps} steps x {S} sessions: wall {wall*1e3:.1f} ms ({1e3*wall/args.steps:.2f} ms/step, "
            f"clone+rewind {1e3*host_s/args.steps:.2f} ms/step) -> {value:.1f} tok/s aggregate")

        # PCIe-inclusive: one step with every session's logits row copied to the host
        t1 = time.perf_counter()
        step(want_logits=True)
        pcie_s = time.perf_counter() - t1

        # one step with each kernel class bracketed by HIP events
        fork_and_rewind()
        bes = [spkv.Backend.wrap(s.backend_handle()) for s in sess]
        pos_before = [s.position() for s in sess]
        nxt, ms, nl, by = spkv.Backend.decode_batch_times(bes, toks)
        # the timed step went around the session layer: take it back on the
        # backends so sessions and backends agree on every position again
        for i, s in enumerate(sess):
            assert bes[i].position() == pos_before[i] + 1
            spkv.check(bes[i].rewind(1), "sp_hipkv_rewind")
        cls = []
        for i, name in enumerate(CLASSES):
            if nl[i]:
                cls.append(dict(kernel=name, launches=int(nl[i]), avg_us=1e3 * ms[i] / nl[i], total_ms=float(ms[i]),
                                bytes=float(by[i]), gbs=float(by[i] / (ms[i] * 1e-3) / 1e9) if ms[i] > 0 else None))
        for c in cls:
            log(f"  {c['kernel']:26s} launches {c['launches']:6d} avg {c['avg_us']:9.2f} us  {c['gbs'] or 0:8.1f} GB/s")
        dom = max(cls, key=lambda c: c["total_ms"])
        kv = [c for c in cls if c["kernel"].startswith("gqa")]
        kv_gb, kv_ms = sum(c["bytes"] for c in kv) / 1e9, sum(c["total_ms"] for c in kv)
        step_bytes = sum(c["bytes"] for c in cls)
        names = {"gqa_decode_attn_global": [BATCH_ATTN_NAMES[exact]]}
        rec = {
            "metric": BATCH_METRIC, "value": round(value, 3), "unit": "tokens/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(1e3 * wall / args.steps, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "int8 MFMA digit-plane GEMMs (int4 weights), int32 KV (exact mode)" if exact
                     else "int8 MFMA digit-plane GEMMs (int4 weights), f32 KV/attention",
            "data": "synthetic: seeded random-init OK_Q4B weights (seed 0), contexts U[1024,16384] (seed 2), "
                    "prompts (seed 1), rewinds U{0..4} (seed 3)",
            "config": {"workload": f"{args.workload}: {wl['shape']}-shape, {S} sessions, ctx U[{lo},{hi}], "
                                   f"per step clone + rewind 0-4 + one batched decode of all sessions",
                       "sessions": S, "ctx_mean": float(ctxs.mean()), "mode": args.mode, "b_kv": 4, "pmax": pmax},
            "roofline": {"bound": "hbm", "kernel": dom["kernel"], "rocprof_kernels": names.get(dom["kernel"], []),
                         "achieved": round(dom["gbs"], 1), "peak": PEAK_GBS, "unit": "GB/s",
                         "frac": round(dom["gbs"] / PEAK_GBS, 4),
                         "algorithmic_bytes_per_launch": round(dom["bytes"] / dom["launches"]),
                         "avg_launch_us": round(dom["avg_us"], 3), "traffic": None},
            "kv_read": {"gbs": round(kv_gb / (kv_ms * 1e-3), 1), "frac": round(kv_gb / (kv_ms * 1e-3) / PEAK_GBS, 4),
                        "bytes_per_step": kv_gb * 1e9},
            "step_algorithmic_bytes": step_bytes,
            "step_hbm_frac": round(step_bytes / (wall / args.steps) / 1e9 / PEAK_GBS, 4),
            "clone_rewind_ms_per_step": round(1e3 * host_s / args.steps, 3),
            "pcie_inclusive_tokens_per_s": round(S / pcie_s, 2),
            "prefill_tokens_per_s": round(float(ctxs.sum()) / prefill_s, 1),
            "kernels": cls,
            "cpu_baseline": None,
        }
        if not args.no_cpu_baseline:
            be0 = bes[0]
            cpu = cpu_baseline(spm, be0, None, shape, exact, args.cpu_steps, toks[0], sess[0])
            cpu["sample"] = "session 0 of the batch only: " + cpu["sample"]
            rec["cpu_baseline"] = cpu
        print(json.dumps(rec), flush=True)
        for s in sess:
            s.close()
        model.close()
    finally:
        if not args.workdir:
            shutil.rmtree(work, ignore_errors=True)


def pmc_summary(path, counter):
    """Per-kernel dispatch count and mean / max of one counter (KiB per dispatch for
    FETCH_SIZE / WRITE_SIZE) from a rocprofv3 --pmc counter_collection.csv."""
    import csv
    from collections import defaultdict
    rows = [r for r in csv.DictReader(open(path)) if r.get("Counter_Name") == counter]
    grids = defaultdict(set)
    for r in rows:
        grids[r["Kernel_Name"]].add(r.get("Grid_Size", ""))
    agg = defaultdict(lambda: [0, 0.0, 0.0])
    for r in rows:
        k = r["Kernel_Name"]
        # a kernel launched with several grid sizes (the same attention kernel on
        # window and full-attention layers) is listed per grid size
        if len(grids[k]) > 1:
            k = f"{k} [grid {r.get('Grid_Size', '')}]"
        a = agg[k]
        v = float(r["Counter_Value"])
        a[0] += 1; a[1] += v; a[2] = max(a[2], v)
    print(f"# {counter} per dispatch (KiB), from {os.path.basename(path)}")
    print(f"{'kernel':100s} {'dispatches':>10s} {'mean':>14s} {'max':>14s}")
    for k, (n, sm, mx) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        print(f"{k:100s} {n:10d} {sm / n:14.1f} {mx:14.1f}")


def calib_copy(nbytes):
    """One plain device-to-device copy of nbytes (the HIP runtime's copy kernel):
    its FETCH_SIZE / WRITE_SIZE counters calibrate the HBM traffic figures."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(a), ctypes.c_size_t(nbytes)) or hip.hipMalloc(ctypes.byref(b), ctypes.c_size_t(nbytes)):
        raise RuntimeError("calibration copy: hipMalloc failed")
    hip.hipMemset(a, 1, ctypes.c_size_t(nbytes))
    hip.hipDeviceSynchronize()
    rc = hip.hipMemcpy(b, a, ctypes.c_size_t(nbytes), 3)       # hipMemcpyDeviceToDevice
    hip.hipDeviceSynchronize()
    hip.hipFree(a); hip.hipFree(b)
    if rc:
        raise RuntimeError(f"calibration copy failed ({rc})")
    log(f"calibration copy of {nbytes >> 20} MiB done")


def cpu_baseline(spm, be, info, shape, exact, n_steps, tok, sess, spinor=False, recall=None):
    """The oracle's decode steps on the host at the same context, the K/V state
    loaded from the device.  Rows: float mode (the reference's arithmetic) and
    exact mode, each n_steps greedy steps on one core (the reference decode is
    single-threaded by contract) and the same steps on all host cores (the
    row-parallel oracle: GEMV rows and attention heads over threads,
    bit-identical to one thread).  In the GPU's mode every threaded oracle step
    is compared with the GPU's logits for the same token (exact mode: bit for
    bit).  The reported value is the float row on one core."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import orc
    spkv = __import__("spkv")
    pos = be.position()
    kvd = shape["n_kv_heads"] * shape["head_dim"]
    win = shape.get("swa_window", 0) if shape.get("arch_id") == spkv.ARCH_GEMMA3 else 0
    threads = min(16, os.cpu_count() or 1)
    rows, kv = [], None

    def load(o, mode):
        t0 = time.time()
        for layer in range(shape["n_layers"]):
            # window layers attend the last `win` positions only (Gemma-3: global iff layer % 6 == 5)
            p0 = max(0, pos - win) if (win and layer % 6 != 5) else 0
            k, v = be.read_kv(layer, p0, pos - p0, kvd)
            # the other mode's row times its decode over the device state carried
            # to its grid (int32 values / 2^16, or floats on the Q16 grid), not a
            # bit-exact replay
            if mode == "float" and exact:
                k = k.view(np.int32).astype(np.float32) / np.float32(65536.0)
                v = v.view(np.int32).astype(np.float32) / np.float32(65536.0)
            elif mode == "exact" and not exact:
                k = np.rint(k * np.float32(65536.0)).astype(np.int32).view(np.float32)
                v = np.clip(np.rint(v * np.float32(65536.0)), -8388607, 8388607).astype(np.int32).view(np.float32)
            o.set_kv(layer, p0, k, v)
            if recall and (not win or layer % 6 == 5):
                # the global layers' recall sidecar (window layers keep none)
                o.set_recall_sidecar(layer, 0, be.recall_sidecar(layer, 0, pos, shape["n_kv_heads"], recall[3]))
        o.set_pos(pos)
        log(f"cpu baseline: KV of {pos} positions loaded in {time.time()-t0:.1f}s")

    glog = np.zeros(shape["vocab"], np.float32)
    L = orc.lib()
    for mode in ("float", "exact"):
        gpu_mode = (mode == "exact") == exact
        o = orc.Oracle(spm, pos + n_steps + 2, orc.EXACT if mode == "exact" else orc.FLOAT,
                       kv_flags=orc.KV_SPINOR if spinor else 0)
        if recall:
            o.set_recall(*recall)
        load(o, mode)
        L.orc_set_threads(1)                                  # one core, n_steps greedy steps
        t_tok, one_s = tok, 0.0
        for i in range(n_steps):
            t0 = time.time(); ol = o.step(t_tok); one_s += time.time() - t0
            t_tok = int(ol.argmax())
            log(f"cpu baseline {mode}: 1-core step {i + 1}/{n_steps} ({one_s:.1f}s)")   # long contexts: minutes
        assert o.rewind(n_steps) == 0
        L.orc_set_threads(threads)                            # all cores, the same n_steps steps
        t_tok, cpu_s, same, worst = tok, 0.0, True, 0.0
        for i in range(n_steps):
            t0 = time.time(); ol = o.step(t_tok); cpu_s += time.time() - t0
            if gpu_mode:
                spkv.check(sess.decode(t_tok, glog), "sp_decode_step")
                same = same and bool(np.array_equal(ol.view(np.uint32), glog.view(np.uint32)))
                worst = max(worst, float(np.abs(ol - glog).max() / max(np.abs(ol).max(), 1e-30)))
            t_tok = int(ol.argmax())
        o.close()
        row = {"mode": mode, "steps": n_steps, "single_core_value": round(n_steps / one_s, 5),
               "cores": threads, "value": round(n_steps / cpu_s, 5)}
        if gpu_mode:
            row.update(gpu_logits_bitexact=same, gpu_logits_max_rel=worst)
        log(f"cpu baseline {mode}: {n_steps} steps on 1 core {one_s:.1f}s ({row['single_core_value']} tok/s), "
            f"on {threads} threads {cpu_s:.1f}s ({row['value']} tok/s)"
            + (f"; gpu==cpu bit-exact {same}, max rel {worst:.2e}" if gpu_mode else ""))
        rows.append(row)
    first = rows[0]
    return {"value": first["single_core_value"], "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{n_steps} greedy decode steps of the same model at ctx {pos} (float-mode oracle, the "
                      f"reference's arithmetic, one core; K/V loaded from the device), {cpu_model()}, "
                      f"nproc {os.cpu_count()}; rows: float and exact mode on 1 core and on {threads} threads",
            "rows": rows,
            "gpu_logits_bitexact": next((r.get("gpu_logits_bitexact") for r in rows if "gpu_logits_bitexact" in r), None),
            "gpu_logits_max_rel": next((r.get("gpu_logits_max_rel") for r in rows if "gpu_logits_max_rel" in r), None)}


if __name__ == "__main__":
    main()
