"""Benchmark of the fused per-layer ops on one MI355X.

Workload (BASELINE.json configs[2] + configs[3], T = 4096 tokens): one
"step" is one pass of every fused op of the path over one batch of
synthetic, HBM-resident inputs:

    embed_q4_0   token gather + Q4_0 dequant x sqrt(1536)     [262144 x 1536] table
    embed_q6_k   token gather + Q6_K dequant x sqrt(1536)     [262144 x 1536] table
    ple_q4_0     PLE gather + dequant x 16 + proj, x 1/sqrt2  [262144 x 35*256] table
    rms_norm     pre-norm RMSNorm                             [4096 x 1536], eps 1e-6
    qk_norm_rope per-head QK-RMSNorm + RoPE (theta 1e4)       Q [4096,8,256], K [4096,1,256]
    rms_residual post-norm RMSNorm + residual epilogue        [4096 x 1536]
    geglu        gelu_tanh(gate) * up                         [4096 x 6144]

`value` = tokens / s for the whole step (T / wall time per step, inputs
already resident).  Per-op achieved GB/s uses algorithmic bytes (each input
read once, each output written once) over the op's average launch duration
from HIP events around back-to-back launches that rotate over >= 4 buffer
sets (> 1 GB in aggregate, so the 256 MB MALL cannot serve repeats).  The
CPU baseline is the oracle (a single-threaded C restatement of the reference
CPU operators) timed on this host over a bounded token sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--reduction sequential|wide]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "achieved HBM GB/s (% of peak) per fused op; fused-op tokens/s at T=4096, 1 GPU"
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_sets(rt, wl, nsets):
    """Device buffers: shared tables + `nsets` rotating activation sets."""
    L, Q = wl.GemmaLayerShape(), wl.QuantGatherShape()
    T, H, D, QH, F = L.tokens, L.hidden, L.head_dim, L.q_heads, L.ffn
    r = wl.rng(2024)
    log("generating tables")
    tables = {
        "q4": rt.upload(wl.q4_0_table(r, Q.vocab, Q.hidden)),
        "q6": rt.upload(wl.q6_k_table(r, Q.vocab, Q.hidden)),
        "ple": rt.upload(wl.q4_0_table(r, Q.vocab, Q.ple_layers * Q.ple_width)),
        "w": rt.upload(wl.normal(r, H, 1.0, 0.1)),
        "qw": rt.upload(wl.normal(r, D, 1.0, 0.1)),
        "kw": rt.upload(wl.normal(r, D, 1.0, 0.1)),
    }
    from atlas_amd import rope_tables_gemma4

    cos, sin = rope_tables_gemma4(np.arange(T, dtype=np.uint32), D // 2, D, L.theta_local)
    log("generating activations")
    host = {
        "x": wl.normal(r, T * H), "res": wl.normal(r, T * H),
        "q": wl.normal(r, T * QH * D), "k": wl.normal(r, T * D), "cos": cos, "sin": sin,
        "gate": wl.normal(r, T * F), "up": wl.normal(r, T * F),
        "proj": wl.normal(r, T * Q.ple_layers * Q.ple_width),
    }
    outs = {"y": T * H, "out": T * H, "qo": T * QH * D, "ko": T * D, "glu": T * F, "e4": T * H, "e6": T * H,
            "pleo": T * Q.ple_layers * Q.ple_width}
    sets = []
    for i in range(nsets):
        s = {k: rt.upload(v) for k, v in host.items()}
        s["ids"] = rt.upload(wl.token_ids(wl.rng(77 + i), T, Q.vocab))
        for k, n in outs.items():
            s[k] = rt.empty(n)
        sets.append(s)
    return tables, sets


def op_table(wl):
    L, Q = wl.GemmaLayerShape(), wl.QuantGatherShape()
    T, H, D, QH, F = L.tokens, L.hidden, L.head_dim, L.q_heads, L.ffn
    ple_row = Q.ple_layers * Q.ple_width
    scale = float(wl.f32_sqrt(H))
    es, os_ = 16.0, float(wl.SQRT_2_RECIP)
    return {
        # name: (algorithmic bytes per launch, launch(rt, tables, set))
        "embed_q4_0": (T * wl.q_row_bytes(H, False) + T * 4 + T * H * 4,
                       lambda rt, t, s: rt.embed_q4_0(t["q4"], s["ids"], s["e4"], Q.vocab, H, T, scale)),
        "embed_q6_k": (T * wl.q_row_bytes(H, True) + T * 4 + T * H * 4,
                       lambda rt, t, s: rt.embed_q6_k(t["q6"], s["ids"], s["e6"], Q.vocab, H, T, scale)),
        "ple_q4_0": (T * wl.q_row_bytes(ple_row, False) + T * 4 + 2 * T * ple_row * 4,
                     lambda rt, t, s: rt.ple_q4_0(t["ple"], s["ids"], s["proj"], s["pleo"], Q.vocab, Q.ple_layers,
                                                  Q.ple_width, T, es, os_)),
        "rms_norm": (2 * T * H * 4 + H * 4,
                     lambda rt, t, s: rt.rms_norm(s["x"], t["w"], s["y"], T, H, L.eps)),
        "qk_norm_rope": (2 * T * (QH + 1) * D * 4 + 2 * T * (D // 2) * 4 + 2 * D * 4,
                         lambda rt, t, s: rt.qk_norm_rope(s["q"], s["k"], t["qw"], t["kw"], s["cos"], s["sin"],
                                                          s["qo"], s["ko"], T, QH, 1, D, D // 2, L.eps)),
        "rms_residual": (3 * T * H * 4 + H * 4,
                         lambda rt, t, s: rt.rms_norm_residual(s["x"], t["w"], s["res"], None, s["out"], T, H,
                                                               L.eps)),
        "geglu": (3 * T * F * 4, lambda rt, t, s: rt.geglu(s["gate"], s["up"], s["glu"], T * F)),
    }


def time_op(rt, launch, tables, sets, iters):
    for i in range(3):
        launch(rt, tables, sets[i % len(sets)])
    rt.sync()
    a, b = rt.event(), rt.event()
    rt.record(a)
    for i in range(iters):
        launch(rt, tables, sets[i % len(sets)])
    rt.record(b)
    rt.sync()
    return rt.elapsed_ms(a, b) / iters


def cpu_baseline(wl, budget_s=10.0):
    """Single-threaded oracle over a token sample of the same step (TEST-ONLY oracle)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as ora

    L, Q = wl.GemmaLayerShape(), wl.QuantGatherShape()
    Ts, H, D, QH, F = 64, L.hidden, L.head_dim, L.q_heads, L.ffn
    ple_row = Q.ple_layers * Q.ple_width
    r = wl.rng(99)
    vocab = 4096  # gather cost does not depend on the vocabulary size
    q4, q6, pt = wl.q4_0_table(r, vocab, H), wl.q6_k_table(r, vocab, H), wl.q4_0_table(r, vocab, ple_row)
    ids = wl.token_ids(r, Ts, vocab)
    x, res, w = wl.normal(r, Ts * H), wl.normal(r, Ts * H), wl.normal(r, H, 1, 0.1)
    q, k, qw, kw = wl.normal(r, Ts * QH * D), wl.normal(r, Ts * D), wl.normal(r, D, 1, 0.1), wl.normal(r, D, 1, 0.1)
    c, s = ora.rope_tables_gemma4(np.arange(Ts, dtype=np.uint32), D // 2, D, L.theta_local)
    g, u, proj = wl.normal(r, Ts * F), wl.normal(r, Ts * F), wl.normal(r, Ts * ple_row)
    scale = float(wl.f32_sqrt(H))

    def step():
        ora.embed_q4_0(q4, ids, vocab, H, scale)
        ora.embed_q6_k(q6, ids, vocab, H, scale)
        ora.ple(pt, ids, proj, vocab, Q.ple_layers, Q.ple_width, 16.0, float(wl.SQRT_2_RECIP))
        ora.rms_norm(x, w, Ts, H, L.eps)
        ora.qk_norm_rope(q, k, qw, kw, c, s, Ts, QH, True, D, D // 2, L.eps)
        ora.rms_norm_residual(x, w, res, Ts, H, L.eps)
        ora.geglu(g, u)

    step()
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        step()
        reps += 1
    el = time.perf_counter() - t0
    return {"value": round(Ts * reps / el, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{reps} passes of the full step over {Ts} tokens ({el:.1f} s), single-threaded C oracle "
                      f"(-O2, -ffp-contract=off), same op list and shapes per token"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--sets", type=int, default=4)
    ap.add_argument("--op-iters", type=int, default=100)
    ap.add_argument("--reduction", choices=["sequential", "wide"], default="sequential")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma-separated op subset for per-op timing (profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every op of this path is row-independent and no multi-GPU "
              "figure is produced (see DESIGN.md for how tokens would shard). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    from atlas_amd import ATLAS_REDUCTION_SEQUENTIAL, ATLAS_REDUCTION_WIDE, HipRuntime
    from atlas_amd import workloads as wl

    rt = HipRuntime(0, ATLAS_REDUCTION_WIDE if args.reduction == "wide" else ATLAS_REDUCTION_SEQUENTIAL)
    tables, sets = build_sets(rt, wl, args.sets)
    ops = op_table(wl)
    L = wl.GemmaLayerShape()
    T = L.tokens
    only = [o for o in args.only.split(",") if o]

    def step(i):
        s = sets[i % len(sets)]
        for _, (_, launch) in ops.items():
            launch(rt, tables, s)

    per_op = {}
    for name, (nbytes, launch) in ops.items():
        if only and name not in only:
            continue
        log(f"timing {name}")
        ms = time_op(rt, launch, tables, sets, args.op_iters)
        gbs = nbytes / (ms * 1e-3) / 1e9
        per_op[name] = {"us": round(ms * 1e3, 3), "bytes": nbytes, "GB/s": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "tokens_per_s": round(T / (ms * 1e-3), 1)}
    if only:
        print(json.dumps({"per_op": per_op}))
        return

    log("timed steps")
    for i in range(args.warmup):
        step(i)
    rt.sync()
    a, b = rt.event(), rt.event()
    t0 = time.perf_counter()
    rt.record(a)
    for i in range(args.steps):
        step(i)
    rt.record(b)
    rt.sync()
    wall = time.perf_counter() - t0
    ev_ms = rt.elapsed_ms(a, b)
    ms_per_step = wall * 1e3 / args.steps
    step_bytes = sum(v[0] for v in ops.values())

    dom = max(ops, key=lambda n: ops[n][0])
    d = per_op[dom]
    result = {
        "metric": METRIC,
        "value": round(T / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "gemma4-e2b-fused-ops-T4096 (C3 layer ops + C4 gathers, one pass of each op)",
                   "tokens": T, "hidden": L.hidden, "q_heads": L.q_heads, "head_dim": L.head_dim, "ffn": L.ffn,
                   "vocab": wl.QuantGatherShape().vocab, "ple": "35x256 Q4_0", "reduction": args.reduction,
                   "buffer_sets": args.sets, "step_bytes": step_bytes,
                   "step_GB/s": round(step_bytes / (ev_ms * 1e-3 / args.steps) / 1e9, 1)},
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": d["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": d["frac"], "traffic": None,
                     "algorithmic_bytes_per_launch": d["bytes"], "avg_launch_us": d["us"]},
        "ops": per_op,
    }
    if not args.no_cpu:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(wl, args.cpu_seconds)
    print(json.dumps(result))
    rt.close()


if __name__ == "__main__":
    main()
