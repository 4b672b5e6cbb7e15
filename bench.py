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
already resident in HBM).  Per-op achieved GB/s = algorithmic bytes (each
input read once, each output written once) / the op's average launch
duration, from HIP events on the library's stream around back-to-back
launches.  Every op rotates over its own buffer sets -- table copies
included -- totalling >= 1 GiB, so the 256 MB MALL cannot serve repeats.
Each op line also carries `floor_us`: a plain streaming kernel that reads
the op's input bytes and writes its output bytes (measurement only,
atlas_amd/libatlas_stream_floor.so), timed the same way -- the size-matched
floor of launch plus memory system -- and `of_floor` = floor_us / us.
The CPU baseline is the oracle (a single-threaded C restatement of the
reference CPU operators) timed on this host over a bounded token sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--reduction auto|sequential|wide]
       python bench.py --only geglu,rms_norm        (per-op timing only, for profiling)
       python bench.py --copy-mib 256               (a D2D copy of known size: the PMC
                                                      calibration kernel)
       python bench.py --floor-sweep                (the streaming floor alone over the ops' sizes)
       python bench.py --policy-sweep --op-iters 100 (the floor kernel over cache policies and grid shapes)
       python bench.py --decode [--batch 1]         (configs[4] batched decode, separate line; --batch 1:
                                                      one sequence, next to the reference's per-token figures)
       python bench.py --config c1|c2|gemv|kv|logits (other op configurations, per-op lines)
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "achieved HBM GB/s (% of peak) per fused op; fused-op tokens/s at T=4096, 1 GPU"
HBM_PEAK_GBS = 8000.0
ROTATION_BYTES = 1 << 30


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Arena:
    """One device allocation made before anything is timed and kept until the
    bench ends: every op's rotating buffer sets and the streaming floor's
    buffers are carved from it.  On MI355X a buffer allocated after others
    were freed measured up to 3.5 % slower for the same kernel (qk_norm_rope
    at T=4096: 14.92 us against 14.39 us on a fresh allocation), so per-op
    allocate/free would make each op's time depend on the ops timed before
    it."""

    def __init__(self, rt, nbytes):
        self.rt = rt
        self.nbytes = nbytes
        self.buf = rt.alloc(nbytes)

    def region(self, nbytes):
        if nbytes > self.nbytes:
            raise RuntimeError(f"bench arena holds {self.nbytes} bytes, {nbytes} requested")
        return self.buf


def _align(n, a=4096):
    return -(-max(n, 16) // a) * a


class Ops:
    """The step's ops: host inputs, algorithmic bytes and launchers."""

    def __init__(self, wl, rope_tables):
        L, Q = wl.GemmaLayerShape(), wl.QuantGatherShape()
        self.L, self.Q = L, Q
        T, H, D, QH, F = L.tokens, L.hidden, L.head_dim, L.q_heads, L.ffn
        ple_row = Q.ple_layers * Q.ple_width
        r = wl.rng(2024)
        log("generating inputs")
        cos, sin = rope_tables(np.arange(T, dtype=np.uint32), D // 2, D, L.theta_local)
        self.host = {
            "q4": wl.q4_0_table(r, Q.vocab, Q.hidden), "q6": wl.q6_k_table(r, Q.vocab, Q.hidden),
            "ple": wl.q4_0_table(r, Q.vocab, ple_row), "ids": wl.token_ids(r, T, Q.vocab),
            "w": wl.normal(r, H, 1.0, 0.1), "qw": wl.normal(r, D, 1.0, 0.1), "kw": wl.normal(r, D, 1.0, 0.1),
            "x": wl.normal(r, T * H), "res": wl.normal(r, T * H), "q": wl.normal(r, T * QH * D),
            "k": wl.normal(r, T * D), "cos": cos, "sin": sin, "gate": wl.normal(r, T * F),
            "up": wl.normal(r, T * F), "proj": wl.normal(r, T * ple_row),
        }
        scale = float(wl.f32_sqrt(H))
        es, os_ = 16.0, float(wl.SQRT_2_RECIP)
        f4 = 4
        # name: (inputs copied per set, outputs per set (elements), algorithmic bytes, launch)
        self.table = {
            "embed_q4_0": (["q4", "ids"], {"e4": T * H}, T * wl.q_row_bytes(H, False) + T * 4 + T * H * f4,
                           lambda rt, s: rt.embed_q4_0(s["q4"], s["ids"], s["e4"], Q.vocab, H, T, scale)),
            "embed_q6_k": (["q6", "ids"], {"e6": T * H}, T * wl.q_row_bytes(H, True) + T * 4 + T * H * f4,
                           lambda rt, s: rt.embed_q6_k(s["q6"], s["ids"], s["e6"], Q.vocab, H, T, scale)),
            "ple_q4_0": (["ple", "ids", "proj"], {"pleo": T * ple_row},
                         T * wl.q_row_bytes(ple_row, False) + T * 4 + 2 * T * ple_row * f4,
                         lambda rt, s: rt.ple_q4_0(s["ple"], s["ids"], s["proj"], s["pleo"], Q.vocab, Q.ple_layers,
                                                   Q.ple_width, T, es, os_)),
            "rms_norm": (["x", "w"], {"y": T * H}, 2 * T * H * f4 + H * f4,
                         lambda rt, s: rt.rms_norm(s["x"], s["w"], s["y"], T, H, L.eps)),
            "qk_norm_rope": (["q", "k", "qw", "kw", "cos", "sin"], {"qo": T * QH * D, "ko": T * D},
                             2 * T * (QH + 1) * D * f4 + 2 * T * (D // 2) * f4 + 2 * D * f4,
                             lambda rt, s: rt.qk_norm_rope(s["q"], s["k"], s["qw"], s["kw"], s["cos"], s["sin"],
                                                           s["qo"], s["ko"], T, QH, 1, D, D // 2, L.eps)),
            "rms_residual": (["x", "w", "res"], {"out": T * H}, 3 * T * H * f4 + H * f4,
                             lambda rt, s: rt.rms_norm_residual(s["x"], s["w"], s["res"], None, s["out"], T, H,
                                                                L.eps)),
            "geglu": (["gate", "up"], {"glu": T * F}, 3 * T * F * f4,
                      lambda rt, s: rt.geglu(s["gate"], s["up"], s["glu"], T * F)),
        }

    def set_bytes(self, name):
        ins, outs, _, _ = self.table[name]
        return sum(self.host[k].nbytes for k in ins) + sum(n * 4 for n in outs.values())

    def out_bytes(self, name):
        """Bytes the op writes: its output buffers (counted in f32 elements),
        or `written[name]` where a buffer is larger than what one launch
        writes (a cache) or the op writes in place."""
        written = getattr(self, "written", {})
        if name in written:
            return written[name]
        return sum(n * 4 for n in self.table[name][1].values())

    def _layout(self, names):
        keys = sorted({k for n in names for k in self.table[n][0]})
        outs = {}
        for n in names:
            outs.update(self.table[n][1])
        layout, off = {}, 0
        for k, nb, dt in ([(k, self.host[k].nbytes, self.host[k].dtype) for k in keys]
                          + [(k, n * 4, np.dtype(np.float32)) for k, n in outs.items()]):
            layout[k] = (off, dt)
            off += _align(nb)
        return keys, layout, off

    def sets_bytes(self, names, nsets):
        return nsets * self._layout(names)[2]

    def build_sets(self, rt, names, nsets, arena):
        """`nsets` buffer sets holding every input/output of `names`, carved
        from `arena` (one set after another, tensors at 4 KiB-aligned offsets).
        Set 0 is uploaded; the others are device-to-device copies."""
        keys, layout, per_set = self._layout(names)
        base = arena.region(nsets * per_set)
        sets = []
        for i in range(nsets):
            s = {k: base.offset(i * per_set + o, dt) for k, (o, dt) in layout.items()}
            for k in keys:
                if i == 0:
                    s[k].upload(self.host[k])
                else:
                    rt.copy(s[k], sets[0][k], self.host[k].nbytes)
            sets.append(s)
        rt.sync()
        return sets


class ConfigOps(Ops):
    """Per-op timing at the other op configurations (separate lines, not the headline):
    c1 = BASELINE configs[0] (SmolLM2-135M-shaped FP32 ops, T=128),
    c2 = BASELINE configs[1] (SmolLM2-1.7B-shaped FP16 storage, T=2048),
    gemv = the RMS-folded Q4_0 decode projections, the PLE input gate and the normed F16 PLE projection of one
           Gemma-4-E2B-like token,
    kv = the KV append with the fused V RMSNorm (prefill batch and one decode token),
    logits = the soft cap + greedy argmax decode tail (256 sequences and one token)."""

    def __init__(self, wl, rope_tables, cfg):
        r = wl.rng(2025)
        h16 = lambda a: a.astype(np.float16).view(np.uint16)
        self.host, self.table = {}, {}
        if cfg == "c2":
            S = wl.LlamaPrefillShape()
            T, H, NH, D, F = S.tokens, S.hidden, S.heads, S.head_dim, S.ffn
            cos, sin = rope_tables(np.arange(T, dtype=np.uint32), D, S.theta)
            self.tokens = T
            self.host = {"x": h16(wl.normal(r, T * H)), "res": h16(wl.normal(r, T * H)),
                         "w": h16(wl.normal(r, H, 1.0, 0.1)), "q": h16(wl.normal(r, T * NH * D)),
                         "k": h16(wl.normal(r, T * NH * D)), "cos": cos, "sin": sin,
                         "gate": h16(wl.normal(r, T * F)), "up": h16(wl.normal(r, T * F))}
            self.table = {
                "add_rms_norm_f16": (["x", "res", "w"], {"rs": T * H // 2, "y": T * H // 2}, 4 * T * H * 2 + H * 2,
                                     lambda rt, s: rt.add_rms_norm_f16(s["x"], s["res"], s["w"], s["rs"], s["y"], T,
                                                                       H, S.eps)),
                "rope_half_f16_qk": (["q", "k", "cos", "sin"], {"qo": T * NH * D // 2, "ko": T * NH * D // 2},
                                     4 * T * NH * D * 2 + 2 * T * (D // 2) * 4,
                                     lambda rt, s: rt.rope_half_qk(s["q"], s["k"], s["cos"], s["sin"], s["qo"],
                                                                   s["ko"], T, NH, NH, D, D // 2, f16=True)),
                "swiglu_f16": (["gate", "up"], {"o": T * F // 2}, 3 * T * F * 2,
                               lambda rt, s: rt.swiglu_f16(s["gate"], s["up"], s["o"], T * F)),
            }
        elif cfg == "gemv":
            # the RMS-folded Q4_0 decode projections of one
            # Gemma-4-E2B-like token (hidden 1536; Q 8x256, K/V 1x256; FFN 6144)
            L = wl.GemmaLayerShape()
            H, QN, KVN, F = L.hidden, L.q_heads * L.head_dim, L.head_dim, L.ffn
            rb = wl.q_row_bytes(H, False)
            self.tokens = 1
            PW, PL = wl.QuantGatherShape().ple_width, wl.QuantGatherShape().ple_layers
            self.host = {"x": wl.normal(r, H), "w": wl.normal(r, H, 1.0, 0.1), "qw": wl.q4_0_table(r, QN, H),
                         "kw": wl.q4_0_table(r, KVN, H), "vw": wl.q4_0_table(r, KVN, H),
                         "gw": wl.q4_0_table(r, F, H), "uw": wl.q4_0_table(r, F, H),
                         "pgw": wl.q4_0_table(r, PW, H), "ple": wl.normal(r, PL * PW),
                         "ppw": wl.normal(r, PL * PW * H, 0.0, 0.05).astype(np.float16).view(np.uint16),
                         "pnw": wl.normal(r, PW, 1.0, 0.1)}
            eps = L.eps
            self.table = {
                "qkv_rms": (["x", "w", "qw", "kw", "vw"], {"qo": QN, "ko": KVN, "vo": KVN},
                            (QN + 2 * KVN) * rb + 2 * H * 4 + (QN + 2 * KVN) * 4,
                            lambda rt, s: rt.matmul_q4_0_qkv_rms(s["x"], s["qw"], s["kw"], s["vw"], s["qo"], s["ko"],
                                                                 s["vo"], H, QN, KVN, s["w"], eps)),
                "gate_up_rms": (["x", "w", "gw", "uw"], {"go": F, "uo": F}, 2 * F * rb + 2 * H * 4 + 2 * F * 4,
                                lambda rt, s: rt.matmul_q4_0_gate_up_rms(s["x"], s["gw"], s["uw"], s["go"], s["uo"],
                                                                         H, F, s["w"], eps)),
                # the PLE input gate of one layer (256 rows, layer 17's PLE slice)
                "ple_gate_gelu": (["x", "pgw", "ple"], {"pgo": PW}, PW * rb + H * 4 + PW * 4 + PW * 4,
                                  lambda rt, s: rt.ple_gate_gelu(s["x"], s["pgw"], s["ple"], 17 * PW, s["pgo"], H,
                                                                 PW)),
                # ... and the PLE projection it follows: F16 [35 * 256, 1536] times the token's state,
                # the projection scale, the stable group norm as epilogue
                "ple_projection_f16": (["x", "ppw", "pnw"], {"ppo": PL * PW},
                                       PL * PW * H * 2 + H * 4 + PW * 4 + PL * PW * 4,
                                       lambda rt, s: rt.ple_projection_f16(s["x"], s["ppw"], s["pnw"], s["ppo"], H,
                                                                           PW, PL, H ** -0.5, eps)),
            }
        elif cfg == "kv":
            # KV append with the fused V RMSNorm at the
            # Gemma-4-E2B-like shape (one KV head of 256): a 4096-token prefill
            # batch into a 4096-position cache, and one decode token
            L = wl.GemmaLayerShape()
            T, W, cap = L.tokens, L.head_dim, L.tokens
            self.tokens = T
            self.host = {"k": wl.normal(r, T * W), "v": wl.normal(r, T * W),
                         "pos": np.arange(T, dtype=np.uint32), "pos1": np.array([T // 2], np.uint32)}
            rows = {"f32": W * 4, "q8_0": W // 32 * 34, "q4_0": W // 32 * 18}
            self.table = {}
            for fmt in ("f32", "q8_0", "q4_0"):
                cache_f = 2 * cap * rows[fmt] // 4
                self.table[f"kv_append_{fmt}_vnorm_T{T}"] = (
                    ["k", "v", "pos"], {f"c_{fmt}": cache_f}, 2 * T * W * 4 + T * 4 + 2 * T * rows[fmt],
                    (lambda f: lambda rt, s: rt.kv_append(f, s["k"], s["v"], s[f"c_{f}"], W, cap, s["pos"], T,
                                                          True, L.eps))(fmt))
            self.table["kv_append_q4_0_vnorm_decode"] = (
                ["k", "v", "pos1"], {"c1": 2 * cap * rows["q4_0"] // 4}, 2 * W * 4 + 4 + 2 * rows["q4_0"],
                lambda rt, s: rt.kv_append("q4_0", s["k"], s["v"], s["c1"], W, cap, s["pos1"], 1, True, L.eps))
            # the cache outputs are whole caches; a launch writes its tokens' rows
            self.written = {f"kv_append_{fmt}_vnorm_T{T}": 2 * T * rows[fmt] for fmt in ("f32", "q8_0", "q4_0")}
            self.written["kv_append_q4_0_vnorm_decode"] = 2 * rows["q4_0"]
        elif cfg == "logits":
            # the decode tail, soft cap (30) + greedy argmax
            # over the 262144-entry vocabulary: the C5 batch of 256 sequences
            # (in place, as the reference caps its logits buffer) and one token
            V, cap = wl.QuantGatherShape().vocab, 30.0
            self.tokens = 256
            self.host = {"l256": wl.normal(r, 256 * V, 0.0, 10.0), "l1": wl.normal(r, V, 0.0, 10.0)}
            self.table = {
                "softcap_argmax_B256": (["l256"], {"s256": 256}, 2 * 256 * V * 4 + 256 * 4,
                                        lambda rt, s: rt.softcap_argmax(s["l256"], s["l256"], s["s256"], 256, V, cap)),
                "argmax_B256": (["l256"], {"a256": 256}, 256 * V * 4 + 256 * 4,
                                lambda rt, s: rt.argmax(s["l256"], s["a256"], 256, V)),
                "softcap_argmax_B1": (["l1"], {"s1": 1}, 2 * V * 4 + 4,
                                      lambda rt, s: rt.softcap_argmax(s["l1"], s["l1"], s["s1"], 1, V, cap)),
            }
            # the soft cap rewrites the logits in place
            self.written = {"softcap_argmax_B256": 256 * V * 4 + 256 * 4, "softcap_argmax_B1": V * 4 + 4}
        else:
            S = wl.SmolShape()
            T, H, QH, KH, D, F, V = S.tokens, S.hidden, S.q_heads, S.kv_heads, S.head_dim, S.ffn, S.vocab
            cos, sin = rope_tables(np.arange(T, dtype=np.uint32), D, S.theta)
            self.tokens = T
            self.host = {"x": wl.normal(r, T * H), "w": wl.normal(r, H, 1.0, 0.1), "q": wl.normal(r, T * QH * D),
                         "k": wl.normal(r, T * KH * D), "cos": cos, "sin": sin, "gate": wl.normal(r, T * F),
                         "up": wl.normal(r, T * F), "table": wl.normal(wl.rng(0), V * H, 0.0, 0.02),
                         "ids": wl.token_ids(wl.rng(0), T, V)}
            self.table = {
                "rms_norm": (["x", "w"], {"y": T * H}, 2 * T * H * 4 + H * 4,
                             lambda rt, s: rt.rms_norm(s["x"], s["w"], s["y"], T, H, S.eps)),
                "rope_half_qk": (["q", "k", "cos", "sin"], {"qo": T * QH * D, "ko": T * KH * D},
                                 2 * T * (QH + KH) * D * 4 + 2 * T * (D // 2) * 4,
                                 lambda rt, s: rt.rope_half_qk(s["q"], s["k"], s["cos"], s["sin"], s["qo"], s["ko"],
                                                               T, QH, KH, D, D // 2)),
                "swiglu": (["gate", "up"], {"o": T * F}, 3 * T * F * 4,
                           lambda rt, s: rt.swiglu(s["gate"], s["up"], s["o"], T * F)),
                "embed_f32": (["table", "ids"], {"e": T * H}, T * H * 4 + T * 4 + T * H * 4,
                              lambda rt, s: rt.embed_f32(s["table"], s["ids"], s["e"], V, H, T)),
            }



class _RecordingLib:
    """Records the C-ABI calls made through it: (entry point, arguments
    converted to their ctypes types once) instead of making them."""

    def __init__(self, lib, calls):
        self._lib, self._calls = lib, calls

    def __getattr__(self, name):
        fn = getattr(self._lib, name)

        def record(*args):
            conv = tuple(a if isinstance(a, t) else t(a) for t, a in zip(fn.argtypes, args))
            self._calls.append((fn, conv))
            return 0

        return record


class _Recorder:
    """Stands in for a HipRuntime while an op's launcher runs once on the
    host: the runtime's method runs with this object as `self` and every
    C-ABI call it would make is recorded instead."""

    def __init__(self, rt):
        self.rt, self.ctx, self.calls = rt, rt.ctx, []
        self.lib = _RecordingLib(rt.lib, self.calls)

    def _check(self, rc):
        pass

    def __getattr__(self, name):
        return getattr(type(self.rt), name).__get__(self)


def bind_launch(rt, launch, s):
    """The op launch `launch(rt, s)` as a list of (C entry point, converted
    arguments): the timed loops call the library directly, so what they time
    is the launches themselves and not the Python wrapper around each one
    (a Rust or C caller has none).  Every call still goes through the same
    C-ABI entry point with its argument checks."""
    rec = _Recorder(rt)
    launch(rec, s)
    if not rec.calls:
        raise RuntimeError("the op launcher made no library call to bind")
    return rec.calls


def run_bound(rt, calls):
    for fn, args in calls:
        rc = fn(*args)
        if rc:
            rt._check(rc)


def time_launches(rt, launch, sets, iters, batches=5, bind=True):
    """Milliseconds per launch: the median over `batches` runs of iters /
    batches back-to-back launches (HIP events on the library stream), after
    iters / 2 untimed launches.  An op is timed right after its buffer sets
    were uploaded, with the GPU idle meanwhile; with 50 warm-up launches the
    first 1000 timed ones of the C4 Q6_K gather measured 5.58 us against 5.44
    for the next 1000.  bind: `launch` is a runtime op, timed as its bound
    C-ABI calls (bind_launch); otherwise it is called as given."""
    if bind:
        bound = [bind_launch(rt, launch, st) for st in sets]
        go = lambda i: run_bound(rt, bound[i % len(bound)])  # noqa: E731
    else:
        go = lambda i: launch(rt, sets[i % len(sets)])  # noqa: E731
    warm = max(3, iters // 2)
    for i in range(warm):
        go(i)
    rt.sync()
    n = max(1, iters // batches)
    a, b = rt.event(), rt.event()
    per = []
    for _ in range(batches):
        rt.record(a)
        for i in range(n):
            go(i)
        rt.record(b)
        rt.sync()
        per.append(rt.elapsed_ms(a, b) / n)
    return float(np.median(per))


class StreamFloor:
    """Size-matched streaming floor for an op: plain streaming kernels
    (atlas_amd/libatlas_stream_floor.so, measurement only) that read the op's
    input bytes and write its output bytes as contiguous 128-bit streams, in
    three shapes (one float4 per thread with nontemporal loads and stores; a
    4096-workgroup grid striding over the streams with sc1+nt stores; one
    float4 per thread with plain loads), the fastest of a sweep over cache
    policies and grid shapes; the floor is the fastest of the three.  Timed
    like the ops: HIP events on the library's stream around back-to-back
    launches, rotating over >= 1 GiB of distinct buffers.  What the launch
    path and the memory system give for that many bytes at that size, with no
    arithmetic, reduction or gather."""

    def __init__(self, rt, arena):
        import ctypes

        path = os.path.join(ROOT, "atlas_amd", "libatlas_stream_floor.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
        self.lib = ctypes.CDLL(path)
        self.lib.atlas_floor_stream_kind.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                                     ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int]
        self.lib.atlas_floor_stream_kind.restype = ctypes.c_int
        self.lib.atlas_floor_kinds.restype = ctypes.c_int
        self.lib.atlas_floor_launch.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p]
        self.lib.atlas_floor_launch.restype = ctypes.c_int
        self.lib.atlas_floor_gather.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                                ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint32]
        self.lib.atlas_floor_gather.restype = ctypes.c_int
        self.rt = rt
        self.arena = arena
        self.stream = rt.lib.atlas_hip_get_stream(rt.ctx)
        self.sink = rt.alloc(256)

    @staticmethod
    def pool_bytes(in_bytes, out_bytes):
        per_set = (in_bytes + 255) // 256 * 256 + (out_bytes + 255) // 256 * 256
        return max(4, math.ceil(ROTATION_BYTES / per_set)) * per_set

    def us(self, in_bytes, out_bytes, iters):
        return min(self.us_kinds(in_bytes, out_bytes, iters).values())

    def us_kinds(self, in_bytes, out_bytes, iters):
        """Microseconds per launch of every shape, {kind: us}, on one pool."""
        rt = self.rt
        ib, ob = (in_bytes + 255) // 256 * 256, (out_bytes + 255) // 256 * 256
        per_set = ib + ob
        nsets = max(4, math.ceil(ROTATION_BYTES / per_set))
        pool = self.arena.region(nsets * per_set)
        rt.memset(pool, 0, nsets * per_set)
        result = {}
        for kind in range(self.lib.atlas_floor_kinds()):
            def launch(_rt, i):
                base = pool.ptr + i * per_set
                rc = self.lib.atlas_floor_stream_kind(self.stream, base, in_bytes, base + ib, out_bytes,
                                                      self.sink.ptr, kind)
                if rc != 0:
                    raise RuntimeError(f"stream floor launch failed: HIP error {rc}")

            result[kind] = time_launches(rt, launch, list(range(nsets)), iters, bind=False) * 1e3
        return result

    def gather_us(self, sets, table, ids, out, row_bytes, vocab, tokens, out_row_bytes, iters):
        """The token gather's dependency chain without its decode (id, then
        row, then the output row) on an op's own rotating sets: what a
        gather of these rows can reach at this size."""
        rt = self.rt

        def launch(_rt, s):
            rc = self.lib.atlas_floor_gather(self.stream, s[table].ptr, row_bytes, vocab, s[ids].ptr, tokens,
                                             s[out].ptr, out_row_bytes)
            if rc != 0:
                raise RuntimeError(f"gather floor launch failed: HIP error {rc}")

        return time_launches(rt, launch, sets, iters, bind=False) * 1e3

    def calls_us(self, in_bytes, out_bytes, n, distinct, iters, graphs=True):
        """Microseconds per launch of every shape, {kind: us}, when n launches
        run back to back as one HIP graph (or eagerly), over n distinct buffer
        pairs (distinct) or one: the way the decode step's ops are timed."""
        rt = self.rt
        ib, ob = (in_bytes + 255) // 256 * 256, (out_bytes + 255) // 256 * 256
        per_set = ib + ob
        sets = n if distinct else 1
        pool = self.arena.region(sets * per_set)
        rt.memset(pool, 0, sets * per_set)
        result = {}
        for kind in range(self.lib.atlas_floor_kinds()):
            def launch(i):
                base = pool.ptr + (i % sets) * per_set
                rc = self.lib.atlas_floor_stream_kind(self.stream, base, in_bytes, base + ib, out_bytes,
                                                      self.sink.ptr, kind)
                if rc != 0:
                    raise RuntimeError(f"stream floor launch failed: HIP error {rc}")

            g = None
            if graphs:
                rt.graph_begin()
                try:
                    for i in range(n):
                        launch(i)
                finally:
                    g = rt.graph_end()

            def run():
                if g is not None:
                    rt.graph_launch(g)
                else:
                    for i in range(n):
                        launch(i)

            for _ in range(3):
                run()
            rt.sync()
            a, b = rt.event(), rt.event()
            rt.record(a)
            for _ in range(iters):
                run()
            rt.record(b)
            rt.sync()
            if g is not None:
                rt.graph_destroy(g)
            result[kind] = rt.elapsed_ms(a, b) / (iters * n) * 1e3
        return result

    def launch_us(self, blocks, iters):
        """Back-to-back launches of `blocks` empty one-wavefront workgroups."""
        rt = self.rt

        def launch():
            rc = self.lib.atlas_floor_launch(self.stream, blocks, self.sink.ptr)
            if rc != 0:
                raise RuntimeError(f"launch floor failed: HIP error {rc}")

        for _ in range(3):
            launch()
        rt.sync()
        a, b = rt.event(), rt.event()
        rt.record(a)
        for _ in range(iters):
            launch()
        rt.record(b)
        rt.sync()
        return rt.elapsed_ms(a, b) / iters * 1e3


POLICY_NAMES = ["plain", "nt", "sc1", "sc1+nt", "sc0+sc1+nt"]
# token gathers timed against the gather floor too: (table, output, Q6_K)
GATHER_FLOOR = {"embed_q4_0": ("q4", "e4", False), "embed_q6_k": ("q6", "e6", True)}


def policy_sweep(rt, iters):
    """The streaming kernel over every load x store cache policy and two grid
    shapes at the ops' sizes (one JSON line per size): the evidence for the
    floor's three shapes."""
    import ctypes

    sizes = [("rms", 25.2, 25.2), ("gather", 3.5, 25.2), ("residual", 50.3, 25.2), ("qk", 42.0, 37.7),
             ("geglu", 201.3, 100.7)]
    arena = Arena(rt, max(StreamFloor.pool_bytes(int(r * 1e6), int(w * 1e6)) for _, r, w in sizes))
    floor = StreamFloor(rt, arena)
    lib = floor.lib
    lib.atlas_floor_stream_policy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                              ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_uint32]
    lib.atlas_floor_stream_policy.restype = ctypes.c_int
    for name, r_mb, w_mb in sizes:
        ib, ob = int(r_mb * 1e6) // 256 * 256, int(w_mb * 1e6) // 256 * 256
        per_set = ib + ob
        nsets = max(4, math.ceil(ROTATION_BYTES / per_set))
        pool = arena.region(nsets * per_set)
        rt.memset(pool, 0, nsets * per_set)
        res = {}
        for grid in (0, 4096):
            for lp in range(lib.atlas_floor_policy_count()):
                for sp in range(lib.atlas_floor_policy_count()):
                    def launch(i):
                        base = pool.ptr + (i % nsets) * per_set
                        rc = lib.atlas_floor_stream_policy(floor.stream, base, ib, base + ib, ob, floor.sink.ptr, lp,
                                                           sp, grid)
                        if rc != 0:
                            raise RuntimeError(f"policy sweep launch failed: HIP error {rc}")
                    for i in range(3):
                        launch(i)
                    rt.sync()
                    a, b = rt.event(), rt.event()
                    rt.record(a)
                    for i in range(iters):
                        launch(i)
                    rt.record(b)
                    rt.sync()
                    res[f"{'full' if grid == 0 else grid}/{POLICY_NAMES[lp]}/{POLICY_NAMES[sp]}"] = round(
                        rt.elapsed_ms(a, b) / iters * 1e3, 3)
        best = min(res, key=res.get)
        print(json.dumps({"size": name, "read_MB": r_mb, "write_MB": w_mb, "best": best, "best_us": res[best],
                          "best_frac": round((ib + ob) / (res[best] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                          "us": res}), flush=True)


def floor_fields(floor, nbytes, out_bytes, op_us, iters):
    """floor_us: the size-matched streaming floor; of_floor = floor_us / op_us
    (1.0 = the op moves its bytes as fast as a plain stream of the same size)."""
    out_bytes = min(out_bytes, nbytes)
    kinds = floor.us_kinds(nbytes - out_bytes, out_bytes, iters)
    fu = min(kinds.values())
    return {"floor_us": round(fu, 3), "of_floor": round(fu / op_us, 4),
            "floor_us_by_kind": [round(kinds[k], 3) for k in sorted(kinds)]}


def floor_sweep(rt, iters):
    """The floor alone over the sizes the ops move (read MB, write MB): one JSON
    line per size, for the committed floor summary."""
    sizes = [(1.57, 1.57), (6.3, 6.3), (12.6, 12.6), (25.2, 0.0), (0.0, 25.2), (3.5, 25.2), (25.2, 25.2),
             (16.8, 16.8), (42.0, 37.7), (50.3, 25.2), (67.1, 33.6), (201.3, 100.7), (171.1, 143.2)]
    floor = StreamFloor(rt, Arena(rt, max(StreamFloor.pool_bytes(int(r * 1e6), int(w * 1e6)) for r, w in sizes)))
    for blocks in (256, 4096, 16384):
        print(json.dumps({"empty_workgroups": blocks, "us": round(floor.launch_us(blocks, iters), 3)}), flush=True)
    for r_mb, w_mb in sizes:
        ib, ob = int(r_mb * 1e6) // 16 * 16, int(w_mb * 1e6) // 16 * 16
        kinds = floor.us_kinds(ib, ob, iters)
        us = min(kinds.values())
        print(json.dumps({"read_MB": r_mb, "write_MB": w_mb, "us": round(us, 3),
                          "us_by_kind": {k: round(v, 3) for k, v in kinds.items()},
                          "GB/s": round((ib + ob) / (us * 1e-6) / 1e9, 1),
                          "frac": round((ib + ob) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}), flush=True)


def cpu_baseline(wl, budget_s=1.0, max_threads=16, host=None):
    """The C oracle (-O3, -ffp-contract=off; the restatement of the reference
    CPU operators) on the same step's ops, timed on this host: each op alone
    over 64-token slices of the full-size inputs (the 262144-row tables
    included, so gathers read cache-cold rows), for `budget_s` seconds on one
    thread and then `budget_s` on every host core of the box's share (the
    affinity set, capped at OMP_NUM_THREADS -- 16 per GPU on the MI355X
    boxes -- and at max_threads; each thread on its own token slices; ctypes
    releases the GIL during each C call).  The line records the affinity
    count, the share and the threads used.  Per op: GB/s (algorithmic bytes)
    and tokens/s on 1 and N cores; the step's tokens/s is 1 / the sum of the
    ops' seconds per token.  `host`: the step's full-size inputs (Ops.host); generated
    here when None.  The oracle is test infrastructure; here it is the
    reported CPU baseline, never the product."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import threading
    import oracle as ora

    L, Q = wl.GemmaLayerShape(), wl.QuantGatherShape()
    T, Ts, H, D, QH, F = L.tokens, 64, L.hidden, L.head_dim, L.q_heads, L.ffn
    ple_row = Q.ple_layers * Q.ple_width
    vocab = Q.vocab
    scale = float(wl.f32_sqrt(H))
    if host is None:
        r = wl.rng(2024)
        host = {"q4": wl.q4_0_table(r, vocab, H), "q6": wl.q6_k_table(r, vocab, H),
                "ple": wl.q4_0_table(r, vocab, ple_row), "ids": wl.token_ids(r, T, vocab),
                "w": wl.normal(r, H, 1.0, 0.1), "qw": wl.normal(r, D, 1.0, 0.1), "kw": wl.normal(r, D, 1.0, 0.1),
                "x": wl.normal(r, T * H), "res": wl.normal(r, T * H), "q": wl.normal(r, T * QH * D),
                "k": wl.normal(r, T * D), "gate": wl.normal(r, T * F), "up": wl.normal(r, T * F),
                "proj": wl.normal(r, T * ple_row)}
    h = host
    cos, sin = ora.rope_tables_gemma4(np.arange(T, dtype=np.uint32), D // 2, D, L.theta_local)

    def sl(a, t0, width):
        return a[t0 * width:(t0 + Ts) * width]

    # name: (algorithmic bytes per token, call on tokens [t0, t0 + Ts))
    per_tok = {
        "embed_q4_0": (wl.q_row_bytes(H, False) + 4 + H * 4,
                       lambda t0: ora.embed_q4_0(h["q4"], h["ids"][t0:t0 + Ts], vocab, H, scale)),
        "embed_q6_k": (wl.q_row_bytes(H, True) + 4 + H * 4,
                       lambda t0: ora.embed_q6_k(h["q6"], h["ids"][t0:t0 + Ts], vocab, H, scale)),
        "ple_q4_0": (wl.q_row_bytes(ple_row, False) + 4 + 2 * ple_row * 4,
                     lambda t0: ora.ple(h["ple"], h["ids"][t0:t0 + Ts], sl(h["proj"], t0, ple_row), vocab,
                                        Q.ple_layers, Q.ple_width, 16.0, float(wl.SQRT_2_RECIP))),
        "rms_norm": (2 * H * 4, lambda t0: ora.rms_norm(sl(h["x"], t0, H), h["w"], Ts, H, L.eps)),
        "qk_norm_rope": (2 * (QH + 1) * D * 4 + 2 * (D // 2) * 4,
                         lambda t0: ora.qk_norm_rope(sl(h["q"], t0, QH * D), sl(h["k"], t0, D), h["qw"], h["kw"],
                                                     cos[t0:t0 + Ts], sin[t0:t0 + Ts], Ts, QH, True, D, D // 2,
                                                     L.eps)),
        "rms_residual": (3 * H * 4, lambda t0: ora.rms_norm_residual(sl(h["x"], t0, H), h["w"], sl(h["res"], t0, H),
                                                                      Ts, H, L.eps)),
        "geglu": (3 * F * 4, lambda t0: ora.geglu(sl(h["gate"], t0, F), sl(h["up"], t0, F))),
    }

    def run(fn, threads):
        """Calls of fn on `threads` threads for budget_s; seconds per token."""
        reps, stop = [0] * threads, [0.0]
        start = threading.Barrier(threads + 1, action=lambda: stop.__setitem__(0, time.perf_counter() + budget_s))

        def work(i):
            t0 = (i * 977 * Ts) % (T - Ts)
            fn(t0)  # warm
            start.wait()
            while time.perf_counter() < stop[0]:
                fn(t0)
                reps[i] += 1
                t0 = (t0 + 7 * Ts) % (T - Ts)
        pool = [threading.Thread(target=work, args=(i,)) for i in range(threads)]
        for t in pool:
            t.start()
        start.wait()
        t_begin = stop[0] - budget_s
        for t in pool:
            t.join()
        el = time.perf_counter() - t_begin
        return el / (Ts * max(1, sum(reps)))

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    # the host CPUs this process may use (affinity) and the share of them the
    # GPU box grants one GPU's job (OMP_NUM_THREADS, set to 16 there; a pool
    # sized past the share competes with the driver's own work)
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or max_threads
    threads = max(1, min(share, cores, max_threads))
    ops, s1, sn = {}, 0.0, 0.0
    for name, (bpt, fn) in per_tok.items():
        one = run(fn, 1)
        many = run(fn, threads) if threads > 1 else one
        s1, sn = s1 + one, sn + many
        ops[name] = {"GB/s_1core": round(bpt / one / 1e9, 3), f"GB/s_{threads}cores": round(bpt / many / 1e9, 3),
                     "tokens_per_s_1core": round(1.0 / one, 1), f"tokens_per_s_{threads}cores": round(1.0 / many, 1)}
    return {"value": round(1.0 / sn, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "affinity_cores": cores, "cpu_share": share,
            "single_thread": round(1.0 / s1, 1), "ops": ops,
            "sample": f"each op of the step alone over 64-token slices of the full-size inputs (262144-row "
                      f"tables), the C oracle built -O3 -ffp-contract=off: {budget_s:g} s on 1 thread and "
                      f"{budget_s:g} s on {threads} threads per op; step tokens/s = 1 / sum of the ops' "
                      f"seconds per token"}


# The reference's published decode figures for this path (Apple M2 Max, one
# sequence, whole model; docs/atlas-metal-phases/README.md:51-54): context only, not comparable
# hardware or batch.
M2_MAX_CONTEXT = {
    "qk_norm_rope_ms_per_token": 2.31,      # docs/atlas-metal-phases/next-improvements.md:51-56
    "ple_family_ms_per_token": 1.7,         # docs/atlas-metal-phases/README.md:51-54
    "decode_gpu_ms_per_token": 18.8,        # docs/atlas-metal-phases/README.md:51
}


def decode_bench(rt, steps, warmup, batch=256, graphs=True, floor=True):
    """`batch` sequences x 1 token (256 by default; 1 for
    the single-sequence decode the reference publishes), 35 layers of the
    fused ops in the reference decode order (atlas_amd.decode), eager and as
    one HIP graph; then each op alone, timed as a graph of its 35 per-layer
    launches (the whole step's dispatch mode)."""
    from atlas_amd import workloads as wl
    from atlas_amd.decode import GemmaDecodeStep

    S = wl.DecodeShape(batch=batch)
    log(f"building the decode step ({batch} sequences, 35 layers of seeded weights and stand-ins)")
    step = GemmaDecodeStep(rt, S, seed=5)

    def timed(fn, n):
        for _ in range(warmup):
            fn()
        rt.sync()
        a, b = rt.event(), rt.event()
        rt.record(a)
        for _ in range(n):
            fn()
        rt.record(b)
        rt.sync()
        return rt.elapsed_ms(a, b) * 1e3 / n

    eager_us = timed(step.enqueue, steps)
    if graphs:
        step.capture()
        graph_us = timed(step.replay, steps)
    else:
        graph_us = eager_us

    def per_launch_us(calls):
        """Microseconds per call of `calls` run back to back: as one graph
        (the step's dispatch mode), or eagerly with graphs off."""
        if not graphs:
            return timed(lambda: [c() for c in calls], steps) / len(calls)
        rt.graph_begin()
        try:
            for c in calls:
                c()
        finally:
            g = rt.graph_end()
        us = timed(lambda: rt.graph_launch(g), steps) / len(calls)
        rt.graph_destroy(g)
        return us

    L = S.layers
    per_op = {}
    heads = step.head_ops()
    for i, (name, nbytes, _) in enumerate(heads):
        us = per_launch_us([heads[i][2]] * L)
        per_op[name] = {"us": round(us, 3), "bytes": nbytes, "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "per": "step"}
    layer_ops = [step.layer_ops(layer) for layer in range(L)]
    for k, (name, nbytes, _) in enumerate(layer_ops[0]):
        us = per_launch_us([ops[k][2] for ops in layer_ops])
        per_op[name] = {"us": round(us, 3), "bytes": nbytes, "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "per": "layer"}
    head_us = sum(v["us"] for v in per_op.values() if v["per"] == "step")
    if floor:
        # each op against the streaming floor of its own bytes, timed the same
        # way: L launches as one graph, over L distinct buffers for the
        # per-layer ops and one buffer for the per-step gathers (as above)
        written = step.written_bytes()
        need = max((L if v["per"] == "layer" else 1) * ((v["bytes"] - written[k] + 255) // 256 * 256
                                                       + (written[k] + 255) // 256 * 256)
                   for k, v in per_op.items())
        fl = StreamFloor(rt, Arena(rt, need))
        for k, v in per_op.items():
            out_b = min(written[k], v["bytes"])
            fu = min(fl.calls_us(v["bytes"] - out_b, out_b, L, v["per"] == "layer", steps, graphs).values())
            v.update({"floor_us": round(fu, 3), "of_floor": round(fu / v["us"], 4)})
    step.close()
    per_layer = (graph_us - head_us) / L
    mode = "graph replay" if graphs else "eager launches"
    result = {"metric": f"C5 decode ({batch} sequence{'s' if batch > 1 else ''}): per-layer latency of the fused "
                        f"ops ({mode}), 1 GPU",
              "value": round(per_layer, 3), "unit": "us/layer", "higher_is_better": False, "n_gpus": 1,
              "steps": steps, "warmup": warmup, "dtype": "f32", "data": "synthetic",
              "config": {"workload": "gemma4-e2b-batched-decode (configs[4])", "sequences": batch,
                         "layers": L, "hidden": S.hidden, "ffn": S.ffn, "q_heads": S.q_heads,
                         "head_dim": S.head_dim, "vocab": S.vocab, "theta": "1e4 local / 1e6 global, 4:1",
                         "ops_per_layer": 6},
              "step_us_graph": round(graph_us, 2), "step_us_eager": round(eager_us, 2),
              "embed_ple_us": round(head_us, 2), "bytes_per_layer": step.bytes_per_layer(),
              "layer_GB/s": round(step.bytes_per_layer() / (per_layer * 1e-6) / 1e9, 1),
              "step_GB/s": round(step.bytes_per_step() / (graph_us * 1e-6) / 1e9, 1),
              "per_op_us": per_op}
    if batch == 1:
        # per-token totals of this build next to the reference's published
        # per-token figures (other hardware, whole model: context only)
        result["per_token_ms"] = {
            "qk_norm_rope_35_layers": round(per_op["qk_norm_rope"]["us"] * L / 1e3, 4),
            "ple_family": round((per_op["ple_q4_0"]["us"] + L * (per_op["geglu_offset_ple"]["us"] +
                                                                 per_op["rms_add_scale_ple"]["us"])) / 1e3, 4),
            "fused_ops_step_graph": round(graph_us / 1e3, 4)}
        result["reference_m2_max_context"] = M2_MAX_CONTEXT
    return result


def pmc_traffic(kernel_op):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, or None."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    entry = data.get("ops", {}).get(kernel_op)
    return None if entry is None else entry.get("traffic_bytes")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # ~45 ms of untimed steps: clocks and memory reach steady state after a few
    # hundred launches (10 warm-up steps measured ~1.5 % lower)
    ap.add_argument("--warmup", type=int, default=300)
    # per-op timing: 1000 back-to-back launches (~50 ms at the large ops) so
    # the average is taken at steady clocks (100 measured 1-2 % slower)
    ap.add_argument("--op-iters", type=int, default=1000)
    ap.add_argument("--step-sets", type=int, default=4)
    ap.add_argument("--reduction", choices=["auto", "sequential", "wide"], default="auto",
                    help="row-sum order: auto (the library default: tree where the output is a plain scaled row, "
                         "sequential where an epilogue cancels), sequential (bit-identical everywhere), wide")
    ap.add_argument("--cpu-seconds", type=float, default=1.0, help="CPU baseline: seconds per op and thread count")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-floor", action="store_true",
                    help="skip the size-matched streaming floor per op")
    ap.add_argument("--floor-sweep", action="store_true",
                    help="time the streaming floor alone over the ops' sizes (one JSON line per size)")
    ap.add_argument("--policy-sweep", action="store_true",
                    help="the streaming kernel over every load x store cache policy and two grid shapes at the ops' "
                         "sizes (one JSON line per size)")
    ap.add_argument("--only", default="", help="comma-separated op subset: per-op timing only (profiling)")
    ap.add_argument("--copy-mib", type=int, default=0, help="also time a device-to-device copy of this size")
    ap.add_argument("--config", choices=["c3c4", "c1", "c2", "gemv", "kv", "logits"], default="c3c4",
                    help="c1 / c2: per-op lines for BASELINE configs[0] / configs[1]; gemv: the RMS-folded "
                         "Q4_0 decode projections of one token; kv: the KV append with the fused V norm; "
                         "logits: the soft cap + argmax decode tail -- instead of the headline")
    ap.add_argument("--decode", action="store_true",
                    help="BASELINE configs[4] batched decode (per-layer latency, eager and HIP graph) instead")
    ap.add_argument("--no-graph", action="store_true",
                    help="--decode: eager launches only (for tracing tools that do not follow graph replays)")
    ap.add_argument("--batch", type=int, default=256,
                    help="--decode: sequences per step (256 = configs[4]; 1 = the single-sequence decode the "
                         "reference publishes per-token figures for)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every op of this path is row-independent and this build "
              "produces no multi-GPU figure (a batch would shard by token rows with no exchange). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    from atlas_amd import (ATLAS_REDUCTION_AUTO, ATLAS_REDUCTION_SEQUENTIAL, ATLAS_REDUCTION_WIDE, HipRuntime,
                           rope_tables_gemma4)
    from atlas_amd import workloads as wl

    rt = HipRuntime(0, {"auto": ATLAS_REDUCTION_AUTO, "sequential": ATLAS_REDUCTION_SEQUENTIAL,
                        "wide": ATLAS_REDUCTION_WIDE}[args.reduction])
    if args.floor_sweep:
        floor_sweep(rt, args.op_iters)
        rt.close()
        return
    if args.policy_sweep:
        policy_sweep(rt, args.op_iters)
        rt.close()
        return
    if args.decode:
        print(json.dumps(decode_bench(rt, min(args.steps, 50), min(args.warmup, 5), args.batch, not args.no_graph,
                                      not args.no_floor)))
        rt.close()
        return

    def arena_for(o, nsets_of, names, step_sets=0):
        """The arena every timed region below carves its buffers from."""
        need = [o.sets_bytes([n], nsets_of(n)) for n in names]
        if step_sets:
            need.append(o.sets_bytes(list(o.table), step_sets))
        if not args.no_floor:
            need += [StreamFloor.pool_bytes(o.table[n][2] - min(o.out_bytes(n), o.table[n][2]),
                                            min(o.out_bytes(n), o.table[n][2])) for n in names]
        arena = Arena(rt, max(need, default=1 << 20))
        return arena, None if args.no_floor else StreamFloor(rt, arena)

    if args.config != "c3c4":
        from atlas_amd import rope_tables_llama

        cops = ConfigOps(wl, rope_tables_llama, args.config)
        # the weight-streaming projections need >= 1 GiB of distinct weights
        # to keep the 256 MB MALL out of the measurement
        cap = 1024 if args.config in ("gemv", "kv", "logits") else 64

        def cnsets(name):
            return min(cap, max(4, math.ceil(ROTATION_BYTES / cops.set_bytes(name))))

        arena, floor = arena_for(cops, cnsets, list(cops.table))
        per_op = {}
        for name, (_, _, nbytes, launch) in cops.table.items():
            nsets = cnsets(name)
            log(f"timing {args.config} {name} ({nsets} rotating sets)")
            sets = cops.build_sets(rt, [name], nsets, arena)
            ms = time_launches(rt, launch, sets, args.op_iters)
            gbs = nbytes / (ms * 1e-3) / 1e9
            per_op[name] = {"us": round(ms * 1e3, 3), "bytes": nbytes, "GB/s": round(gbs, 1),
                            "frac": round(gbs / HBM_PEAK_GBS, 4),
                            "tokens_per_s": round(cops.tokens / (ms * 1e-3), 1), "rotating_sets": nsets}
            if floor is not None:
                per_op[name].update(floor_fields(floor, nbytes, cops.out_bytes(name), ms * 1e3, args.op_iters))
        print(json.dumps({"config": args.config, "per_op": per_op}))
        rt.close()
        return
    ops = Ops(wl, rope_tables_gemma4)
    T = ops.L.tokens
    only = [o for o in args.only.split(",") if o]
    for o in only:
        if o not in ops.table:
            sys.exit(f"unknown op {o}; choose from {', '.join(ops.table)}")

    def nsets_of(name):
        return max(4, math.ceil(ROTATION_BYTES / ops.set_bytes(name)))

    timed = [n for n in ops.table if not ((only or args.copy_mib) and n not in only)]
    arena, floor = arena_for(ops, nsets_of, timed, 0 if (only or args.copy_mib) else args.step_sets)
    per_op = {}
    for name in timed:
        _, _, nbytes, launch = ops.table[name]
        nsets = nsets_of(name)
        log(f"timing {name} ({nsets} rotating sets)")
        sets = ops.build_sets(rt, [name], nsets, arena)
        ms = time_launches(rt, launch, sets, args.op_iters)
        gbs = nbytes / (ms * 1e-3) / 1e9
        per_op[name] = {"us": round(ms * 1e3, 3), "bytes": nbytes, "GB/s": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
                        "rotating_sets": nsets}
        if floor is not None and name in GATHER_FLOOR:
            # on the op's own sets, before the streaming floor reuses the arena
            tk, ok, q6 = GATHER_FLOOR[name]
            H = ops.L.hidden
            gu = floor.gather_us(sets, tk, "ids", ok, wl.q_row_bytes(H, q6), ops.Q.vocab, T, H * 4, args.op_iters)
            per_op[name].update({"gather_floor_us": round(gu, 3), "of_gather_floor": round(gu / (ms * 1e3), 4)})
        if not (only or args.copy_mib or args.no_floor):
            # the same bytes moved by a plain stream: what launch + memory give at this size
            per_op[name].update(floor_fields(floor, nbytes, ops.out_bytes(name), ms * 1e3, args.op_iters))
    if args.copy_mib:
        n = args.copy_mib << 20
        src, dst = rt.alloc(n), rt.alloc(n)
        rt.memset(src, 1, n)
        for _ in range(5):
            rt.copy(dst, src, n)
        rt.sync()
        log(f"copied {args.copy_mib} MiB x5 (PMC calibration)")
    if only or args.copy_mib:
        print(json.dumps({"per_op": per_op}))
        rt.close()
        return

    log("timed steps")
    names = list(ops.table)
    sets = ops.build_sets(rt, names, args.step_sets, arena)

    bound = [[call for nm in names for call in bind_launch(rt, ops.table[nm][3], st)] for st in sets]

    def step(i):
        run_bound(rt, bound[i % len(bound)])

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
    step_bytes = sum(v[2] for v in ops.table.values())

    dom = max(per_op, key=lambda n: per_op[n]["us"])
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
        "config": {"workload": "gemma4-e2b-fused-ops-T4096 (configs[2] layer ops + configs[3] gathers, "
                               "one pass of each op per step)",
                   "tokens": T, "hidden": ops.L.hidden, "q_heads": ops.L.q_heads, "head_dim": ops.L.head_dim,
                   "ffn": ops.L.ffn, "vocab": ops.Q.vocab, "ple": "35x256 Q4_0", "reduction": args.reduction,
                   "step_sets": args.step_sets, "step_bytes": step_bytes,
                   "step_GB/s": round(step_bytes / (ev_ms * 1e-3 / args.steps) / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": d["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": d["frac"], "traffic": pmc_traffic(dom), "kernel": dom,
                     "algorithmic_bytes_per_launch": d["bytes"], "avg_launch_us": d["us"]},
        "ops": per_op,
    }
    if not args.no_cpu:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(wl, args.cpu_seconds, host=ops.host)
    print(json.dumps(result))
    rt.close()


if __name__ == "__main__":
    main()
