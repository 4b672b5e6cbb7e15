"""C5 batched decode chain (atlas_amd.decode.GemmaDecodeStep) on the GPU:
eager execution and HIP-graph replays, bit-identical to the oracle's
composition of the same ops in the reference decode order
(crates/atlas-model/src/gemma4_executor.rs:4123-4690)."""
import sys

import numpy as np
import pytest

from atlas_amd import workloads as wl
from atlas_amd.decode import GemmaDecodeStep

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-decode] {msg}", flush=True)
    sys.stdout.flush()


def oracle_step(ora, step):
    """The same chain on the CPU oracle."""
    S, h = step.S, step.host
    B, H, QH, D, F, L, W = S.batch, S.hidden, S.q_heads, S.head_dim, S.ffn, S.layers, S.ple_width
    state = ora.embed_q4_0(h["token_table"], h["ids"], step.vocab, H, wl.f32_sqrt(H))
    ple = ora.ple(h["ple_table"], h["ids"], h["ple_proj_in"], step.vocab, L, W, 16.0, wl.SQRT_2_RECIP)
    local = ora.rope_tables_gemma4(h["positions"], D // 2, D, 1e4)
    glob = ora.rope_tables_gemma4(h["positions"], D // 2, D, 1e6)
    out = {"q_out": [], "k_out": [], "ffn_act": [], "ple_act": []}
    for layer, lay in enumerate(step.layers):
        c, s = glob if S.is_global(layer) else local
        qo, ko = ora.qk_norm_rope(lay["q"], lay["k"], lay["qw"], lay["kw"], c, s, B, QH, True, D, D // 2, S.eps)
        _, state = ora.rms_norm_residual(lay["attn_out"], lay["post_attn_w"], state, B, H, S.eps)
        act = ora.geglu(lay["gate"], lay["up"])
        _, state = ora.rms_norm_residual(lay["ffn_out"], lay["post_ffn_w"], state, B, H, S.eps)
        pact = ora.geglu_offset(lay["ple_gate"], ple, layer * W, L * W, W, B)
        state = ora.rms_norm_add_scale(lay["ple_proj"], lay["post_norm_w"], state, lay["scale"][0], B, H, S.eps)
        out["q_out"].append(qo)
        out["k_out"].append(ko)
        out["ffn_act"].append(act)
        out["ple_act"].append(pact)
    out["state"], out["ple"] = state, ple
    return out


def assert_same(got, exp, tag):
    for key in ("state", "ple"):
        assert np.array_equal(got[key].view(np.uint32), np.asarray(exp[key]).view(np.uint32)), f"{tag}: {key}"
    for key in ("q_out", "k_out", "ffn_act", "ple_act"):
        for layer, (g, e) in enumerate(zip(got[key], exp[key])):
            assert np.array_equal(g.view(np.uint32), np.asarray(e).view(np.uint32)), f"{tag}: {key}[{layer}]"


@pytest.mark.parametrize("batch,vocab", [(64, 8192), (256, 262144)])
def test_decode_step_eager_and_graph_replays(rt, ora, batch, vocab):
    """A small chain, and BASELINE configs[4] at its stated shape: 256
    sequences at positions drawn from [0, 131072), 35 layers with local and
    global theta interleaved 4:1, the Gemma vocabulary of 262144 rows for the
    Q4_0 token and PLE tables."""
    shape = wl.DecodeShape(batch=batch)
    say(f"building decode step {shape} vocab={vocab}")
    step = GemmaDecodeStep(rt, shape, seed=3, vocab=vocab)
    try:
        exp_a = oracle_step(ora, step)
        say("eager step")
        step.enqueue()
        rt.sync()
        assert_same(step.results(), exp_a, "eager")
        say("capture")
        step.capture()
        ids_a, pos_a = step.host["ids"].copy(), step.host["positions"].copy()
        ids_b, pos_b = step.draw_tokens(99)
        exp_b = None
        for i, which in enumerate("ABBA"):
            ids, pos = (ids_a, pos_a) if which == "A" else (ids_b, pos_b)
            step.set_tokens(ids, pos)
            rt.sync()
            # eager work on the same stream between replays
            rt.memset(step.out["state"], 0, shape.batch * shape.hidden * 4)
            say(f"replay {i} tokens {which}")
            step.replay()
            rt.sync()
            if which == "A":
                exp = exp_a
            else:
                if exp_b is None:
                    exp_b = oracle_step(ora, step)
                exp = exp_b
            assert_same(step.results(), exp, f"replay {i} ({which})")
    finally:
        step.close()


def test_decode_step_under_auto_reduction(rt_auto, ora):
    """The library's default reduction, which bench.py --decode and every
    integrator use: every norm of the C5 chain is an epilogue that can cancel
    (residual, add-scale) or the QK-norm, so AUTO keeps the sequential fold and
    the chain is bit-identical to the oracle, eager and replayed."""
    shape = wl.DecodeShape(batch=64)
    say(f"building decode step {shape} vocab=8192 (AUTO)")
    step = GemmaDecodeStep(rt_auto, shape, seed=4, vocab=8192)
    try:
        exp = oracle_step(ora, step)
        say("eager step (AUTO)")
        step.enqueue()
        rt_auto.sync()
        assert_same(step.results(), exp, "eager AUTO")
        step.capture()
        for i in range(2):
            rt_auto.memset(step.out["state"], 0, shape.batch * shape.hidden * 4)
            say(f"replay {i} (AUTO)")
            step.replay()
            rt_auto.sync()
            assert_same(step.results(), exp, f"replay {i} AUTO")
    finally:
        step.close()


def test_graph_capture_rejects_synchronising_calls(rt):
    from atlas_amd import OperatorError
    rt.graph_begin()
    try:
        with pytest.raises(OperatorError) as e:
            rt.sync()
        assert e.value.kind == "InvalidInput"
    finally:
        g = rt.graph_end()
        rt.graph_destroy(g)
    rt.sync()
