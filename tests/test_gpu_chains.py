"""The Llama resident decode token and the Gemma layer-major prefill chunk
(atlas_amd.chains) on the GPU, eager and as HIP-graph replays, against the
oracle's composition of the same ops in the reference executors' order:
`ResidentExecutor::forward_token` (crates/atlas-model/src/executor.rs:
1042-1429) and `encode_prefill_layer_major_layer` (crates/atlas-model/src/
gemma4_executor.rs:3694-4121) at the 512-token prefill chunk (:23)."""
import sys

import numpy as np
import pytest

from atlas_amd import workloads as wl
from atlas_amd.chains import GemmaPrefillChunk, LlamaDecodeStep, PrefillShape

pytestmark = pytest.mark.gpu
u32 = np.uint32


def say(msg):
    print(f"[gpu-chains] {msg}", flush=True)
    sys.stdout.flush()


def same(tag, got, exp):
    g, e = np.asarray(got), np.asarray(exp)
    assert g.shape == e.shape, (tag, g.shape, e.shape)
    assert np.array_equal(g.view(np.uint8), e.view(np.uint8)), tag


# ------------------------------------------------------------ Llama decode

def llama_oracle(ora, step, token, position, caches):
    """One token of the chain on the CPU oracle; `caches` (one per layer) is
    updated in place like the device caches."""
    S, L = step.S, step.L
    H, QH, KH, D = S.hidden, S.q_heads, S.kv_heads, S.head_dim
    pos = np.array([position], u32)
    state = ora.embed_f32(step.host["table"], np.array([token], u32), S.vocab, H)
    c, s = ora.rope_tables_llama(pos, D, S.theta)
    out = {"q_rot": [], "k_rot": [], "act": []}
    norm = ora.rms_norm(state, step.layers[0]["input_w"], 1, H, S.eps)
    for layer, lay in enumerate(step.layers):
        qr = ora.rope_half(lay["q"], c, s, 1, QH, D, D // 2)
        kr = ora.rope_half(lay["k"], c, s, 1, KH, D, D // 2)
        caches[layer] = ora.kv_append("f32", kr, lay["v"], caches[layer], KH * D, step.capacity, pos, False, S.eps)
        residual, norm = ora.add_rms_norm(lay["attn_out"], state, lay["post_attn_w"], 1, H, S.eps)
        act = ora.swiglu(lay["gate"], lay["up"])
        nxt = step.layers[layer + 1]["input_w"] if layer + 1 < L else step.host["final_w"]
        state, norm = ora.add_rms_norm(lay["ffn_out"], residual, nxt, 1, H, S.eps)
        out["q_rot"].append(qr)
        out["k_rot"].append(kr)
        out["act"].append(act)
    out.update(state=state, residual=residual, norm=norm, kv=[np.array(x, copy=True) for x in caches])
    return out


def llama_same(got, exp, tag):
    for key in ("state", "residual", "norm"):
        same(f"{tag}: {key}", got[key], exp[key])
    for key in ("q_rot", "k_rot", "act", "kv"):
        for layer, (g, e) in enumerate(zip(got[key], exp[key])):
            same(f"{tag}: {key}[{layer}]", g, e)


def test_llama_resident_decode_eager_and_graph_replays(rt, ora):
    """SmolLM2-135M shapes, 30 layers, one sequence: three eager
    tokens at positions 0-2, then one recorded step replayed for positions
    3, 4 and 3 again with other tokens; the KV caches accumulate across
    steps and are compared whole after each."""
    step = LlamaDecodeStep(rt)
    caches = [np.zeros(step.cache_bytes, np.uint8) for _ in range(step.L)]
    r = wl.rng(77)
    try:
        for position in range(3):
            token = int(r.integers(0, step.S.vocab))
            say(f"llama eager token {token} at {position}")
            step.set_token(token, position)
            step.enqueue()
            rt.sync()
            llama_same(step.results(), llama_oracle(ora, step, token, position, caches), f"eager {position}")
        say("llama capture")
        step.capture()
        for i, position in enumerate((3, 4, 3)):
            token = int(r.integers(0, step.S.vocab))
            step.set_token(token, position)
            rt.memset(step.out["state"], 0, step.S.hidden * 4)   # eager work between replays
            rt.sync()
            say(f"llama replay {i}: token {token} at {position}")
            step.replay()
            rt.sync()
            llama_same(step.results(), llama_oracle(ora, step, token, position, caches), f"replay {i}")
    finally:
        step.close()


# ---------------------------------------------------------- Gemma prefill

def prefill_oracle(ora, ch, ids, positions, caches):
    S = ch.S
    T, H, QH, D, L, W = S.tokens, S.hidden, S.q_heads, S.head_dim, S.layers, S.ple_width
    h = ch.host
    state = ora.embed_q4_0(h["token_table"], ids, S.vocab, H, wl.f32_sqrt(H))
    ple = ora.ple(h["ple_table"], ids, h["ple_proj_in"], S.vocab, L, W, 16.0, wl.SQRT_2_RECIP)
    local = ora.rope_tables_gemma4(positions, D // 2, D, 1e4)
    glob = ora.rope_tables_gemma4(positions, D // 2, D, 1e6)
    out = {k: [] for k in ("norm", "q_rot", "k_rot", "ffn_norm", "product", "activated")}
    for layer, lay in enumerate(ch.layers):
        c, s = glob if S.is_global(layer) else local
        key = S.has_key(layer)
        out["norm"].append(ora.rms_norm(state, lay["attn_w"], T, H, S.eps))
        qo, ko = ora.qk_norm_rope(lay["q"], lay["k"], lay["qw"], lay["kw"], c, s, T, QH, key, D, D // 2, S.eps)
        if key:
            caches[layer] = ora.kv_append(ch.kv_format, ko, lay["v"], caches[layer], D, ch.capacity, positions, True,
                                          S.eps)
        _, residual = ora.rms_norm_residual(lay["attn_out"], lay["post_attn_w"], state, T, H, S.eps)
        out["ffn_norm"].append(ora.rms_norm(residual, lay["ffn_w"], T, H, S.eps))
        out["product"].append(ora.geglu(lay["gate"], lay["up"]))
        _, state = ora.rms_norm_residual(lay["ffn_out"], lay["post_ffn_w"], residual, T, H, S.eps)
        out["activated"].append(ora.geglu_offset(lay["ple_gate"], ple, layer * W, L * W, W, T))
        state = ora.rms_norm_add_scale(lay["ple_proj"], lay["post_norm_w"], state, lay["scale"][0], T, H, S.eps)
        out["q_rot"].append(qo)
        out["k_rot"].append(ko)
    # after the last layer `work` holds the stand-in PLE projection written by
    # the scale-by-one pass (the add-scale epilogue does not write it)
    out.update(state=state, ple=ple, residual=residual, work=ch.layers[-1]["ple_proj"],
               kv=[np.array(x, copy=True) for x in caches])
    return out


def prefill_same(got, exp, ch, tag, tree_norms=False):
    """Bit-identity everywhere; with tree_norms (the AUTO reduction) the plain
    norms' outputs (`norm`, `ffn_norm`, read only by the stand-in GEMMs) are
    held to 1e-5 relative instead."""
    for key in ("state", "ple", "residual", "work"):
        same(f"{tag}: {key}", got[key], exp[key])
    for key in ("q_rot", "product", "activated"):
        for layer, (g, e) in enumerate(zip(got[key], exp[key])):
            same(f"{tag}: {key}[{layer}]", g, e)
    for layer in range(ch.S.layers):
        if ch.S.has_key(layer):
            same(f"{tag}: k_rot[{layer}]", got["k_rot"][layer], exp["k_rot"][layer])
        same(f"{tag}: kv[{layer}]", got["kv"][layer], exp["kv"][layer])
    for key in ("norm", "ffn_norm"):
        for layer, (g, e) in enumerate(zip(got[key], exp[key])):
            if tree_norms:
                rel = np.max(np.abs(g - e) / np.maximum(np.abs(e), np.float32(1e-30)))
                assert rel <= 1e-5, (tag, key, layer, rel)
            else:
                same(f"{tag}: {key}[{layer}]", g, e)


def run_prefill(rt, ora, ch, tree_norms):
    S = ch.S
    r = wl.rng(31)
    caches = [np.zeros(ch.cache_bytes, np.uint8) for _ in range(S.layers)]
    chunk_a = (wl.token_ids(r, S.tokens, S.vocab), np.arange(S.tokens, dtype=u32))
    chunk_b = (wl.token_ids(r, S.tokens, S.vocab), np.arange(S.tokens, 2 * S.tokens, dtype=u32))
    chunk_a[0][:2] = [0, S.vocab - 1]
    try:
        say(f"prefill eager chunk A ({ch.kv_format} cache)")
        ch.set_chunk(*chunk_a)
        ch.enqueue()
        rt.sync()
        prefill_same(ch.results(), prefill_oracle(ora, ch, *chunk_a, caches), ch, "eager A", tree_norms)
        say("prefill capture")
        ch.capture()
        for i, which in enumerate("BAB"):
            ids, pos = chunk_a if which == "A" else chunk_b
            ch.set_chunk(ids, pos)
            rt.memset(ch.out["state"], 0, S.tokens * S.hidden * 4)   # eager work between replays
            rt.sync()
            say(f"prefill replay {i} chunk {which}")
            ch.replay()
            rt.sync()
            prefill_same(ch.results(), prefill_oracle(ora, ch, ids, pos, caches), ch, f"replay {i} ({which})",
                         tree_norms)
    finally:
        ch.close()


@pytest.mark.parametrize("kv_format", ["q8_0", "q4_0"])
def test_gemma_prefill_chunk_eager_and_graph_replays(rt, ora, kv_format):
    """T = 512 tokens, five layers (four sliding-window, one full; the last
    reads an earlier layer's KV, so it has no K head), a Q8_0 or Q4_0 KV cache
    with the fused V norm; chunk A at positions 0-511, then replays of chunks
    B (512-1023), A and B."""
    run_prefill(rt, ora, GemmaPrefillChunk(rt, PrefillShape(), kv_format=kv_format), tree_norms=False)


def test_gemma_prefill_chunk_under_auto_reduction(rt_auto, ora):
    """The library's default reduction: the cancelling epilogues, QK-norm and
    the V norm keep their bits; the two plain norms per layer take the tree
    sum (1e-5 relative).  F32 KV cache."""
    run_prefill(rt_auto, ora, GemmaPrefillChunk(rt_auto, PrefillShape(), kv_format="f32"), tree_norms=True)
