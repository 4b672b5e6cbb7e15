"""Two more executor chains over the fused ops, beside the Gemma decode step
(decode.py): the Llama resident decode token and the Gemma layer-major
prefill chunk.  Each enqueues the path's ops in the reference executor's
order, with seeded stand-in buffers for the GEMM, attention and matvec
outputs between them (outside this path); per-step inputs (token ids,
positions, RoPE tables) live in device buffers, so `capture()` records a
step once and `replay()` recomputes it from new inputs.

LlamaDecodeStep -- `ResidentExecutor::forward_token`
(crates/atlas-model/src/executor.rs:1042-1429), one sequence, one token:

    embedding_lookup_f32                          (:1062-1074)
    rms_norm_decode (layer 0 input_layernorm)     (:1080-1089)
    for each layer:
        RoPE on Q and K: the half_to_interleaved / rope_f32 /
        interleaved_to_half dispatches per tensor  (:1120-1166)
        kv_append_decode_f32                       (:1167-1177)
        vector_add (state + o_proj) + rms_norm_decode (post_attention_layernorm)
                                                   (:1258-1286)
        silu_f32 + vector_multiply_f32             (:1318-1327)
        vector_add (residual + down) and the next layer's input
        rms_norm_decode (or model.norm after the last layer)
                                                   (:1343-1346, :1080-1089, :1353-1362)

  so per layer: rope_half_qk, kv_append f32, add_rms_norm, swiglu,
  add_rms_norm -- the closing residual add fuses with the norm that reads it.

GemmaPrefillChunk -- the layer-major prefill of one chunk
(`encode_prefill_layer_major_layer`, crates/atlas-model/src/
gemma4_executor.rs:3694-4121; chunk size GEMMA4_PREFILL_BATCH_CAPACITY,
:23), after the chunk's token embedding and PLE gather (:3533-3631):

    embedding_lookup_q4_0 x sqrt(h) and the PLE chain      (:3533-3631)
    for each layer:
        rms_norm (attn_norm)                               (:3731-3737)
        QK-RMSNorm + RoPE, has_key on KV-source layers      (:3799-3825)
        V RMSNorm + KV append (KV-source layers)            (:3826-3850)
        rms_norm in place on work (post_attention_norm),
        residual = state + work                              (:3952-3967)
        rms_norm (ffn_norm)                                  (:3970-3975)
        gelu_multiply                                        (:4007-4016)
        rms_norm in place on work (post_ffw_norm),
        state = residual + work                              (:4029-4044)
        gelu + vector_multiply_offset_batch (PLE slice)      (:4063-4081)
        rms_norm in place on work (post_norm), state += work,
        state *= layer_output_scale                          (:4094-4119)

  The stand-in GEMM outputs are written into `work` by a scale-by-one pass
  (exact for every finite value), as the GEMM writes it, because the
  residual epilogues normalise `work` in place.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import workloads as wl
from .runtime import HipRuntime, rope_tables_gemma4, rope_tables_llama


class LlamaDecodeStep:
    """One decode token of the Llama resident executor at SmolLM2-135M shapes
    (hidden 576, 9 Q heads, 3 KV heads, head_dim
    64, FFN 1536, vocab 49152, eps 1e-5, theta 1e4)."""

    def __init__(self, rt: HipRuntime, shape: wl.SmolShape = wl.SmolShape(), layers: int = 30,
                 capacity: int = 128, seed: int = 11):
        self.rt, self.S, self.L, self.capacity = rt, shape, layers, capacity
        S = shape
        H, QH, KH, D, F = S.hidden, S.q_heads, S.kv_heads, S.head_dim, S.ffn
        r = wl.rng(seed)
        self.kv_width = KH * D
        self.host = {"table": wl.normal(r, S.vocab * H, 0.0, 0.02),
                     "final_w": wl.normal(r, H, 1.0, 0.1)}
        self.layers = []
        for _ in range(layers):
            self.layers.append({
                "input_w": wl.normal(r, H, 1.0, 0.1),
                "q": wl.normal(r, QH * D), "k": wl.normal(r, KH * D), "v": wl.normal(r, KH * D),
                "attn_out": wl.normal(r, H), "post_attn_w": wl.normal(r, H, 1.0, 0.1),
                "gate": wl.normal(r, F), "up": wl.normal(r, F), "ffn_out": wl.normal(r, H),
            })
        self.dev = {k: rt.upload(v) for k, v in self.host.items()}
        self.dlayers = [{k: rt.upload(v) for k, v in lay.items()} for lay in self.layers]
        self.dev["token"] = rt.empty(1, np.uint32)
        self.dev["position"] = rt.empty(1, np.uint32)
        self.dev["cos"], self.dev["sin"] = rt.empty(D // 2), rt.empty(D // 2)
        self.cache_bytes = 2 * capacity * self.kv_width * 4
        self.out = {
            "state": rt.empty(H), "residual": rt.empty(H), "norm": rt.empty(H),
            "q_rot": [rt.empty(QH * D) for _ in range(layers)], "k_rot": [rt.empty(KH * D) for _ in range(layers)],
            "act": [rt.empty(F) for _ in range(layers)],
            "kv": [rt.alloc(self.cache_bytes, np.uint8) for _ in range(layers)],
        }
        for c in self.out["kv"]:
            rt.memset(c, 0, self.cache_bytes)
        self.graph = None

    def set_token(self, token: int, position: int) -> None:
        """The token and its position for the next step; the host RoPE row for
        that position (write_rope_tables, executor.rs:632-647)."""
        self.token, self.position = int(token), int(position)
        self.dev["token"].upload(np.array([token], np.uint32))
        self.dev["position"].upload(np.array([position], np.uint32))
        c, s = rope_tables_llama(np.array([position], np.uint32), self.S.head_dim, self.S.theta)
        self.dev["cos"].upload(c)
        self.dev["sin"].upload(s)

    def enqueue(self) -> None:
        rt, S, d, o = self.rt, self.S, self.dev, self.out
        H, QH, KH, D, F = S.hidden, S.q_heads, S.kv_heads, S.head_dim, S.ffn
        rt.embed_f32(d["table"], d["token"], o["state"], S.vocab, H, 1)
        rt.rms_norm(o["state"], self.dlayers[0]["input_w"], o["norm"], 1, H, S.eps)
        for layer, lay in enumerate(self.dlayers):
            rt.rope_half_qk(lay["q"], lay["k"], d["cos"], d["sin"], o["q_rot"][layer], o["k_rot"][layer], 1, QH, KH,
                            D, D // 2)
            rt.kv_append("f32", o["k_rot"][layer], lay["v"], o["kv"][layer], self.kv_width, self.capacity,
                         d["position"], 1, False, S.eps)
            # residual = state + o_proj(attention); norm = RMSNorm(residual)
            rt.add_rms_norm(lay["attn_out"], o["state"], lay["post_attn_w"], o["residual"], o["norm"], 1, H, S.eps)
            rt.swiglu(lay["gate"], lay["up"], o["act"][layer], F)
            # state = residual + down(product); norm = the next layer's input norm (model.norm after the last)
            nxt = self.dlayers[layer + 1]["input_w"] if layer + 1 < self.L else d["final_w"]
            rt.add_rms_norm(lay["ffn_out"], o["residual"], nxt, o["state"], o["norm"], 1, H, S.eps)

    def capture(self) -> int:
        if self.graph is not None:
            self.rt.graph_destroy(self.graph)
        self.rt.graph_begin()
        try:
            self.enqueue()
        finally:
            graph = self.rt.graph_end()
        self.graph = graph
        return graph

    def replay(self) -> None:
        self.rt.graph_launch(self.graph)

    def close(self) -> None:
        if self.graph is not None:
            self.rt.graph_destroy(self.graph)
            self.graph = None

    def results(self) -> dict:
        o = self.out
        return {"state": o["state"].download(), "residual": o["residual"].download(), "norm": o["norm"].download(),
                "q_rot": [b.download() for b in o["q_rot"]], "k_rot": [b.download() for b in o["k_rot"]],
                "act": [b.download() for b in o["act"]],
                "kv": [b.download(self.cache_bytes, np.uint8) for b in o["kv"]]}


@dataclass(frozen=True)
class PrefillShape:
    """One layer-major prefill chunk at the Gemma-4-E2B-like layer shape."""

    tokens: int = 512          # GEMMA4_PREFILL_BATCH_CAPACITY (gemma4_executor.rs:23)
    layers: int = 5            # four sliding-window layers, then a full one (4:1)
    hidden: int = 1536
    q_heads: int = 8
    head_dim: int = 256
    ffn: int = 6144
    ple_width: int = 256
    vocab: int = 8192
    eps: float = 1e-6

    def is_global(self, layer: int) -> bool:
        return layer % 5 == 4

    def has_key(self, layer: int) -> bool:
        # the last layer reads an earlier layer's KV cache (kv_sources,
        # gemma4_executor.rs:1538,3730), so it has no K head of its own
        return layer != self.layers - 1


class GemmaPrefillChunk:
    def __init__(self, rt: HipRuntime, shape: PrefillShape = PrefillShape(), capacity: int = 1024,
                 kv_format: str = "q8_0", seed: int = 13):
        self.rt, self.S, self.capacity, self.kv_format = rt, shape, capacity, kv_format
        S = shape
        T, H, QH, D, F, L, W = S.tokens, S.hidden, S.q_heads, S.head_dim, S.ffn, S.layers, S.ple_width
        r = wl.rng(seed)
        self.host = {"token_table": wl.q4_0_table(r, S.vocab, H), "ple_table": wl.q4_0_table(r, S.vocab, L * W),
                     "ple_proj_in": wl.normal(r, T * L * W)}
        self.layers = []
        for _ in range(L):
            self.layers.append({
                "attn_w": wl.normal(r, H, 1.0, 0.1), "q": wl.normal(r, T * QH * D), "k": wl.normal(r, T * D),
                "v": wl.normal(r, T * D), "qw": wl.normal(r, D, 1.0, 0.1), "kw": wl.normal(r, D, 1.0, 0.1),
                "attn_out": wl.normal(r, T * H), "post_attn_w": wl.normal(r, H, 1.0, 0.1),
                "ffn_w": wl.normal(r, H, 1.0, 0.1), "gate": wl.normal(r, T * F), "up": wl.normal(r, T * F),
                "ffn_out": wl.normal(r, T * H), "post_ffn_w": wl.normal(r, H, 1.0, 0.1),
                "ple_gate": wl.normal(r, T * W), "ple_proj": wl.normal(r, T * H),
                "post_norm_w": wl.normal(r, H, 1.0, 0.1),
                "scale": np.array([r.uniform(0.5, 1.5)], np.float32),
            })
        self.dev = {k: rt.upload(v) for k, v in self.host.items()}
        self.dlayers = [{k: rt.upload(v) for k, v in lay.items()} for lay in self.layers]
        self.dev["ids"] = rt.empty(T, np.uint32)
        self.dev["positions"] = rt.empty(T, np.uint32)
        for name in ("cos_local", "sin_local", "cos_global", "sin_global"):
            self.dev[name] = rt.empty(T * (D // 2))
        self.cache_bytes = 2 * capacity * _kv_row_bytes(kv_format, D)
        self.out = {
            "state": rt.empty(T * H), "ple": rt.empty(T * L * W), "norm": [rt.empty(T * H) for _ in range(L)],
            "residual": rt.empty(T * H), "work": rt.empty(T * H),
            "q_rot": [rt.empty(T * QH * D) for _ in range(L)], "k_rot": [rt.empty(T * D) for _ in range(L)],
            "ffn_norm": [rt.empty(T * H) for _ in range(L)], "product": [rt.empty(T * F) for _ in range(L)],
            "activated": [rt.empty(T * W) for _ in range(L)],
            "kv": [rt.alloc(self.cache_bytes, np.uint8) for _ in range(L)],
        }
        for c in self.out["kv"]:
            rt.memset(c, 0, self.cache_bytes)
        self.graph = None

    def set_chunk(self, ids, positions) -> None:
        """The chunk's token ids and positions; host RoPE tables for them
        (gemma4_executor.rs:3494-3519)."""
        S = self.S
        self.ids = np.ascontiguousarray(ids, np.uint32)
        self.positions = np.ascontiguousarray(positions, np.uint32)
        self.dev["ids"].upload(self.ids)
        self.dev["positions"].upload(self.positions)
        half = S.head_dim // 2
        for kind, theta in (("local", 1e4), ("global", 1e6)):
            c, s = rope_tables_gemma4(self.positions, half, S.head_dim, theta)
            self.dev[f"cos_{kind}"].upload(c)
            self.dev[f"sin_{kind}"].upload(s)

    def enqueue(self) -> None:
        rt, S, d, o = self.rt, self.S, self.dev, self.out
        T, H, QH, D, F, L, W = S.tokens, S.hidden, S.q_heads, S.head_dim, S.ffn, S.layers, S.ple_width
        rt.embed_q4_0(d["token_table"], d["ids"], o["state"], S.vocab, H, T, wl.f32_sqrt(H))
        rt.ple_q4_0(d["ple_table"], d["ids"], d["ple_proj_in"], o["ple"], S.vocab, L, W, T, 16.0, wl.SQRT_2_RECIP)
        for layer, lay in enumerate(self.dlayers):
            kind = "global" if S.is_global(layer) else "local"
            key = S.has_key(layer)
            rt.rms_norm(o["state"], lay["attn_w"], o["norm"][layer], T, H, S.eps)
            rt.qk_norm_rope(lay["q"], lay["k"], lay["qw"], lay["kw"], d[f"cos_{kind}"], d[f"sin_{kind}"],
                            o["q_rot"][layer], o["k_rot"][layer], T, QH, 1 if key else 0, D, D // 2, S.eps)
            if key:
                rt.kv_append(self.kv_format, o["k_rot"][layer], lay["v"], o["kv"][layer], D, self.capacity,
                             d["positions"], T, True, S.eps)
            rt.scale(lay["attn_out"], 1.0, o["work"], T * H)
            rt.rms_norm_residual(o["work"], lay["post_attn_w"], o["state"], o["work"], o["residual"], T, H, S.eps)
            rt.rms_norm(o["residual"], lay["ffn_w"], o["ffn_norm"][layer], T, H, S.eps)
            rt.geglu(lay["gate"], lay["up"], o["product"][layer], T * F)
            rt.scale(lay["ffn_out"], 1.0, o["work"], T * H)
            rt.rms_norm_residual(o["work"], lay["post_ffn_w"], o["residual"], o["work"], o["state"], T, H, S.eps)
            rt.geglu_offset(lay["ple_gate"], o["ple"], o["activated"][layer], layer * W, L * W, W, T)
            rt.scale(lay["ple_proj"], 1.0, o["work"], T * H)
            rt.rms_norm_add_scale(o["work"], lay["post_norm_w"], o["state"], lay["scale"], T, H, S.eps)

    def capture(self) -> int:
        if self.graph is not None:
            self.rt.graph_destroy(self.graph)
        self.rt.graph_begin()
        try:
            self.enqueue()
        finally:
            graph = self.rt.graph_end()
        self.graph = graph
        return graph

    def replay(self) -> None:
        self.rt.graph_launch(self.graph)

    def close(self) -> None:
        if self.graph is not None:
            self.rt.graph_destroy(self.graph)
            self.graph = None

    def results(self) -> dict:
        o = self.out
        per_layer = ("norm", "q_rot", "k_rot", "ffn_norm", "product", "activated")
        res = {k: o[k].download() for k in ("state", "ple", "residual", "work")}
        res.update({k: [b.download() for b in o[k]] for k in per_layer})
        res["kv"] = [b.download(self.cache_bytes, np.uint8) for b in o["kv"]]
        return res


def _kv_row_bytes(fmt: str, width: int) -> int:
    """Bytes of one cache row: f32, or 34-byte Q8_0 / 18-byte Q4_0 blocks of 32."""
    return width * 4 if fmt == "f32" else (width // 32) * (34 if fmt == "q8_0" else 18)
