"""Batched Gemma decode step over the fused per-layer ops.

`GemmaDecodeStep` is the executor side of the drop-in: it enqueues, for B
sequences x 1 token, the path's ops in the order of the reference decode
encoder `encode_current_token` (crates/atlas-model/src/gemma4_executor.rs:
4123-4690):

    token embed Q4_0 x sqrt(h)              (:4145-4161)
    PLE gather + combine                    (:4162-4237)
    for each of the layers (:4238-4660):
        QK-RMSNorm + RoPE (local / global theta, 4:1)   (:4314-4325)
        post-attention RMSNorm + residual                (:4492-4506)
        GeGLU on the FFN width                           (:4527-4531)
        post-FFN RMSNorm + residual                      (:4543-4557)
        PLE gate: GELU(gate) * PLE layer slice           (:4596-4607)
        PLE RMSNorm + add + layer scale epilogue         (:4627-4641)

The GEMMs and attention between these ops are not part of this path; their
outputs (Q/K projections, attention output, FFN down output, PLE gate and
projection outputs) are seeded stand-in buffers, one set per layer.  The
residual stream `state` flows through every layer, so each op consumes the
previous op's result exactly as in the reference chain.

`enqueue()` issues one step eagerly on the runtime's stream; `capture()`
records the same chain once into a HIP graph (atlas_hip_graph_*) that
`replay()` submits in one call -- per-step inputs (token ids, RoPE tables)
live in device buffers, so a replay recomputes the whole step from them.
"""
from __future__ import annotations

import numpy as np

from . import workloads as wl
from .runtime import HipRuntime, rope_tables_gemma4


class GemmaDecodeStep:
    def __init__(self, rt: HipRuntime, shape: wl.DecodeShape = wl.DecodeShape(), seed: int = 5,
                 vocab: int | None = None):
        self.rt, self.S = rt, shape
        S = shape
        B, H, QH, D, F, L, W = S.batch, S.hidden, S.q_heads, S.head_dim, S.ffn, S.layers, S.ple_width
        self.vocab = vocab if vocab is not None else S.vocab
        r = wl.rng(seed)
        self.host = {
            "token_table": wl.q4_0_table(r, self.vocab, H),
            "ple_table": wl.q4_0_table(r, self.vocab, L * W),
            "ple_proj_in": wl.normal(r, B * L * W),
        }
        self.host["ids"], self.host["positions"] = self.draw_tokens(seed)
        self.layers = []
        for _ in range(L):
            self.layers.append({
                "q": wl.normal(r, B * QH * D), "k": wl.normal(r, B * D),
                "qw": wl.normal(r, D, 1.0, 0.1), "kw": wl.normal(r, D, 1.0, 0.1),
                "attn_out": wl.normal(r, B * H), "post_attn_w": wl.normal(r, H, 1.0, 0.1),
                "gate": wl.normal(r, B * F), "up": wl.normal(r, B * F),
                "ffn_out": wl.normal(r, B * H), "post_ffn_w": wl.normal(r, H, 1.0, 0.1),
                "ple_gate": wl.normal(r, B * W), "ple_proj": wl.normal(r, B * H),
                "post_norm_w": wl.normal(r, H, 1.0, 0.1),
                "scale": np.array([r.uniform(0.5, 1.5)], np.float32),
            })
        self.dev = {k: rt.upload(v) for k, v in self.host.items()}
        self._upload_tables()
        self.dlayers = [{k: rt.upload(v) for k, v in lay.items()} for lay in self.layers]
        self.out = {
            "state": rt.empty(B * H), "ple": rt.empty(B * L * W),
            "q_out": [rt.empty(B * QH * D) for _ in range(L)], "k_out": [rt.empty(B * D) for _ in range(L)],
            "ffn_act": [rt.empty(B * F) for _ in range(L)], "ple_act": [rt.empty(B * W) for _ in range(L)],
        }
        self.graph = None

    # -- per-step inputs (device buffers, so a captured graph reads new values)
    def draw_tokens(self, seed: int):
        r = wl.rng(10_000 + seed)
        ids = wl.token_ids(r, self.S.batch, self.vocab)
        pos = r.integers(0, self.S.max_position, self.S.batch, dtype=np.uint32)
        return ids, pos

    def _tables(self, positions):
        S = self.S
        half = S.head_dim // 2
        return (rope_tables_gemma4(positions, half, S.head_dim, 1e4),
                rope_tables_gemma4(positions, half, S.head_dim, 1e6))

    def _upload_tables(self):
        (lc, ls), (gc, gs) = self._tables(self.host["positions"])
        for name, arr in (("cos_local", lc), ("sin_local", ls), ("cos_global", gc), ("sin_global", gs)):
            if name in self.dev:
                self.dev[name].upload(arr)
            else:
                self.dev[name] = self.rt.upload(arr)

    def set_tokens(self, ids, positions) -> None:
        """New token ids / positions for the next step (host RoPE tables, as the
        reference computes them per token, gemma4_executor.rs:3293-3326)."""
        self.host["ids"] = np.ascontiguousarray(ids, np.uint32)
        self.host["positions"] = np.ascontiguousarray(positions, np.uint32)
        self.dev["ids"].upload(self.host["ids"])
        self._upload_tables()

    # -- the chain ---------------------------------------------------------
    def head_ops(self):
        """The step's two gathers, [(name, algorithmic bytes, launch)]:
        the Q4_0 token embedding x sqrt(hidden) and the PLE chain
        (gemma4_executor.rs:4145-4237)."""
        rt, S, d, o = self.rt, self.S, self.dev, self.out
        B, H, L, W = S.batch, S.hidden, S.layers, S.ple_width
        return [
            ("embed_q4_0", B * wl.q_row_bytes(H, False) + B * 4 + B * H * 4,
             lambda: rt.embed_q4_0(d["token_table"], d["ids"], o["state"], self.vocab, H, B, wl.f32_sqrt(H))),
            ("ple_q4_0", B * wl.q_row_bytes(L * W, False) + B * 4 + 2 * B * L * W * 4,
             lambda: rt.ple_q4_0(d["ple_table"], d["ids"], d["ple_proj_in"], o["ple"], self.vocab, L, W, B, 16.0,
                                 wl.SQRT_2_RECIP)),
        ]

    def layer_ops(self, layer: int):
        """One layer's six fused ops in the reference decode order
        (encode_current_token, gemma4_executor.rs:4123-4690),
        [(name, algorithmic bytes, launch)]."""
        rt, S, d, o = self.rt, self.S, self.dev, self.out
        B, H, QH, D, F, L, W = S.batch, S.hidden, S.q_heads, S.head_dim, S.ffn, S.layers, S.ple_width
        lay = self.dlayers[layer]
        g = S.is_global(layer)
        cos, sin = (d["cos_global"], d["sin_global"]) if g else (d["cos_local"], d["sin_local"])
        rms_res = 3 * B * H * 4 + H * 4
        return [
            ("qk_norm_rope", 2 * B * (QH + 1) * D * 4 + 2 * B * (D // 2) * 4 + 2 * D * 4,
             lambda: rt.qk_norm_rope(lay["q"], lay["k"], lay["qw"], lay["kw"], cos, sin, o["q_out"][layer],
                                     o["k_out"][layer], B, QH, 1, D, D // 2, S.eps)),
            ("rms_residual_attn", rms_res,
             lambda: rt.rms_norm_residual(lay["attn_out"], lay["post_attn_w"], o["state"], None, o["state"], B, H,
                                          S.eps)),
            ("geglu", 3 * B * F * 4, lambda: rt.geglu(lay["gate"], lay["up"], o["ffn_act"][layer], B * F)),
            ("rms_residual_ffn", rms_res,
             lambda: rt.rms_norm_residual(lay["ffn_out"], lay["post_ffn_w"], o["state"], None, o["state"], B, H,
                                          S.eps)),
            ("geglu_offset_ple", 3 * B * W * 4,
             lambda: rt.geglu_offset(lay["ple_gate"], o["ple"], o["ple_act"][layer], layer * W, L * W, W, B)),
            ("rms_add_scale_ple", 3 * B * H * 4 + H * 4 + 4,
             lambda: rt.rms_norm_add_scale(lay["ple_proj"], lay["post_norm_w"], o["state"], lay["scale"], B, H,
                                           S.eps)),
        ]

    def enqueue(self) -> None:
        for _, _, launch in self.head_ops():
            launch()
        for layer in range(self.S.layers):
            for _, _, launch in self.layer_ops(layer):
                launch()

    def capture(self) -> int:
        """Record one step into a HIP graph (kept on the object)."""
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

    # -- accounting --------------------------------------------------------
    def written_bytes(self) -> dict:
        """Bytes each op writes (its outputs once), by op name."""
        S = self.S
        B, H, QH, D, F, L, W = S.batch, S.hidden, S.q_heads, S.head_dim, S.ffn, S.layers, S.ple_width
        return {"embed_q4_0": B * H * 4, "ple_q4_0": B * L * W * 4, "qk_norm_rope": B * (QH + 1) * D * 4,
                "rms_residual_attn": B * H * 4, "geglu": B * F * 4, "rms_residual_ffn": B * H * 4,
                "geglu_offset_ple": B * W * 4, "rms_add_scale_ple": B * H * 4}

    def bytes_per_layer(self) -> int:
        """Algorithmic HBM bytes of one layer's six ops (inputs once, outputs once)."""
        return sum(b for _, b, _ in self.layer_ops(0))

    def bytes_per_step(self) -> int:
        return sum(b for _, b, _ in self.head_ops()) + self.S.layers * self.bytes_per_layer()

    def results(self) -> dict:
        S = self.S
        o = self.out
        return {"state": o["state"].download(S.batch * S.hidden), "ple": o["ple"].download(),
                "q_out": [b.download() for b in o["q_out"]], "k_out": [b.download() for b in o["k_out"]],
                "ffn_act": [b.download() for b in o["ffn_act"]], "ple_act": [b.download() for b in o["ple_act"]]}
