"""Synthetic workloads for the BASELINE configurations (C1-C5).

Seeded numpy generators (PCG64) for activations, weights, token ids,
positions and packed Q4_0 / Q6_K tables.  Shapes follow the benchmark
configurations; nothing here touches the GPU.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

f32 = np.float32

SQRT_2_RECIP = np.float32(1.0) / np.sqrt(np.float32(2.0))  # 2.0f32.sqrt().recip() (gemma4_executor.rs:1888)


def f32_sqrt(x: float) -> np.float32:
    """(x as f32).sqrt() -- correctly rounded in f32 (embed_scale, gemma4_executor.rs:1886)."""
    return np.sqrt(np.float32(x))


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def normal(r: np.random.Generator, shape, mean=0.0, std=1.0) -> np.ndarray:
    x = r.standard_normal(shape, dtype=np.float32)
    if std != 1.0:
        x = x * np.float32(std)
    if mean != 0.0:
        x = x + np.float32(mean)
    return x.astype(np.float32, copy=False)


def token_ids(r: np.random.Generator, tokens: int, vocab: int) -> np.ndarray:
    return r.integers(0, vocab, size=tokens, dtype=np.uint32)


def q4_0_table(r: np.random.Generator, vocab: int, hidden: int) -> np.ndarray:
    """Q4_0 rows [vocab, hidden/32 blocks x 18 B]: f16 d ~ U(0.001, 0.05) (IEEE RNE) + 16 random bytes."""
    blocks = hidden // 32
    table = np.frombuffer(r.bytes(vocab * blocks * 18), dtype=np.uint8).reshape(vocab, blocks, 18).copy()
    d = r.uniform(0.001, 0.05, size=(vocab, blocks)).astype(np.float16)
    table[:, :, 0:2] = d.view(np.uint8).reshape(vocab, blocks, 2)
    return table.reshape(-1)


def q6_k_table(r: np.random.Generator, vocab: int, hidden: int) -> np.ndarray:
    """Q6_K rows [vocab, hidden/256 super-blocks x 210 B]: random ql/qh bytes, random int8
    sub-scales, finite f16 d ~ U(1e-4, 2e-3) (IEEE RNE)."""
    blocks = hidden // 256
    table = np.frombuffer(r.bytes(vocab * blocks * 210), dtype=np.uint8).reshape(vocab, blocks, 210).copy()
    d = r.uniform(1e-4, 2e-3, size=(vocab, blocks)).astype(np.float16)
    table[:, :, 208:210] = d.view(np.uint8).reshape(vocab, blocks, 2)
    return table.reshape(-1)


def q8_0_table(r: np.random.Generator, vocab: int, hidden: int) -> np.ndarray:
    """Q8_0 rows [vocab, hidden/32 blocks x 34 B]: f16 d ~ U(0.001, 0.05) (IEEE RNE) + 32 random int8."""
    blocks = hidden // 32
    table = np.frombuffer(r.bytes(vocab * blocks * 34), dtype=np.uint8).reshape(vocab, blocks, 34).copy()
    d = r.uniform(0.001, 0.05, size=(vocab, blocks)).astype(np.float16)
    table[:, :, 0:2] = d.view(np.uint8).reshape(vocab, blocks, 2)
    return table.reshape(-1)


def q_row_bytes(hidden: int, q6: bool) -> int:
    return (hidden // 256) * 210 if q6 else (hidden // 32) * 18


@dataclass(frozen=True)
class GemmaLayerShape:
    """C3: Gemma-4-E2B-like layer ops at T tokens."""

    tokens: int = 4096
    hidden: int = 1536
    q_heads: int = 8
    head_dim: int = 256
    ffn: int = 6144
    eps: float = 1e-6
    theta_local: float = 1e4
    theta_global: float = 1e6


@dataclass(frozen=True)
class QuantGatherShape:
    """C4: quantized embedding + PLE gathers."""

    tokens: int = 4096
    vocab: int = 262144
    hidden: int = 1536
    ple_layers: int = 35
    ple_width: int = 256


@dataclass(frozen=True)
class LlamaPrefillShape:
    """C2: SmolLM2-1.7B-shaped FP16 prefill."""

    tokens: int = 2048
    hidden: int = 2048
    heads: int = 32
    head_dim: int = 64
    ffn: int = 8192
    eps: float = 1e-5
    theta: float = 130000.0


@dataclass(frozen=True)
class SmolShape:
    """C1: SmolLM2-135M-shaped FP32 ops."""

    tokens: int = 128
    hidden: int = 576
    q_heads: int = 9
    kv_heads: int = 3
    head_dim: int = 64
    ffn: int = 1536
    vocab: int = 49152
    eps: float = 1e-5
    theta: float = 1e4


@dataclass(frozen=True)
class DecodeShape:
    """C5: batched decode, 256 sequences x 1 token, 35 layers."""

    batch: int = 256
    layers: int = 35
    hidden: int = 1536
    q_heads: int = 8
    head_dim: int = 256
    ffn: int = 6144
    vocab: int = 262144
    ple_width: int = 256
    max_position: int = 131072
    eps: float = 1e-6

    def is_global(self, layer: int) -> bool:
        # local/global interleaved 4:1 (E2B: 28 sliding-window + 7 full layers)
        return layer % 5 == 4


def sqrt_f32(x: float) -> float:
    return float(np.sqrt(np.float32(x)))


def bytes_gb(n: float) -> float:
    return n / 1e9


__all__ = [
    "SQRT_2_RECIP", "f32_sqrt", "rng", "normal", "token_ids", "q4_0_table", "q6_k_table", "q_row_bytes",
    "GemmaLayerShape", "QuantGatherShape", "LlamaPrefillShape", "SmolShape", "DecodeShape", "sqrt_f32", "math",
]
