"""Inputs for the RMS-folded Q4_0 projection tests.

`reference_*` restate the seeded generators of the reference's own parity
test (crates/atlas-metal/tests/matvec_rms_fused_parity.rs:16-49) so the GPU
is checked on the same inputs under the same contract (max-abs < 1e-3
against the normalise-then-matvec oracle).  `random_q4_0` builds Q4_0 rows
with IEEE-encoded f16 scales for the shape and tolerance tests.
"""
import numpy as np

f32 = np.float32


class Lcg:
    """next_u32 / next_f32 of the reference test (state * 1664525 + 1013904223 mod 2^32)."""

    def __init__(self, state: int):
        self.state = state & 0xFFFFFFFF

    def next_u32(self) -> int:
        self.state = (self.state * 1_664_525 + 1_013_904_223) & 0xFFFFFFFF
        return self.state

    def next_f32(self) -> np.float32:
        return f32(self.next_u32() >> 8) / f32(1 << 24)


def reference_fill_f32(n: int, lcg: Lcg) -> np.ndarray:
    return np.array([(lcg.next_f32() - f32(0.5)) * f32(2.0) for _ in range(n)], dtype=f32)


def reference_fill_rms_weight(n: int, lcg: Lcg) -> np.ndarray:
    return np.array([f32(0.5) + lcg.next_f32() for _ in range(n)], dtype=f32)


def reference_q4_weights(rows: int, blocks: int) -> np.ndarray:
    """build_q4_weights: block i has 16-bit scale bits round((0.005 + (i % 101) * 0.0003) * 32768)
    (f32 arithmetic, the bits used as-is) and bytes nibble | nibble << 4 with
    nibble = (i * 7 + j * 13) % 16."""
    n = rows * blocks
    i = np.arange(n)
    scale = f32(0.005) + np.fmod(i.astype(f32), f32(101.0)) * f32(0.0003)
    bits = np.floor(scale.astype(np.float64) * 32768.0 + 0.5).astype(np.uint16)  # round half away (positive)
    out = np.zeros((n, 18), np.uint8)
    out[:, 0] = bits & 0xFF
    out[:, 1] = bits >> 8
    j = np.arange(16)
    nib = ((i[:, None] * 7 + j[None, :] * 13) % 16).astype(np.uint8)
    out[:, 2:] = nib | (nib << 4)
    return out.reshape(-1)


def random_q4_0(r: np.random.Generator, rows: int, input_width: int) -> np.ndarray:
    blocks = input_width // 32
    w = np.frombuffer(r.bytes(rows * blocks * 18), np.uint8).reshape(rows, blocks, 18).copy()
    d = r.uniform(0.002, 0.03, size=(rows, blocks)).astype(np.float16)
    w[:, :, 0:2] = d.view(np.uint8).reshape(rows, blocks, 2)
    return w.reshape(-1)


def q4_0_dequant_numpy(weights: np.ndarray, rows: int, input_width: int) -> np.ndarray:
    """Independent vectorised Q4_0 decode from the format definition
    (crates/atlas-core/src/gguf.rs:418-429): value j < 16 = (low nibble of
    byte j - 8) * d, value j + 16 = (high nibble of byte j - 8) * d."""
    blocks = input_width // 32
    b = weights.reshape(rows, blocks, 18)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    q = b[:, :, 2:].astype(np.int64)
    vals = np.concatenate([(q & 15) - 8, (q >> 4) - 8], axis=2).astype(np.float64)
    return (vals * d[:, :, None]).reshape(rows, input_width)
