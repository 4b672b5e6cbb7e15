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


def kv_tie_blocks():
    """Two blocks whose encodings depend on the tie rules, with their bytes
    derived by hand from the reference's steps (kernels.metal:1222-1256):
    - Q8_0: max |v| = 127, so the scale is exactly 1 and every quotient v/s
      is v; Metal's round() takes halfway cases away from zero, so 2.5 -> 3,
      -2.5 -> -3, 0.5 -> 1, -0.5 -> -1, 126.5 -> 127 (half-even: 2, -2, 0, 0,
      126).
    - Q4_0: |v| = 4 at index 0 (-4) and index 1 (+4); the forward scan's
      strict > keeps the first, so the signed maximum is -4 and the scale
      -4 / -8 = 0.5 (f16 0x3800); codes int(v / 0.5 + 8.5) clamped to
      [0, 15]: -4 -> 0, 4 -> 15, and v_j = (j - 16) / 4 for j >= 2 ->
      int(j / 2 + 1 / 2) = (j + 1) // 2, clamped (the last maximum would give
      scale -0.5, 0xB800, and mirrored codes)."""
    q8 = np.zeros(32, np.float32)
    q8[:10] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5, 3.0]
    codes8 = [127, 3, -3, 1, -1, 2, -2, 127, -127, 3] + [0] * 22
    want8 = bytes([0x00, 0x3C]) + bytes((c & 0xFF) for c in codes8)
    q4 = np.array([-4.0, 4.0] + [(j - 16) / 4.0 for j in range(2, 32)], np.float32)
    codes4 = [0, 15] + [min((j + 1) // 2, 15) for j in range(2, 32)]
    want4 = bytes([0x00, 0x38]) + bytes(codes4[i] | (codes4[i + 16] << 4) for i in range(16))
    return q8, want8, q4, want4
