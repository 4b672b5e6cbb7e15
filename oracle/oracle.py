"""ctypes binding of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of Atlas's operators used as the parity checker by
tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py.  The
product (atlas_amd / libatlas_hip_ops.so) never imports this module.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_size_t, c_uint16, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

P = c_void_p
SZ = c_size_t
F = c_float

_SIGS = {
    "oracle_f16_to_f32": ([c_uint16], c_float),
    "oracle_f32_to_f16_rne": ([c_float], c_uint16),
    "oracle_f16_to_f32_n": ([P, P, SZ], None),
    "oracle_f32_to_f16_rne_n": ([P, P, SZ], None),
    "oracle_expf": ([F], c_float),
    "oracle_tanhf": ([F], c_float),
    "oracle_silu": ([F], c_float),
    "oracle_gelu_tanh": ([F], c_float),
    "oracle_inverse_rms": ([P, SZ, F], c_float),
    "oracle_rms_norm_f32": ([P, P, P, SZ, SZ, F], None),
    "oracle_rms_norm_residual_f32": ([P, P, P, P, P, SZ, SZ, F], None),
    "oracle_add_rms_norm_f32": ([P, P, P, P, P, SZ, SZ, F], None),
    "oracle_rms_norm_add_scale_f32": ([P, P, P, F, SZ, SZ, F], None),
    "oracle_rms_norm_groups_stable_f32": ([P, P, SZ, SZ, F], None),
    "oracle_ple_projection_f16": ([P, P, P, P, SZ, SZ, SZ, F, F], None),
    "oracle_rms_norm_f16": ([P, P, P, SZ, SZ, F], None),
    "oracle_add_rms_norm_f16": ([P, P, P, P, P, SZ, SZ, F], None),
    "oracle_gemma4_rope_angle": ([SZ, SZ, SZ, F, F], c_float),
    "oracle_rope_tables_gemma4": ([P, SZ, SZ, SZ, F, P, P, P], None),
    "oracle_rope_tables_llama": ([P, SZ, SZ, F, P, P], None),
    "oracle_rope_interleaved_f32": ([P, SZ, SZ, P, P, P], None),
    "oracle_rope_half_f32": ([P, P, P, P, SZ, SZ, SZ, SZ], None),
    "oracle_rope_half_f16": ([P, P, P, P, SZ, SZ, SZ, SZ], None),
    "oracle_qk_norm_rope_f32": ([P, P, P, P, P, P, P, P, SZ, SZ, c_int, SZ, SZ, F], None),
    "oracle_silu_f32": ([P, P, SZ], None),
    "oracle_gelu_f32": ([P, P, SZ], None),
    "oracle_swiglu_f32": ([P, P, P, SZ], None),
    "oracle_swiglu_f16": ([P, P, P, SZ], None),
    "oracle_geglu_f32": ([P, P, P, SZ], None),
    "oracle_geglu_offset_f32": ([P, P, P, SZ, SZ, SZ, SZ], None),
    "oracle_dequant_q4_0_block": ([P, P], None),
    "oracle_dequant_q8_0_block": ([P, P], None),
    "oracle_dequant_q6_k_block": ([P, P], None),
    "oracle_dequant_q6_k_block_llama_order": ([P, P], None),
    "oracle_embed_f32": ([P, P, P, SZ, SZ, SZ], None),
    "oracle_embed_q4_0": ([P, P, P, SZ, SZ, SZ, F], None),
    "oracle_embed_q8_0": ([P, P, P, SZ, SZ, SZ, F], None),
    "oracle_embed_q6_k": ([P, P, P, SZ, SZ, SZ, F], None),
    "oracle_ple_q4_0": ([P, P, P, P, SZ, SZ, SZ, SZ, F, F], None),
    "oracle_ple_q6_k": ([P, P, P, P, SZ, SZ, SZ, SZ, F, F], None),
    "oracle_combine_ple": ([P, P, P, SZ], None),
    "oracle_matvec_q4_0_rms_ref": ([P, P, P, SZ, SZ, F, P], None),
    "oracle_matvec_q4_0_rms_f64": ([P, P, P, SZ, SZ, F, P, P], None),
    "oracle_encode_q8_0_block": ([P, P], None),
    "oracle_encode_q4_0_block": ([P, P], None),
    "oracle_kv_append": ([c_int, P, P, P, SZ, SZ, P, SZ, c_int, F], None),
    "oracle_add_f32": ([P, P, P, SZ], None),
    "oracle_multiply_f32": ([P, P, P, SZ], None),
    "oracle_scale_f32": ([P, F, P, SZ], None),
    "oracle_tanh_precise": ([F], c_float),
    "oracle_softcap_f32": ([P, P, SZ, F], None),
    "oracle_argmax_f32": ([P, SZ], ctypes.c_uint32),
    "oracle_softcap_argmax_rows": ([P, P, SZ, SZ, F], None),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built (make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


f32 = np.float32
u16 = np.uint16
u32 = np.uint32
u8 = np.uint8


def f16_to_f32(bits):
    b = _c(bits, u16)
    out = np.empty(b.shape, f32)
    lib().oracle_f16_to_f32_n(_p(b), _p(out), b.size)
    return out


def f32_to_f16(values):
    v = _c(values, f32)
    out = np.empty(v.shape, u16)
    lib().oracle_f32_to_f16_rne_n(_p(v), _p(out), v.size)
    return out


def rms_norm(x, w, rows, hidden, eps):
    x, w = _c(x, f32), _c(w, f32)
    out = np.empty(rows * hidden, f32)
    lib().oracle_rms_norm_f32(_p(x), _p(w), _p(out), rows, hidden, eps)
    return out


def rms_norm_residual(x, w, residual, rows, hidden, eps):
    x, w, r = _c(x, f32), _c(w, f32), _c(residual, f32)
    n = np.empty(rows * hidden, f32)
    out = np.empty(rows * hidden, f32)
    lib().oracle_rms_norm_residual_f32(_p(x), _p(w), _p(r), _p(n), _p(out), rows, hidden, eps)
    return n, out


def add_rms_norm(x, residual, w, rows, hidden, eps):
    x, r, w = _c(x, f32), _c(residual, f32), _c(w, f32)
    rs = np.empty(rows * hidden, f32)
    out = np.empty(rows * hidden, f32)
    lib().oracle_add_rms_norm_f32(_p(x), _p(r), _p(w), _p(rs), _p(out), rows, hidden, eps)
    return rs, out


def rms_norm_add_scale(x, w, state, scale, rows, hidden, eps):
    x, w = _c(x, f32), _c(w, f32)
    st = np.array(state, dtype=f32, copy=True).reshape(-1)
    lib().oracle_rms_norm_add_scale_f32(_p(x), _p(w), _p(st), scale, rows, hidden, eps)
    return st


def rms_norm_groups_stable(values, w, width, groups, eps):
    v = np.array(values, dtype=f32, copy=True).reshape(-1)
    w = _c(w, f32)
    lib().oracle_rms_norm_groups_stable_f32(_p(v), _p(w), width, groups, eps)
    return v


def ple_projection_f16(x, weights, norm_weight, hidden, width, groups, scale, eps):
    """matvec_f16 * scale, then the stable group norm (gemma4_executor.rs:4184-4214)."""
    x, weights, nw = _c(x, f32), _c(weights, u16), _c(norm_weight, f32)
    out = np.empty(groups * width, f32)
    lib().oracle_ple_projection_f16(_p(x), _p(weights), _p(nw), _p(out), hidden, width, groups, scale, eps)
    return out


def rms_norm_f16(x, w, rows, hidden, eps):
    x, w = _c(x, u16), _c(w, u16)
    out = np.empty(rows * hidden, u16)
    lib().oracle_rms_norm_f16(_p(x), _p(w), _p(out), rows, hidden, eps)
    return out


def add_rms_norm_f16(x, residual, w, rows, hidden, eps):
    x, r, w = _c(x, u16), _c(residual, u16), _c(w, u16)
    rs = np.empty(rows * hidden, u16)
    out = np.empty(rows * hidden, u16)
    lib().oracle_add_rms_norm_f16(_p(x), _p(r), _p(w), _p(rs), _p(out), rows, hidden, eps)
    return rs, out


def rope_angle(position, pair, rotary, theta, factor=1.0):
    return lib().oracle_gemma4_rope_angle(position, pair, rotary, theta, factor)


def rope_tables_gemma4(positions, rope_pairs, rotary, theta, factors=None):
    pos = _c(positions, u32)
    c = np.empty((pos.size, rope_pairs), f32)
    s = np.empty_like(c)
    ff = None if factors is None else _c(factors, f32)
    lib().oracle_rope_tables_gemma4(_p(pos), pos.size, rope_pairs, rotary, theta, _p(ff), _p(c), _p(s))
    return c, s


def rope_tables_llama(positions, head_dim, theta):
    pos = _c(positions, u32)
    c = np.empty((pos.size, head_dim // 2), f32)
    s = np.empty_like(c)
    lib().oracle_rope_tables_llama(_p(pos), pos.size, head_dim, theta, _p(c), _p(s))
    return c, s


def rope_interleaved(x, rows, hidden, cos, sin):
    x, c, s = _c(x, f32), _c(cos, f32), _c(sin, f32)
    out = np.empty(rows * hidden, f32)
    lib().oracle_rope_interleaved_f32(_p(x), rows, hidden, _p(c), _p(s), _p(out))
    return out


def rope_half(x, cos, sin, tokens, heads, head_dim, rope_stride):
    x, c, s = _c(x, f32), _c(cos, f32), _c(sin, f32)
    out = np.empty(tokens * heads * head_dim, f32)
    lib().oracle_rope_half_f32(_p(x), _p(c), _p(s), _p(out), tokens, heads, head_dim, rope_stride)
    return out


def rope_half_f16(x, cos, sin, tokens, heads, head_dim, rope_stride):
    x, c, s = _c(x, u16), _c(cos, f32), _c(sin, f32)
    out = np.empty(tokens * heads * head_dim, u16)
    lib().oracle_rope_half_f16(_p(x), _p(c), _p(s), _p(out), tokens, heads, head_dim, rope_stride)
    return out


def qk_norm_rope(q, k, qw, kw, cos, sin, tokens, q_heads, has_key, head_dim, rope_stride, eps):
    q, qw, c, s = _c(q, f32), _c(qw, f32), _c(cos, f32), _c(sin, f32)
    k = _c(k, f32) if has_key else None
    kw = _c(kw, f32) if has_key else None
    qo = np.empty(tokens * q_heads * head_dim, f32)
    ko = np.empty(tokens * head_dim, f32) if has_key else None
    lib().oracle_qk_norm_rope_f32(_p(q), _p(k), _p(qw), _p(kw), _p(c), _p(s), _p(qo), _p(ko), tokens, q_heads,
                                  1 if has_key else 0, head_dim, rope_stride, eps)
    return qo, ko


def _unary(name, x):
    x = _c(x, f32)
    out = np.empty(x.size, f32)
    getattr(lib(), name)(_p(x), _p(out), x.size)
    return out


def silu(x):
    return _unary("oracle_silu_f32", x)


def gelu(x):
    return _unary("oracle_gelu_f32", x)


def expf(x):
    return np.array([lib().oracle_expf(float(v)) for v in np.asarray(x, f32).reshape(-1)], f32)


def swiglu(gate, up):
    g, u = _c(gate, f32), _c(up, f32)
    out = np.empty(g.size, f32)
    lib().oracle_swiglu_f32(_p(g), _p(u), _p(out), g.size)
    return out


def swiglu_f16(gate, up):
    g, u = _c(gate, u16), _c(up, u16)
    out = np.empty(g.size, u16)
    lib().oracle_swiglu_f16(_p(g), _p(u), _p(out), g.size)
    return out


def geglu(gate, up):
    g, u = _c(gate, f32), _c(up, f32)
    out = np.empty(g.size, f32)
    lib().oracle_geglu_f32(_p(g), _p(u), _p(out), g.size)
    return out


def geglu_offset(gate, ple, ple_offset, ple_row_stride, width, rows):
    g, p = _c(gate, f32), _c(ple, f32)
    out = np.empty(rows * width, f32)
    lib().oracle_geglu_offset_f32(_p(g), _p(p), _p(out), ple_offset, ple_row_stride, width, rows)
    return out


def dequant_q4_0_block(block):
    b = _c(block, u8)
    out = np.empty(32, f32)
    lib().oracle_dequant_q4_0_block(_p(b), _p(out))
    return out


def dequant_q8_0_block(block):
    b = _c(block, u8)
    out = np.empty(32, f32)
    lib().oracle_dequant_q8_0_block(_p(b), _p(out))
    return out


def dequant_q6_k_block(block, llama_order=False):
    b = _c(block, u8)
    out = np.empty(256, f32)
    fn = lib().oracle_dequant_q6_k_block_llama_order if llama_order else lib().oracle_dequant_q6_k_block
    fn(_p(b), _p(out))
    return out


def embed_f32(table, ids, vocab, hidden):
    t, i = _c(table, f32), _c(ids, u32)
    out = np.empty(i.size * hidden, f32)
    lib().oracle_embed_f32(_p(t), _p(i), _p(out), vocab, hidden, i.size)
    return out


def embed_q4_0(table, ids, vocab, hidden, scale, out=None):
    t, i = _c(table, u8), _c(ids, u32)
    out = np.zeros(i.size * hidden, f32) if out is None else np.array(out, f32, copy=True)
    lib().oracle_embed_q4_0(_p(t), _p(i), _p(out), vocab, hidden, i.size, scale)
    return out


def embed_q8_0(table, ids, vocab, hidden, scale, out=None):
    t, i = _c(table, u8), _c(ids, u32)
    out = np.zeros(i.size * hidden, f32) if out is None else np.array(out, f32, copy=True)
    lib().oracle_embed_q8_0(_p(t), _p(i), _p(out), vocab, hidden, i.size, scale)
    return out


def embed_q6_k(table, ids, vocab, hidden, scale, out=None):
    t, i = _c(table, u8), _c(ids, u32)
    out = np.zeros(i.size * hidden, f32) if out is None else np.array(out, f32, copy=True)
    lib().oracle_embed_q6_k(_p(t), _p(i), _p(out), vocab, hidden, i.size, scale)
    return out


def ple(table, ids, proj, vocab, layers, width, emb_scale, out_scale, q6=False, out=None):
    t, i, p = _c(table, u8), _c(ids, u32), _c(proj, f32)
    out = np.zeros(i.size * layers * width, f32) if out is None else np.array(out, f32, copy=True)
    fn = lib().oracle_ple_q6_k if q6 else lib().oracle_ple_q4_0
    fn(_p(t), _p(i), _p(p), _p(out), vocab, layers, width, i.size, emb_scale, out_scale)
    return out


def combine_ple(identity, context):
    a, b = _c(identity, f32), _c(context, f32)
    out = np.empty(a.size, f32)
    lib().oracle_combine_ple(_p(a), _p(b), _p(out), a.size)
    return out


def add(a, b):
    a, b = _c(a, f32), _c(b, f32)
    out = np.empty(a.size, f32)
    lib().oracle_add_f32(_p(a), _p(b), _p(out), a.size)
    return out


def multiply(a, b):
    a, b = _c(a, f32), _c(b, f32)
    out = np.empty(a.size, f32)
    lib().oracle_multiply_f32(_p(a), _p(b), _p(out), a.size)
    return out


def scale(a, s):
    a = _c(a, f32)
    out = np.empty(a.size, f32)
    lib().oracle_scale_f32(_p(a), s, _p(out), a.size)
    return out


def matvec_q4_0_rms_ref(x, weights, rms_weight, input_width, output_width, eps):
    """The reference test's f32 oracle: normalise, then Q4_0 matvec in order
    (crates/atlas-metal/tests/matvec_rms_fused_parity.rs:51-80)."""
    xx, ww = _c(x, f32), _c(weights, u8)
    rw = None if rms_weight is None else _c(rms_weight, f32)
    out = np.zeros(output_width, f32)
    lib().oracle_matvec_q4_0_rms_ref(_p(xx), _p(ww), None if rw is None else _p(rw), input_width, output_width, eps,
                                     _p(out))
    return out


def matvec_q4_0_rms_f64(x, weights, rms_weight, input_width, output_width, eps):
    """float64 value of the projection and its error magnitude inv * sum |terms|."""
    xx, ww = _c(x, f32), _c(weights, u8)
    rw = None if rms_weight is None else _c(rms_weight, f32)
    out, mag = np.zeros(output_width, np.float64), np.zeros(output_width, np.float64)
    lib().oracle_matvec_q4_0_rms_f64(_p(xx), _p(ww), None if rw is None else _p(rw), input_width, output_width, eps,
                                     _p(out), _p(mag))
    return out, mag


KV_FORMATS = {"f32": 0, "q8_0": 1, "q4_0": 2}
KV_BLOCK_BYTES = {"q8_0": 34, "q4_0": 18}


def kv_row_bytes(fmt, kv_width):
    return kv_width * 4 if fmt == "f32" else (kv_width // 32) * KV_BLOCK_BYTES[fmt]


def kv_append(fmt, key, value, cache, kv_width, capacity, positions, vnorm, eps):
    """kv_append_decode_*[_batch|_vnorm] restated; returns the updated cache bytes."""
    k, v, pos = _c(key, f32), _c(value, f32), _c(positions, u32)
    out = np.array(cache, u8, copy=True)
    lib().oracle_kv_append(KV_FORMATS[fmt], _p(k), _p(v), _p(out), kv_width, capacity, _p(pos), pos.size,
                           1 if vnorm else 0, eps)
    return out


def encode_q8_0_block(values):
    v, out = _c(values, f32), np.zeros(34, u8)
    lib().oracle_encode_q8_0_block(_p(v), _p(out))
    return out


def encode_q4_0_block(values):
    v, out = _c(values, f32), np.zeros(18, u8)
    lib().oracle_encode_q4_0_block(_p(v), _p(out))
    return out



def tanh_precise(x):
    """tanh of the logit soft cap, elementwise over a float32 array."""
    x = _c(x, f32)
    return np.array([lib().oracle_tanh_precise(float(v)) for v in x.ravel()], f32).reshape(x.shape)


def softcap(x, cap):
    x = _c(x, f32)
    out = np.empty_like(x)
    lib().oracle_softcap_f32(_p(x), _p(out), x.size, cap)
    return out


def argmax(values):
    v = _c(values, f32)
    return int(lib().oracle_argmax_f32(_p(v), v.size))


def softcap_argmax_rows(logits, rows, count, cap):
    """Returns (capped logits, selected ids); cap <= 0 skips the soft cap."""
    x = _c(logits, f32).copy()
    sel = np.empty(rows, u32)
    lib().oracle_softcap_argmax_rows(_p(x), _p(sel), rows, count, cap)
    return x, sel
