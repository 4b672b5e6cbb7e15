"""Python host bindings over libatlas_hip_ops.so.

`HipRuntime` owns a context (device + stream) and device buffers; its
`dispatch_*` methods are the resident (device-pointer) vocabulary the
executor call sites use (ResidentCommand, crates/atlas-metal/src/lib.rs:
242-756).  `NeuralOps` mirrors atlas_ops::NeuralOps
(crates/atlas-ops/src/lib.rs:20-147): host slices in, `(output, timing)` out,
errors raised as `OperatorError` carrying the reference's MetalError kind.
"""
from __future__ import annotations

import ctypes
from ctypes import byref, c_float, c_int, c_void_p
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import DispatchTiming


class OperatorError(RuntimeError):
    """OperatorError::Metal(MetalError::...) (crates/atlas-ops/src/lib.rs:14-18)."""

    KINDS = {
        _lib.ATLAS_ERR_NO_DEVICE: "NoDevice",
        _lib.ATLAS_ERR_INVALID_INPUT: "InvalidInput",
        _lib.ATLAS_ERR_COMMAND_FAILED: "CommandFailed",
        _lib.ATLAS_ERR_OUT_OF_MEMORY: "OutOfMemory",
    }

    def __init__(self, code: int, message: str):
        self.code = code
        self.kind = self.KINDS.get(code, f"Unknown({code})")
        super().__init__(f"{self.kind}: {message}")


def _ptr(a) -> int:
    if isinstance(a, DeviceBuffer):
        return a.ptr
    if a is None:
        return None
    if isinstance(a, int):
        return a
    return a.ctypes.data


@dataclass
class DeviceBuffer:
    """A device allocation owned by a HipRuntime (GpuBuffer, lib.rs:225-238)."""

    runtime: "HipRuntime"
    ptr: int
    nbytes: int
    dtype: np.dtype = np.dtype(np.float32)

    def offset(self, byte_offset: int, dtype=None) -> "DeviceBuffer":
        """A view at a byte offset (the `_at` dispatch binding, lib.rs:263-410)."""
        return DeviceBuffer(self.runtime, self.ptr + byte_offset, self.nbytes - byte_offset,
                            np.dtype(dtype) if dtype is not None else self.dtype)

    def upload(self, host: np.ndarray) -> "DeviceBuffer":
        host = np.ascontiguousarray(host)
        assert host.nbytes <= self.nbytes, (host.nbytes, self.nbytes)
        self.runtime._check(self.runtime.lib.atlas_hip_upload(self.runtime.ctx, self.ptr, host.ctypes.data, host.nbytes))
        return self

    def download(self, count: int | None = None, dtype=None) -> np.ndarray:
        dtype = np.dtype(dtype) if dtype is not None else self.dtype
        if count is None:
            count = self.nbytes // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        self.runtime._check(self.runtime.lib.atlas_hip_download(self.runtime.ctx, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            self.runtime.lib.atlas_hip_free(self.runtime.ctx, self.ptr)
            self.ptr = 0


class HipRuntime:
    """Device context: MetalRuntime::new (crates/atlas-metal/src/lib.rs:909-1061)."""

    def __init__(self, device: int = 0, reduction: int = _lib.ATLAS_REDUCTION_AUTO):
        self.lib = _lib.load()
        ctx = c_void_p()
        rc = self.lib.atlas_hip_init(device, byref(ctx))
        if rc != _lib.ATLAS_OK:
            raise OperatorError(rc, "no HIP device is available" if rc == _lib.ATLAS_ERR_NO_DEVICE else "init failed")
        self.ctx = ctx
        self._buffers: list[DeviceBuffer] = []
        self.set_reduction(reduction)

    # -- plumbing -------------------------------------------------------
    def _check(self, rc: int) -> None:
        if rc != _lib.ATLAS_OK:
            msg = self.lib.atlas_hip_last_error(self.ctx)
            raise OperatorError(rc, msg.decode() if msg else "")

    def close(self) -> None:
        if getattr(self, "ctx", None):
            for b in self._buffers:
                b.free()
            self._buffers.clear()
            self.lib.atlas_hip_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_reduction(self, reduction: int) -> None:
        self._check(self.lib.atlas_hip_set_reduction(self.ctx, reduction))

    def alloc(self, nbytes: int, dtype=np.float32) -> DeviceBuffer:
        p = c_void_p()
        self._check(self.lib.atlas_hip_malloc(self.ctx, nbytes, byref(p)))
        b = DeviceBuffer(self, p.value, nbytes, np.dtype(dtype))
        self._buffers.append(b)
        return b

    def upload(self, host: np.ndarray) -> DeviceBuffer:
        host = np.ascontiguousarray(host)
        return self.alloc(max(host.nbytes, 16), host.dtype).upload(host)

    def empty(self, count: int, dtype=np.float32) -> DeviceBuffer:
        return self.alloc(max(count * np.dtype(dtype).itemsize, 16), dtype)

    def free(self, buf: DeviceBuffer) -> None:
        if buf in self._buffers:
            self._buffers.remove(buf)
        buf.free()

    def memset(self, buf: DeviceBuffer, value: int, nbytes: int) -> None:
        self._check(self.lib.atlas_hip_memset(self.ctx, _ptr(buf), value, nbytes))

    def copy(self, dst: DeviceBuffer, src: DeviceBuffer, nbytes: int) -> None:
        """Device-to-device copy on the context stream."""
        self._check(self.lib.atlas_hip_copy_d2d(self.ctx, _ptr(dst), _ptr(src), nbytes))

    def sync(self) -> None:
        self._check(self.lib.atlas_hip_sync(self.ctx))

    def telemetry(self) -> _lib.Telemetry:
        t = _lib.Telemetry()
        self._check(self.lib.atlas_hip_get_telemetry(self.ctx, byref(t)))
        return t

    def event(self) -> int:
        e = c_void_p()
        self._check(self.lib.atlas_hip_event_create(self.ctx, byref(e)))
        return e.value

    def record(self, event: int) -> None:
        self._check(self.lib.atlas_hip_event_record(self.ctx, event))

    def elapsed_ms(self, start: int, stop: int) -> float:
        ms = c_float()
        self._check(self.lib.atlas_hip_event_elapsed_ms(self.ctx, start, stop, byref(ms)))
        return ms.value

    # -- graph capture ---------------------------------------------------
    def graph_begin(self) -> None:
        """Start recording the ops enqueued on this context (atlas_hip_graph_begin)."""
        self._check(self.lib.atlas_hip_graph_begin(self.ctx))

    def graph_end(self) -> int:
        """Finish recording; returns an executable graph handle."""
        g = c_void_p()
        self._check(self.lib.atlas_hip_graph_end(self.ctx, byref(g)))
        return g.value

    def graph_launch(self, graph: int) -> None:
        self._check(self.lib.atlas_hip_graph_launch(self.ctx, graph))

    def graph_destroy(self, graph: int) -> None:
        self._check(self.lib.atlas_hip_graph_destroy(self.ctx, graph))

    # -- resident (device-pointer) ops ----------------------------------
    def rms_norm(self, x, w, y, rows, hidden, eps):
        self._check(self.lib.atlas_hip_rms_norm_f32(self.ctx, _ptr(x), _ptr(w), _ptr(y), rows, hidden, eps))

    def rms_norm_residual(self, x, w, residual, normalized, out, rows, hidden, eps):
        self._check(self.lib.atlas_hip_rms_norm_residual_f32(
            self.ctx, _ptr(x), _ptr(w), _ptr(residual), _ptr(normalized), _ptr(out), rows, hidden, eps))

    def add_rms_norm(self, x, residual, w, residual_out, y, rows, hidden, eps):
        self._check(self.lib.atlas_hip_add_rms_norm_f32(
            self.ctx, _ptr(x), _ptr(residual), _ptr(w), _ptr(residual_out), _ptr(y), rows, hidden, eps))

    def rms_norm_add_scale(self, x, w, state, scale, rows, hidden, eps):
        self._check(self.lib.atlas_hip_rms_norm_add_scale_f32(
            self.ctx, _ptr(x), _ptr(w), _ptr(state), _ptr(scale), rows, hidden, eps))

    def rms_norm_groups_stable(self, values, w, width, groups, eps):
        self._check(self.lib.atlas_hip_rms_norm_groups_stable_f32(self.ctx, _ptr(values), _ptr(w), width, groups, eps))

    def rms_norm_f16(self, x, w, y, rows, hidden, eps):
        self._check(self.lib.atlas_hip_rms_norm_f16(self.ctx, _ptr(x), _ptr(w), _ptr(y), rows, hidden, eps))

    def add_rms_norm_f16(self, x, residual, w, residual_out, y, rows, hidden, eps):
        self._check(self.lib.atlas_hip_add_rms_norm_f16(
            self.ctx, _ptr(x), _ptr(residual), _ptr(w), _ptr(residual_out), _ptr(y), rows, hidden, eps))

    def qk_norm_rope(self, q, k, qw, kw, cos, sin, q_out, k_out, tokens, q_heads, has_key, head_dim,
                     rope_stride, eps):
        self._check(self.lib.atlas_hip_qk_norm_rope_f32(
            self.ctx, _ptr(q), _ptr(k), _ptr(qw), _ptr(kw), _ptr(cos), _ptr(sin), _ptr(q_out), _ptr(k_out),
            tokens, q_heads, has_key, head_dim, rope_stride, eps))

    def rope_half(self, x, cos, sin, y, tokens, heads, head_dim, rope_stride):
        self._check(self.lib.atlas_hip_rope_half_f32(
            self.ctx, _ptr(x), _ptr(cos), _ptr(sin), _ptr(y), tokens, heads, head_dim, rope_stride))

    def rope_half_f16(self, x, cos, sin, y, tokens, heads, head_dim, rope_stride):
        self._check(self.lib.atlas_hip_rope_half_f16(
            self.ctx, _ptr(x), _ptr(cos), _ptr(sin), _ptr(y), tokens, heads, head_dim, rope_stride))

    # Q and K of the same tokens in one launch (the Llama decode's two rope chains, executor.rs:1120-1166)
    def rope_half_qk(self, q, k, cos, sin, q_out, k_out, tokens, q_heads, k_heads, head_dim, rope_stride, f16=False):
        fn = self.lib.atlas_hip_rope_half_qk_f16 if f16 else self.lib.atlas_hip_rope_half_qk_f32
        self._check(fn(self.ctx, _ptr(q), _ptr(k), _ptr(cos), _ptr(sin), _ptr(q_out), _ptr(k_out), tokens, q_heads,
                       k_heads, head_dim, rope_stride))

    def rope_interleaved(self, x, cos, sin, y, rows, hidden):
        self._check(self.lib.atlas_hip_rope_interleaved_f32(self.ctx, _ptr(x), _ptr(cos), _ptr(sin), _ptr(y), rows, hidden))

    def swiglu(self, gate, up, out, n):
        self._check(self.lib.atlas_hip_swiglu_f32(self.ctx, _ptr(gate), _ptr(up), _ptr(out), n))

    def swiglu_f16(self, gate, up, out, n):
        self._check(self.lib.atlas_hip_swiglu_f16(self.ctx, _ptr(gate), _ptr(up), _ptr(out), n))

    def geglu(self, gate, up, out, n):
        self._check(self.lib.atlas_hip_geglu_f32(self.ctx, _ptr(gate), _ptr(up), _ptr(out), n))

    def geglu_offset(self, gate, ple, out, ple_offset, ple_row_stride, width, rows):
        self._check(self.lib.atlas_hip_geglu_offset_f32(
            self.ctx, _ptr(gate), _ptr(ple), _ptr(out), ple_offset, ple_row_stride, width, rows))

    def silu(self, x, y, n):
        self._check(self.lib.atlas_hip_silu_f32(self.ctx, _ptr(x), _ptr(y), n))

    def gelu(self, x, y, n):
        self._check(self.lib.atlas_hip_gelu_f32(self.ctx, _ptr(x), _ptr(y), n))

    def add(self, a, b, y, n):
        self._check(self.lib.atlas_hip_add_f32(self.ctx, _ptr(a), _ptr(b), _ptr(y), n))

    def multiply(self, a, b, y, n):
        self._check(self.lib.atlas_hip_multiply_f32(self.ctx, _ptr(a), _ptr(b), _ptr(y), n))

    def scale(self, a, s, y, n):
        self._check(self.lib.atlas_hip_scale_f32(self.ctx, _ptr(a), s, _ptr(y), n))

    def embed_f32(self, table, ids, out, vocab, hidden, tokens, scale=1.0):
        self._check(self.lib.atlas_hip_embed_f32(self.ctx, _ptr(table), _ptr(ids), _ptr(out), vocab, hidden, tokens, scale))

    def embed_q4_0(self, table, ids, out, vocab, hidden, tokens, scale):
        self._check(self.lib.atlas_hip_embed_q4_0(self.ctx, _ptr(table), _ptr(ids), _ptr(out), vocab, hidden, tokens, scale))

    def embed_q6_k(self, table, ids, out, vocab, hidden, tokens, scale):
        self._check(self.lib.atlas_hip_embed_q6_k(self.ctx, _ptr(table), _ptr(ids), _ptr(out), vocab, hidden, tokens, scale))

    def embed_q8_0(self, table, ids, out, vocab, hidden, tokens, scale=1.0):
        self._check(self.lib.atlas_hip_embed_q8_0(self.ctx, _ptr(table), _ptr(ids), _ptr(out), vocab, hidden, tokens, scale))

    def ple_q4_0(self, table, ids, proj, out, vocab, layers, width, tokens, emb_scale, out_scale):
        self._check(self.lib.atlas_hip_ple_q4_0(self.ctx, _ptr(table), _ptr(ids), _ptr(proj), _ptr(out), vocab, layers,
                                                width, tokens, emb_scale, out_scale))

    def ple_q6_k(self, table, ids, proj, out, vocab, layers, width, tokens, emb_scale, out_scale):
        self._check(self.lib.atlas_hip_ple_q6_k(self.ctx, _ptr(table), _ptr(ids), _ptr(proj), _ptr(out), vocab, layers,
                                                width, tokens, emb_scale, out_scale))

    # RMS-folded Q4_0 decode projections (matvec_q4_0_16row_mv_rms and the fused
    # QKV / gate-up dispatches, kernels.metal:3368-3564, 3786-3864); rms_weight
    # None gives the plain Q4_0 matvec.
    def matvec_q4_0_rms(self, x, weights, out, input_width, output_width, rms_weight, eps):
        self._check(self.lib.atlas_hip_matvec_q4_0_rms_f32(self.ctx, _ptr(x), _ptr(weights), _ptr(out), input_width,
                                                           output_width, _ptr(rms_weight), eps))

    def matmul_q4_0_qkv_rms(self, x, qw, kw, vw, q_out, k_out, v_out, input_width, q_width, kv_width, rms_weight, eps):
        self._check(self.lib.atlas_hip_matmul_q4_0_qkv_rms_f32(self.ctx, _ptr(x), _ptr(qw), _ptr(kw), _ptr(vw),
                                                               _ptr(q_out), _ptr(k_out), _ptr(v_out), input_width,
                                                               q_width, kv_width, _ptr(rms_weight), eps))

    # PLE input gate: gelu(Q4_0 matvec) * PLE slice (gemma4_ple_gate_gelu_f32, kernels.metal:803-881)
    def ple_gate_gelu(self, x, weights, ple, ple_offset, out, input_width, output_width):
        self._check(self.lib.atlas_hip_ple_gate_gelu_f32(self.ctx, _ptr(x), _ptr(weights), _ptr(ple), ple_offset,
                                                         _ptr(out), input_width, output_width))

    # The PLE projection of one decode token with its stable group norm as
    # epilogue (matvec_f16 + scalar_multiply_f32 + rms_norm_groups_in_place_stable_f32,
    # kernels.metal:731-740, 897-917; gemma4_executor.rs:4184-4214); weights are F16 bits.
    def ple_projection_f16(self, x, weights, norm_weight, out, hidden, width, groups, scale, eps):
        self._check(self.lib.atlas_hip_ple_projection_f16(self.ctx, _ptr(x), _ptr(weights), _ptr(norm_weight),
                                                          _ptr(out), hidden, width, groups, scale, eps))

    # KV-cache append with the fused V RMSNorm (kv_append_decode_*[_batch|_vnorm],
    # kernels.metal:1197-1436); fmt is "f32", "q8_0" or "q4_0".
    def kv_append(self, fmt, key, value, cache, kv_width, capacity, positions, tokens, vnorm, eps):
        fn = {"f32": self.lib.atlas_hip_kv_append_f32, "q8_0": self.lib.atlas_hip_kv_append_q8_0,
              "q4_0": self.lib.atlas_hip_kv_append_q4_0}[fmt]
        self._check(fn(self.ctx, _ptr(key), _ptr(value), _ptr(cache), kv_width, capacity, _ptr(positions), tokens,
                       1 if vnorm else 0, eps))

    # Decode tail: softcap_f32 / argmax_f32 (kernels.metal:931-934, 2033-2066)
    def softcap(self, x, y, n, cap):
        self._check(self.lib.atlas_hip_softcap_f32(self.ctx, _ptr(x), _ptr(y), n, cap))

    def argmax(self, values, selected, rows, count):
        self._check(self.lib.atlas_hip_argmax_f32(self.ctx, _ptr(values), _ptr(selected), rows, count))

    def softcap_argmax(self, logits, capped, selected, rows, count, cap):
        self._check(self.lib.atlas_hip_softcap_argmax_f32(self.ctx, _ptr(logits), _ptr(capped), _ptr(selected), rows,
                                                          count, cap))

    def softcap_argmax_noalloc(self, logits, capped, selected, rows, count, cap):
        """The no-allocation variant (static device scratch, one launch pair)."""
        self._check(self.lib.atlas_hip_softcap_argmax_f32_noalloc(self.ctx, _ptr(logits), _ptr(capped),
                                                                  _ptr(selected), rows, count, cap))

    def matmul_q4_0_gate_up_rms(self, x, gw, uw, g_out, u_out, input_width, output_width, rms_weight, eps):
        self._check(self.lib.atlas_hip_matmul_q4_0_gate_up_rms_f32(self.ctx, _ptr(x), _ptr(gw), _ptr(uw), _ptr(g_out),
                                                                   _ptr(u_out), input_width, output_width,
                                                                   _ptr(rms_weight), eps))


def rope_tables_gemma4(positions, rope_pairs, rotary, theta, frequency_factors=None):
    """Host cos/sin tables [tokens, rope_pairs] (gemma4_executor.rs:622-633, 3494-3519)."""
    lib = _lib.load()
    pos = np.ascontiguousarray(positions, dtype=np.uint32)
    cos = np.empty((pos.size, rope_pairs), np.float32)
    sin = np.empty_like(cos)
    ff = None if frequency_factors is None else np.ascontiguousarray(frequency_factors, np.float32)
    rc = lib.atlas_rope_tables_gemma4(pos.ctypes.data, pos.size, rope_pairs, rotary, theta,
                                      None if ff is None else ff.ctypes.data, cos.ctypes.data, sin.ctypes.data)
    if rc:
        raise OperatorError(rc, "invalid RoPE table arguments")
    return cos, sin


def rope_tables_llama(positions, head_dim, theta):
    """Host cos/sin tables [tokens, head_dim/2] (executor.rs:632-647)."""
    lib = _lib.load()
    pos = np.ascontiguousarray(positions, dtype=np.uint32)
    cos = np.empty((pos.size, head_dim // 2), np.float32)
    sin = np.empty_like(cos)
    rc = lib.atlas_rope_tables_llama(pos.ctypes.data, pos.size, head_dim, theta, cos.ctypes.data, sin.ctypes.data)
    if rc:
        raise OperatorError(rc, "invalid RoPE table arguments")
    return cos, sin


class NeuralOps:
    """atlas_ops::NeuralOps (crates/atlas-ops/src/lib.rs:20-147) over the HIP library.

    Each method takes host arrays, runs synchronously and returns
    `(output, DispatchTiming)`; invalid input raises OperatorError(InvalidInput).
    """

    def __init__(self, device: int = 0):
        self.rt = HipRuntime(device)

    def runtime(self) -> HipRuntime:
        return self.rt

    def _call(self, fn, *args):
        timing = DispatchTiming()
        self.rt._check(fn(self.rt.ctx, *args, byref(timing)))
        return timing

    @staticmethod
    def _f32(a):
        return np.ascontiguousarray(a, dtype=np.float32)

    def embedding(self, table, vocabulary, hidden, token_ids):
        table = self._f32(table)
        ids = np.ascontiguousarray(token_ids, dtype=np.uint32)
        out = np.empty(ids.size * hidden, np.float32)
        t = self._call(self.rt.lib.atlas_ops_embedding, table.ctypes.data, table.size, vocabulary, hidden,
                       ids.ctypes.data, ids.size, out.ctypes.data, out.size)
        return out, t

    def embedding_lookup_q6_k(self, weights, vocabulary, hidden, token_ids):
        w = np.ascontiguousarray(weights, dtype=np.uint8)
        ids = np.ascontiguousarray(token_ids, dtype=np.uint32)
        out = np.empty(ids.size * hidden, np.float32)
        t = self._call(self.rt.lib.atlas_ops_embedding_q6_k, w.ctypes.data, w.size, vocabulary, hidden,
                       ids.ctypes.data, ids.size, out.ctypes.data, out.size)
        return out, t

    def add(self, lhs, rhs):
        lhs, rhs = self._f32(lhs), self._f32(rhs)
        out = np.empty(lhs.size, np.float32)
        t = self._call(self.rt.lib.atlas_ops_add, lhs.ctypes.data, lhs.size, rhs.ctypes.data, rhs.size,
                       out.ctypes.data, out.size)
        return out, t

    def multiply(self, lhs, rhs):
        lhs, rhs = self._f32(lhs), self._f32(rhs)
        out = np.empty(lhs.size, np.float32)
        t = self._call(self.rt.lib.atlas_ops_multiply, lhs.ctypes.data, lhs.size, rhs.ctypes.data, rhs.size,
                       out.ctypes.data, out.size)
        return out, t

    def scalar_multiply(self, values, scalar):
        x = self._f32(values)
        out = np.empty(x.size, np.float32)
        t = self._call(self.rt.lib.atlas_ops_scalar_multiply, x.ctypes.data, x.size, scalar, out.ctypes.data, out.size)
        return out, t

    def silu(self, values):
        x = self._f32(values)
        out = np.empty(x.size, np.float32)
        t = self._call(self.rt.lib.atlas_ops_silu, x.ctypes.data, x.size, out.ctypes.data, out.size)
        return out, t

    def gelu(self, values):
        x = self._f32(values)
        out = np.empty(x.size, np.float32)
        t = self._call(self.rt.lib.atlas_ops_gelu, x.ctypes.data, x.size, out.ctypes.data, out.size)
        return out, t

    def rms_norm(self, values, rows, hidden, weight, epsilon):
        x, w = self._f32(values), self._f32(weight)
        out = np.empty(rows * hidden, np.float32)
        t = self._call(self.rt.lib.atlas_ops_rms_norm, x.ctypes.data, x.size, rows, hidden, w.ctypes.data, w.size,
                       epsilon, out.ctypes.data, out.size)
        return out, t

    def rope(self, values, rows, hidden, cos, sin):
        x, c, s = self._f32(values), self._f32(cos), self._f32(sin)
        out = np.empty(rows * hidden, np.float32)
        t = self._call(self.rt.lib.atlas_ops_rope, x.ctypes.data, x.size, rows, hidden, c.ctypes.data, c.size,
                       s.ctypes.data, s.size, out.ctypes.data, out.size)
        return out, t
