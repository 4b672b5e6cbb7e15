"""ctypes loader for libatlas_hip_ops.so (the C ABI in include/atlas_hip_ops.h).

The shared library is the product; this module only declares its signatures.
It raises immediately when the library has not been built: there is no
CPU fallback for any op.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_size_t, c_uint8, c_uint16, c_uint32, c_uint64, c_void_p

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PACKAGE_DIR, "libatlas_hip_ops.so")

ATLAS_OK = 0
ATLAS_ERR_NO_DEVICE = -1
ATLAS_ERR_INVALID_INPUT = -2
ATLAS_ERR_COMMAND_FAILED = -3
ATLAS_ERR_OUT_OF_MEMORY = -4

ATLAS_REDUCTION_SEQUENTIAL = 0
ATLAS_REDUCTION_WIDE = 1
ATLAS_REDUCTION_AUTO = 2


class DispatchTiming(ctypes.Structure):
    """DispatchTiming (crates/atlas-metal/src/lib.rs:81-88)."""

    _fields_ = [("wall_ms", c_double), ("gpu_ms", c_double)]


class Telemetry(ctypes.Structure):
    _fields_ = [
        ("dispatches", c_uint64),
        ("syncs", c_uint64),
        ("upload_bytes", c_uint64),
        ("readback_bytes", c_uint64),
        ("allocations", c_uint64),
        ("resident_bytes", c_uint64),
        ("peak_resident_bytes", c_uint64),
    ]


class GgufTensor(ctypes.Structure):
    """atlas_gguf_tensor (include/atlas_gguf.h): GgufTensor, crates/atlas-core/src/gguf.rs:80-87."""

    _fields_ = [("name", c_void_p), ("name_len", c_uint64), ("n_dims", c_uint32), ("dims", c_uint64 * 4), ("type", c_uint32),
                ("offset", c_uint64), ("bytes", c_uint64)]


P = c_void_p  # device or host pointer
CTX = c_void_p
F = c_float
U32 = c_uint32
U64 = c_uint64
SZ = c_size_t
TIMING = POINTER(DispatchTiming)

# name -> argtypes (all return int unless listed in _RESTYPES)
SIGNATURES = {
    "atlas_hip_device_count": [POINTER(c_int)],
    "atlas_hip_init": [c_int, POINTER(c_void_p)],
    "atlas_hip_destroy": [CTX],
    "atlas_hip_sync": [CTX],
    "atlas_hip_set_stream": [CTX, P],
    "atlas_hip_get_stream": [CTX],
    "atlas_hip_set_reduction": [CTX, c_int],
    "atlas_hip_last_error": [CTX],
    "atlas_hip_get_telemetry": [CTX, POINTER(Telemetry)],
    "atlas_hip_malloc": [CTX, SZ, POINTER(c_void_p)],
    "atlas_hip_free": [CTX, P],
    "atlas_hip_upload": [CTX, P, P, SZ],
    "atlas_hip_download": [CTX, P, P, SZ],
    "atlas_hip_memset": [CTX, P, c_int, SZ],
    "atlas_hip_copy_d2d": [CTX, P, P, SZ],
    "atlas_hip_event_create": [CTX, POINTER(c_void_p)],
    "atlas_hip_event_record": [CTX, P],
    "atlas_hip_event_elapsed_ms": [CTX, P, P, POINTER(c_float)],
    "atlas_hip_event_destroy": [CTX, P],
    "atlas_hip_graph_begin": [CTX],
    "atlas_hip_graph_end": [CTX, POINTER(c_void_p)],
    "atlas_hip_graph_launch": [CTX, P],
    "atlas_hip_graph_destroy": [CTX, P],
    "atlas_hip_rms_norm_f32": [CTX, P, P, P, U32, U32, F],
    "atlas_hip_rms_norm_residual_f32": [CTX, P, P, P, P, P, U32, U32, F],
    "atlas_hip_add_rms_norm_f32": [CTX, P, P, P, P, P, U32, U32, F],
    "atlas_hip_rms_norm_add_scale_f32": [CTX, P, P, P, P, U32, U32, F],
    "atlas_hip_rms_norm_groups_stable_f32": [CTX, P, P, U32, U32, F],
    "atlas_hip_rms_norm_f16": [CTX, P, P, P, U32, U32, F],
    "atlas_hip_add_rms_norm_f16": [CTX, P, P, P, P, P, U32, U32, F],
    "atlas_hip_qk_norm_rope_f32": [CTX, P, P, P, P, P, P, P, P, U32, U32, U32, U32, U32, F],
    "atlas_hip_rope_half_f32": [CTX, P, P, P, P, U32, U32, U32, U32],
    "atlas_hip_rope_half_f16": [CTX, P, P, P, P, U32, U32, U32, U32],
    "atlas_hip_rope_interleaved_f32": [CTX, P, P, P, P, U32, U32],
    "atlas_hip_rope_half_qk_f32": [CTX, P, P, P, P, P, P, U32, U32, U32, U32, U32],
    "atlas_hip_rope_half_qk_f16": [CTX, P, P, P, P, P, P, U32, U32, U32, U32, U32],
    "atlas_rope_tables_gemma4": [P, SZ, SZ, SZ, F, P, P, P],
    "atlas_rope_tables_llama": [P, SZ, SZ, F, P, P],
    "atlas_hip_swiglu_f32": [CTX, P, P, P, U64],
    "atlas_hip_swiglu_f16": [CTX, P, P, P, U64],
    "atlas_hip_geglu_f32": [CTX, P, P, P, U64],
    "atlas_hip_geglu_offset_f32": [CTX, P, P, P, U32, U32, U32, U32],
    "atlas_hip_silu_f32": [CTX, P, P, U64],
    "atlas_hip_gelu_f32": [CTX, P, P, U64],
    "atlas_hip_add_f32": [CTX, P, P, P, U64],
    "atlas_hip_multiply_f32": [CTX, P, P, P, U64],
    "atlas_hip_scale_f32": [CTX, P, F, P, U64],
    "atlas_hip_embed_f32": [CTX, P, P, P, U32, U32, U32, F],
    "atlas_hip_embed_q4_0": [CTX, P, P, P, U32, U32, U32, F],
    "atlas_hip_embed_q6_k": [CTX, P, P, P, U32, U32, U32, F],
    "atlas_hip_embed_q8_0": [CTX, P, P, P, U32, U32, U32, F],
    "atlas_hip_ple_q4_0": [CTX, P, P, P, P, U32, U32, U32, U32, F, F],
    "atlas_hip_ple_q6_k": [CTX, P, P, P, P, U32, U32, U32, U32, F, F],
    "atlas_hip_matvec_q4_0_rms_f32": [CTX, P, P, P, U32, U32, P, F],
    "atlas_hip_matmul_q4_0_qkv_rms_f32": [CTX, P, P, P, P, P, P, P, U32, U32, U32, P, F],
    "atlas_hip_matmul_q4_0_gate_up_rms_f32": [CTX, P, P, P, P, P, U32, U32, P, F],
    "atlas_hip_ple_gate_gelu_f32": [CTX, P, P, P, U32, P, U32, U32],
    "atlas_hip_ple_projection_f16": [CTX, P, P, P, P, U32, U32, U32, F, F],
    "atlas_hip_kv_append_f32": [CTX, P, P, P, U32, U32, P, U32, c_int, F],
    "atlas_hip_kv_append_q8_0": [CTX, P, P, P, U32, U32, P, U32, c_int, F],
    "atlas_hip_kv_append_q4_0": [CTX, P, P, P, U32, U32, P, U32, c_int, F],
    "atlas_hip_softcap_f32": [CTX, P, P, U64, F],
    "atlas_hip_argmax_f32": [CTX, P, P, U32, U32],
    "atlas_hip_softcap_argmax_f32": [CTX, P, P, P, U32, U32, F],
    "atlas_hip_softcap_argmax_f32_noalloc": [CTX, P, P, P, U32, U32, F],
    "atlas_gguf_open": [c_char_p, POINTER(c_void_p), c_char_p, SZ],
    "atlas_gguf_from_bytes": [P, SZ, POINTER(c_void_p), c_char_p, SZ],
    "atlas_gguf_close": [P],
    "atlas_gguf_tensor_count": [P],
    "atlas_gguf_tensor_info": [P, U64, POINTER(GgufTensor)],
    "atlas_gguf_find_tensor": [P, c_char_p],
    "atlas_gguf_tensor_data": [P, U64, POINTER(c_void_p), POINTER(c_uint64)],
    "atlas_gguf_upload_tensor": [CTX, P, U64, P],
    "atlas_gguf_metadata_count": [P],
    "atlas_gguf_metadata_entry": [P, U64, POINTER(c_void_p), POINTER(c_uint64), POINTER(c_void_p),
                                  POINTER(c_uint64)],
    "atlas_gguf_metadata_get": [P, c_char_p],
    "atlas_gguf_metadata_array_count": [P],
    "atlas_gguf_metadata_array_entry": [P, U64, POINTER(c_void_p), POINTER(c_uint64), POINTER(c_uint32),
                                        POINTER(c_uint64), POINTER(c_void_p)],
    "atlas_gguf_metadata_array_string": [P, U64, U64, POINTER(c_void_p), POINTER(c_uint64)],
    "atlas_gguf_find_metadata_array": [P, c_char_p],
    "atlas_ops_embedding": [CTX, P, SZ, SZ, SZ, P, SZ, P, SZ, TIMING],
    "atlas_ops_embedding_q6_k": [CTX, P, SZ, SZ, SZ, P, SZ, P, SZ, TIMING],
    "atlas_ops_add": [CTX, P, SZ, P, SZ, P, SZ, TIMING],
    "atlas_ops_multiply": [CTX, P, SZ, P, SZ, P, SZ, TIMING],
    "atlas_ops_scalar_multiply": [CTX, P, SZ, F, P, SZ, TIMING],
    "atlas_ops_silu": [CTX, P, SZ, P, SZ, TIMING],
    "atlas_ops_gelu": [CTX, P, SZ, P, SZ, TIMING],
    "atlas_ops_rms_norm": [CTX, P, SZ, SZ, SZ, P, SZ, F, P, SZ, TIMING],
    "atlas_ops_rope": [CTX, P, SZ, SZ, SZ, P, SZ, P, SZ, P, SZ, TIMING],
}

_RESTYPES = {
    "atlas_gguf_close": None,
    "atlas_gguf_tensor_count": c_uint64,
    "atlas_gguf_find_tensor": ctypes.c_int64,
    "atlas_gguf_metadata_count": c_uint64,
    "atlas_gguf_metadata_get": c_char_p,
    "atlas_gguf_metadata_array_count": c_uint64,
    "atlas_gguf_find_metadata_array": ctypes.c_int64,
    "atlas_hip_destroy": None,
    "atlas_hip_get_stream": c_void_p,
    "atlas_hip_last_error": c_char_p,
}

_LIB = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library and declare every signature.  Raises if it is missing."""
    global _LIB
    if _LIB is not None and path == LIB_PATH:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(there is no CPU fallback for these ops)"
        )
    lib = ctypes.CDLL(path)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, c_int)
    if path == LIB_PATH:
        _LIB = lib
    return lib
