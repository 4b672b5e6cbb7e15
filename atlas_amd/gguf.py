"""GGUF v3 models through the C reader in libatlas_hip_ops.so.

Mirrors atlas_core::gguf (crates/atlas-core/src/gguf.rs:16-235):
`GgufModel.open(path)` / `GgufModel.from_bytes(data)` with `.metadata`
(scalar values as strings), `.metadata_arrays`, `.tensors` (`GgufTensor`)
and `.tensor_data(tensor)`; failures raise OperatorError("InvalidInput"),
as CoreError::InvalidInput.  `upload(runtime, tensor)` places a tensor's
encoded bytes in device memory, where the gather / matvec ops read them
unconverted.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .runtime import DeviceBuffer, HipRuntime, OperatorError

F32, F16, Q4_0, Q8_0, Q6_K = 0, 1, 2, 8, 14
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q6_K: "Q6K"}
_ARRAY_DTYPES = {6: np.float32, 5: np.int32, 4: np.uint32, 10: np.uint64, 11: np.int64, 7: np.bool_}


def _text(ptr, length) -> str:
    return ctypes.string_at(ptr.value, length.value).decode() if length.value else ""


@dataclass(frozen=True)
class GgufTensor:
    """GgufTensor (gguf.rs:80-87); dims in GGUF order, dims[0] contiguous."""

    name: str
    dims: tuple
    tensor_type: int
    offset: int
    bytes: int
    index: int


class GgufModel:
    def __init__(self, handle, lib):
        self._h = handle
        self._lib = lib
        n = lib.atlas_gguf_tensor_count(handle)
        info = _lib.GgufTensor()
        tensors = []
        for i in range(n):
            if lib.atlas_gguf_tensor_info(handle, i, ctypes.byref(info)) != 0:
                raise OperatorError(_lib.ATLAS_ERR_INVALID_INPUT, "tensor info")
            name = ctypes.string_at(info.name, info.name_len).decode()
            tensors.append(GgufTensor(name, tuple(int(d) for d in info.dims[: info.n_dims]), int(info.type),
                                      int(info.offset), int(info.bytes), i))
        self.tensors = tensors
        self.metadata = {}
        kp, kn, vp, vn = ctypes.c_void_p(), ctypes.c_uint64(), ctypes.c_void_p(), ctypes.c_uint64()
        for i in range(lib.atlas_gguf_metadata_count(handle)):
            lib.atlas_gguf_metadata_entry(handle, i, ctypes.byref(kp), ctypes.byref(kn), ctypes.byref(vp),
                                          ctypes.byref(vn))
            self.metadata[_text(kp, kn)] = _text(vp, vn)
        self.metadata_arrays = {}
        for i in range(lib.atlas_gguf_metadata_array_count(handle)):
            key, value = self._array(i)
            self.metadata_arrays[key] = value

    # -- construction (GgufModel::open / from_bytes) -------------------------
    @classmethod
    def open(cls, path) -> "GgufModel":
        lib = _lib.load()
        h, err = ctypes.c_void_p(), ctypes.create_string_buffer(512)
        rc = lib.atlas_gguf_open(str(path).encode(), ctypes.byref(h), err, len(err))
        if rc != 0:
            raise OperatorError(rc, err.value.decode(errors="replace"))
        return cls._finish(h, lib)

    @classmethod
    def from_bytes(cls, data: bytes) -> "GgufModel":
        lib = _lib.load()
        buf = (ctypes.c_uint8 * max(len(data), 1)).from_buffer_copy(bytes(data) or b"\0")
        h, err = ctypes.c_void_p(), ctypes.create_string_buffer(512)
        rc = lib.atlas_gguf_from_bytes(buf, len(data), ctypes.byref(h), err, len(err))
        if rc != 0:
            raise OperatorError(rc, err.value.decode(errors="replace"))
        return cls._finish(h, lib)

    @classmethod
    def _finish(cls, h, lib):
        return cls(h, lib)

    def close(self) -> None:
        if self._h:
            self._lib.atlas_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- queries ---------------------------------------------------------------
    def tensor(self, name: str) -> GgufTensor:
        i = self._lib.atlas_gguf_find_tensor(self._h, name.encode())
        if i < 0:
            raise KeyError(name)
        return self.tensors[i]

    def tensor_data(self, tensor: GgufTensor) -> np.ndarray:
        """The encoded bytes (GgufModel::tensor_data, gguf.rs:226-235): a read-only uint8 view of
        the mapped file, valid until close()."""
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        rc = self._lib.atlas_gguf_tensor_data(self._h, tensor.index, ctypes.byref(p), ctypes.byref(n))
        if rc != 0:
            raise OperatorError(rc, "tensor data")
        view = np.ctypeslib.as_array((ctypes.c_uint8 * n.value).from_address(p.value)) if n.value else np.empty(0, np.uint8)
        view.flags.writeable = False
        return view

    def _array(self, index):
        kp, kn, t, n, p = ctypes.c_void_p(), ctypes.c_uint64(), ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_void_p()
        rc = self._lib.atlas_gguf_metadata_array_entry(self._h, index, ctypes.byref(kp), ctypes.byref(kn),
                                                       ctypes.byref(t), ctypes.byref(n), ctypes.byref(p))
        if rc != 0:
            raise OperatorError(rc, "metadata array")
        key = _text(kp, kn)
        if t.value == 8:
            sp, sn, out = ctypes.c_void_p(), ctypes.c_uint64(), []
            for e in range(n.value):
                self._lib.atlas_gguf_metadata_array_string(self._h, index, e, ctypes.byref(sp), ctypes.byref(sn))
                out.append(_text(sp, sn))
            return key, out
        dtype = np.dtype(_ARRAY_DTYPES[t.value])
        if n.value == 0:
            return key, np.empty(0, dtype)
        raw = np.ctypeslib.as_array((ctypes.c_uint8 * (n.value * dtype.itemsize)).from_address(p.value))
        return key, raw.view(dtype).copy()

    def metadata_array(self, key: str):
        """GgufMetadataArray (gguf.rs:89-100): a list of str, or a numpy array; KeyError when absent."""
        i = self._lib.atlas_gguf_find_metadata_array(self._h, key.encode())
        if i < 0:
            raise KeyError(key)
        return self._array(i)[1]

    def upload(self, runtime: HipRuntime, tensor: GgufTensor) -> DeviceBuffer:
        """Copy the tensor's encoded bytes to a new device buffer (synchronous)."""
        buf = runtime.alloc(max(tensor.bytes, 16), np.uint8)
        runtime._check(self._lib.atlas_gguf_upload_tensor(runtime.ctx, self._h, tensor.index, buf.ptr))
        return buf
