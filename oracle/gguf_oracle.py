"""GGUF v3 reader and writer restated in Python -- TEST INFRASTRUCTURE ONLY.

The parity checker for the product reader (atlas_amd/csrc/gguf.cpp): a
second, independent restatement of atlas_core::gguf
(crates/atlas-core/src/gguf.rs), used by tests/ to decide which files the
reference accepts and what it reads from them.  The product never imports
it.

  parse(data)      GgufModel::from_bytes (gguf.rs:116-225) with Reader
                   (:439-568); returns a dict or raises GgufReject.
  Writer           GgufWriter (gguf.rs:237-311): every metadata value is
                   written as a string (type 8), keys in sorted order,
                   general.alignment = "32" and general.architecture = "llama"
                   set by default, tensor data 32-byte aligned.
  RawWriter        builds files field by field (typed metadata, arbitrary
                   offsets) for the rejection and formatting tests.
"""
from __future__ import annotations

import struct

import numpy as np

ALIGN = 32
BLOCK_BYTES = {0: 4, 1: 2, 2: 18, 8: 34, 14: 210}


class GgufReject(ValueError):
    pass


def encoded_bytes(ttype, elements):
    """GgufTensorType::encoded_bytes (gguf.rs:56-77)."""
    if ttype in (0, 1):
        return elements * BLOCK_BYTES[ttype]
    block = 256 if ttype == 14 else 32
    if elements % block:
        raise GgufReject(f"packed GGUF tensor has {elements} elements, not a multiple of {block}")
    return elements // block * BLOCK_BYTES[ttype]


def rust_f32(v):
    """Rust's Display for f32: shortest round-trip digits, positional."""
    v = np.float32(v)
    if np.isnan(v):
        return "NaN"
    if np.isinf(v):
        return "inf" if v > 0 else "-inf"
    return np.format_float_positional(v, unique=True, trim="-")


def rust_f64(v):
    v = np.float64(v)
    if np.isnan(v):
        return "NaN"
    if np.isinf(v):
        return "inf" if v > 0 else "-inf"
    return np.format_float_positional(v, unique=True, trim="-")


def _rust_parse_usize(s):
    body = s[1:] if s.startswith("+") else s
    if not body or not body.isascii() or not body.isdigit():
        return None
    v = int(body)
    return v if v < 2 ** 64 else None


class _Reader:
    def __init__(self, data):
        self.data = data
        self.at = 0

    def take(self, n):
        if self.at + n > len(self.data):
            raise GgufReject("truncated GGUF")
        b = self.data[self.at:self.at + n]
        self.at += n
        return b

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def string(self):
        n = self.u64()
        raw = self.take(n)
        try:
            return raw.decode("utf-8", errors="strict")
        except UnicodeDecodeError:
            raise GgufReject("GGUF string is not UTF-8") from None

    def value(self, t):
        if t == 0:
            return str(self.take(1)[0])
        if t == 1:
            return str(struct.unpack("<b", self.take(1))[0])
        if t == 2:
            return str(struct.unpack("<H", self.take(2))[0])
        if t == 3:
            return str(struct.unpack("<h", self.take(2))[0])
        if t == 4:
            return str(self.u32())
        if t == 5:
            return str(struct.unpack("<i", self.take(4))[0])
        if t == 6:
            return rust_f32(struct.unpack("<f", self.take(4))[0])
        if t == 7:
            return "true" if self.take(1)[0] != 0 else "false"
        if t == 8:
            return self.string()
        if t == 9:
            raise GgufReject("GGUF array must be read through metadata_array")
        if t == 10:
            return str(self.u64())
        if t == 11:
            return str(struct.unpack("<q", self.take(8))[0])
        if t == 12:
            return rust_f64(struct.unpack("<d", self.take(8))[0])
        raise GgufReject(f"unsupported GGUF metadata type {t}")

    def array(self):
        t = self.u32()
        n = self.u64()
        if t == 8:
            return t, [self.string() for _ in range(n)]
        fmt = {6: "<f", 5: "<i", 4: "<I", 10: "<Q", 11: "<q"}.get(t)
        if fmt:
            size = struct.calcsize(fmt)
            return t, [struct.unpack(fmt, self.take(size))[0] for _ in range(n)]
        if t == 7:
            return t, [self.take(1)[0] != 0 for _ in range(n)]
        for _ in range(n):
            self.value(t)
        return None


def parse(data: bytes) -> dict:
    """GgufModel::from_bytes (gguf.rs:116-225)."""
    r = _Reader(bytes(data))
    if r.take(4) != b"GGUF":
        raise GgufReject("GGUF magic is missing")
    if r.u32() != 3:
        raise GgufReject("only GGUF v3 is supported")
    tensor_count = r.u64()
    metadata_count = r.u64()
    if tensor_count > 1_000_000 or metadata_count > 1_000_000:
        raise GgufReject("GGUF count is unreasonable")
    metadata, arrays = {}, {}
    for _ in range(metadata_count):
        key = r.string()
        t = r.u32()
        if t == 9:
            a = r.array()
            if a is not None:
                arrays[key] = a
        else:
            metadata[key] = r.value(t)
    tensors = []
    for _ in range(tensor_count):
        name = r.string()
        rank = r.u32()
        if rank == 0 or rank > 4:
            raise GgufReject(f"GGUF tensor {name} has invalid rank {rank}")
        dims, elements = [], 1
        for _ in range(rank):
            d = r.u64()
            if d == 0:
                raise GgufReject(f"GGUF tensor {name} has zero dimension")
            elements *= d
            if elements >= 2 ** 64:
                raise GgufReject("GGUF element count overflows")
            dims.append(d)
        ttype = r.u32()
        if ttype not in BLOCK_BYTES:
            raise GgufReject(f"unsupported GGUF tensor type {ttype}")
        offset = r.u64()
        if offset % ALIGN:
            raise GgufReject(f"GGUF tensor {name} offset is not aligned")
        nbytes = encoded_bytes(ttype, elements)
        if nbytes >= 2 ** 64:
            raise GgufReject("GGUF tensor byte size overflows")
        tensors.append({"name": name, "dims": tuple(dims), "type": ttype, "offset": offset, "bytes": nbytes})
    if "general.alignment" in metadata:
        a = _rust_parse_usize(metadata["general.alignment"])
        if a is None:
            raise GgufReject("invalid general.alignment")
        if a != ALIGN:
            raise GgufReject(f"Atlas requires GGUF alignment {ALIGN}, got {a}")
    data_start = (r.at + ALIGN - 1) // ALIGN * ALIGN
    ranges = []
    for t in tensors:
        start = data_start + t["offset"]
        end = start + t["bytes"]
        if start >= 2 ** 64 or end >= 2 ** 64:
            raise GgufReject("GGUF tensor range overflows")
        if end > len(data):
            raise GgufReject(f"GGUF tensor {t['name']} is outside the file")
        ranges.append((start, end, t["name"]))
    ranges.sort(key=lambda x: x[0])
    for a, b in zip(ranges, ranges[1:]):
        if a[1] > b[0]:
            raise GgufReject(f"GGUF tensors {a[2]} and {b[2]} overlap")
    for t in tensors:
        s = data_start + t["offset"]
        t["data"] = bytes(data[s:s + t["bytes"]])
    return {"metadata": metadata, "arrays": arrays, "tensors": tensors, "data_start": data_start}


# ------------------------------------------------------------------ writers

def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


class Writer:
    """GgufWriter (gguf.rs:237-311)."""

    def __init__(self):
        self.metadata = {"general.alignment": "32", "general.architecture": "llama"}
        self.tensors = []

    def meta(self, key, value):
        self.metadata[key] = value

    def push_tensor(self, name, dims, ttype, data):
        elements = int(np.prod(dims))
        data = bytes(data)
        if len(data) != encoded_bytes(ttype, elements):
            raise GgufReject("GGUF tensor data length differs from dimensions")
        self.tensors.append((name, list(dims), ttype, data))

    def finish(self) -> bytes:
        out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(self.tensors), len(self.metadata)))
        for k in sorted(self.metadata):
            out += _str(k) + struct.pack("<I", 8) + _str(self.metadata[k])
        offsets, off = [], 0
        for _, _, _, data in self.tensors:
            off = (off + ALIGN - 1) // ALIGN * ALIGN
            offsets.append(off)
            off += len(data)
        for (name, dims, ttype, _), o in zip(self.tensors, offsets):
            out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", ttype, o)
        for _, _, _, data in self.tensors:
            out += b"\0" * ((-len(out)) % ALIGN)
            out += data
        return bytes(out)


class RawWriter:
    """Field-by-field GGUF builder: typed metadata, explicit offsets, no checks."""

    SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}

    def __init__(self, version=3, magic=b"GGUF"):
        self.magic, self.version = magic, version
        self.meta = []     # encoded key/value records
        self.infos = []    # encoded tensor-info records
        self.blobs = []    # (offset, bytes)
        self.counts = None

    def scalar(self, key, t, value):
        if t == 7:
            payload = bytes([1 if value else 0])
        elif t == 8:
            payload = _str(value)
        else:
            payload = struct.pack(self.SCALAR[t], value)
        self.meta.append(_str(key) + struct.pack("<I", t) + payload)
        return self

    def array(self, key, t, values):
        if t == 8:
            body = b"".join(_str(v) for v in values)
        elif t == 7:
            body = bytes(1 if v else 0 for v in values)
        else:
            body = b"".join(struct.pack(self.SCALAR[t], v) for v in values)
        self.meta.append(_str(key) + struct.pack("<IIQ", 9, t, len(values)) + body)
        return self

    def raw_meta(self, record: bytes):
        self.meta.append(record)
        return self

    def tensor(self, name, dims, ttype, offset, data=None):
        rec = _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        self.infos.append(rec + struct.pack("<IQ", ttype, offset))
        if data is not None:
            self.blobs.append((offset, bytes(data)))
        return self

    def finish(self, trailing=b"") -> bytes:
        nt, nm = self.counts if self.counts else (len(self.infos), len(self.meta))
        out = bytearray(self.magic + struct.pack("<IQQ", self.version, nt, nm))
        for m in self.meta:
            out += m
        for t in self.infos:
            out += t
        start = (len(out) + ALIGN - 1) // ALIGN * ALIGN
        end = max([start + o + len(b) for o, b in self.blobs], default=start if self.blobs else len(out))
        out += b"\0" * (end - len(out))
        for o, b in self.blobs:
            out[start + o:start + o + len(b)] = b
        return bytes(out) + trailing
