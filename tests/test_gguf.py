"""CPU tests of the GGUF v3 reader (include/atlas_gguf.h, atlas_amd/csrc/gguf.cpp).

The reader must accept exactly the files atlas_core::gguf::GgufModel accepts
(crates/atlas-core/src/gguf.rs:112-225) and read the same tensors, offsets,
sizes, bytes and metadata strings from them.  The checker is the Python
restatement in oracle/gguf_oracle.py; the reference's own GGUF tests
(crates/atlas-core/tests/phase_11a_gguf.rs:99-120) are restated first.
"""
import struct

import numpy as np
import pytest

import gguf_oracle as go
from atlas_amd import OperatorError
from atlas_amd.gguf import Q4_0, Q6_K, Q8_0, F16, F32, GgufModel

f32 = np.float32


def agree(data):
    """The product reader and the restatement accept/reject alike and agree on content."""
    try:
        exp = go.parse(data)
    except go.GgufReject as e:
        with pytest.raises(OperatorError) as got:
            GgufModel.from_bytes(data)
        assert got.value.kind == "InvalidInput"
        return str(e), str(got.value)
    m = GgufModel.from_bytes(data)
    assert m.metadata == exp["metadata"]
    assert sorted(m.metadata_arrays) == sorted(exp["arrays"])
    for k, (t, vals) in exp["arrays"].items():
        got = m.metadata_arrays[k]
        if t == 8:
            assert got == vals
        else:
            assert list(np.asarray(got).tolist()) == [bool(v) if t == 7 else v for v in vals] or \
                np.array_equal(np.asarray(got, np.float64), np.asarray(vals, np.float64), equal_nan=True)
    assert len(m.tensors) == len(exp["tensors"])
    for a, b in zip(m.tensors, exp["tensors"]):
        assert (a.name, a.dims, a.tensor_type, a.offset, a.bytes) == (b["name"], b["dims"], b["type"], b["offset"],
                                                                      b["bytes"])
        assert bytes(m.tensor_data(a)) == b["data"]
    m.close()
    return None


def q4_bytes(r, rows, cols):
    return r.integers(0, 256, rows * cols // 32 * 18, dtype=np.uint8).tobytes()


def sample_file(r):
    w = go.Writer()
    w.meta("llama.block_count", "1")
    w.push_tensor("blk.0.attn_q.weight", [32, 32], Q4_0, q4_bytes(r, 32, 32))
    w.push_tensor("token_embd.weight", [256, 8], Q6_K, r.integers(0, 256, 8 * 210, dtype=np.uint8).tobytes())
    w.push_tensor("output_norm.weight", [32], F32, r.standard_normal(32).astype(f32).tobytes())
    w.push_tensor("rope_freqs.weight", [7], F16, r.integers(0, 256, 14, dtype=np.uint8).tobytes())
    w.push_tensor("blk.0.ffn_down.weight", [64, 2], Q8_0, r.integers(0, 256, 4 * 34, dtype=np.uint8).tobytes())
    return w.finish()


# -------------------------------------------------- reference tests restated

def test_writer_and_reader_preserve_aligned_packed_tensors():
    """phase_11a_gguf.rs:99-115."""
    w = go.Writer()
    w.meta("llama.block_count", "1")
    w.push_tensor("blk.0.attn_q.weight", [32, 32], Q4_0, q4_bytes(np.random.default_rng(0), 32, 32))
    m = GgufModel.from_bytes(w.finish())
    assert m.metadata["general.architecture"] == "llama"
    assert m.tensors[0].tensor_type == Q4_0
    assert len(m.tensor_data(m.tensors[0])) == 32 * 18


def test_malformed_gguf_is_rejected_before_tensor_access():
    """phase_11a_gguf.rs:117-120."""
    with pytest.raises(OperatorError):
        GgufModel.from_bytes(b"GGUF\x03\0\0\0")


# ------------------------------------------------------------- acceptance

def test_sample_file_agrees_with_restatement_and_open(tmp_path):
    r = np.random.default_rng(1)
    data = sample_file(r)
    assert agree(data) is None
    p = tmp_path / "model.gguf"
    p.write_bytes(data)
    m = GgufModel.open(p)
    exp = go.parse(data)
    assert [t.name for t in m.tensors] == [t["name"] for t in exp["tensors"]]
    for a, b in zip(m.tensors, exp["tensors"]):
        assert bytes(m.tensor_data(a)) == b["data"]
    assert m.tensor("token_embd.weight").dims == (256, 8)
    with pytest.raises(KeyError):
        m.tensor("absent")
    with pytest.raises(OperatorError):
        GgufModel.open(tmp_path / "missing.gguf")
    (tmp_path / "empty.gguf").write_bytes(b"")
    with pytest.raises(OperatorError):
        GgufModel.open(tmp_path / "empty.gguf")


def test_metadata_scalars_keep_the_reference_string_form():
    w = go.RawWriter()
    cases = [
        ("u8", 0, 255, "255"), ("i8", 1, -128, "-128"), ("u16", 2, 65535, "65535"), ("i16", 3, -32768, "-32768"),
        ("u32", 4, 4294967295, "4294967295"), ("i32", 5, -2147483648, "-2147483648"),
        ("f32.cap", 6, 30.0, "30"), ("f32.eps", 6, 1e-6, "0.000001"), ("f32.tenth", 6, 0.1, "0.1"),
        ("f32.negzero", 6, -0.0, "-0"), ("f32.max", 6, 3.4028234663852886e38, "340282350000000000000000000000000000000"),
        ("f32.tiny", 6, 1.401298464324817e-45, "0." + "0" * 44 + "1"), ("f32.nan", 6, float("nan"), "NaN"),
        ("f32.ninf", 6, float("-inf"), "-inf"), ("f32.theta", 6, 1000000.0, "1000000"),
        ("bool.t", 7, True, "true"), ("bool.f", 7, False, "false"), ("str", 8, "gemma4", "gemma4"),
        ("u64", 10, 2 ** 64 - 1, str(2 ** 64 - 1)), ("i64", 11, -2 ** 63, str(-2 ** 63)),
        ("f64.tenth", 12, 0.1, "0.1"), ("f64.big", 12, 1e300, "1" + "0" * 300),
    ]
    for key, t, v, _ in cases:
        w.scalar(key, t, v)
    data = w.finish()
    assert agree(data) is None
    m = GgufModel.from_bytes(data)
    for key, _, _, text in cases:
        assert m.metadata[key] == text, key


def test_metadata_arrays_kept_and_dropped():
    w = go.RawWriter()
    w.array("tokenizer.ggml.tokens", 8, ["<pad>", "hello", "wörld", ""])
    w.array("scores", 6, [0.5, -1.25, 3.0])
    w.array("i32s", 5, [-1, 2, -3])
    w.array("u32s", 4, [1, 2, 4294967295])
    w.array("u64s", 10, [2 ** 64 - 1])
    w.array("i64s", 11, [-2 ** 63, 7])
    w.array("flags", 7, [True, False, True])
    w.array("dropped.u8", 0, [1, 2, 3])
    w.array("dropped.f64", 12, [1.5])
    w.array("empty", 6, [])
    data = w.finish()
    assert agree(data) is None
    m = GgufModel.from_bytes(data)
    assert m.metadata_arrays["tokenizer.ggml.tokens"] == ["<pad>", "hello", "wörld", ""]
    assert list(m.metadata_arrays["scores"]) == [0.5, -1.25, 3.0]
    assert list(m.metadata_arrays["u64s"]) == [2 ** 64 - 1]
    assert list(m.metadata_arrays["flags"]) == [True, False, True]
    assert "dropped.u8" not in m.metadata_arrays and "dropped.f64" not in m.metadata_arrays
    assert len(m.metadata_arrays["empty"]) == 0


# ------------------------------------------------------------- rejections

def _one_tensor(ttype=Q4_0, dims=(32, 2), offset=0, data=None, rank=None):
    w = go.RawWriter()
    if data is None:
        data = b"\x11" * go.encoded_bytes(ttype, int(np.prod(dims)))
    w.tensor("t", list(dims), ttype, offset, data)
    if rank is not None:
        w.infos[-1] = (go._str("t") + struct.pack("<I", rank) + b"".join(struct.pack("<Q", d) for d in dims)
                       + struct.pack("<IQ", ttype, offset))
    return w


REJECTS = {
    "magic": lambda: go.RawWriter(magic=b"GGUG").finish(),
    "version 2": lambda: go.RawWriter(version=2).finish(),
    "truncated header": lambda: b"GGUF\x03\0\0\0",
    "empty": lambda: b"",
    "tensor count": lambda: (lambda w: (setattr(w, "counts", (1_000_001, 0)), w.finish())[1])(go.RawWriter()),
    "metadata count": lambda: (lambda w: (setattr(w, "counts", (0, 1_000_001)), w.finish())[1])(go.RawWriter()),
    "utf8 key": lambda: go.RawWriter().raw_meta(go._str(b"\xc0\xaf") + struct.pack("<I", 4) + b"\0" * 4).finish(),
    "utf8 surrogate": lambda: go.RawWriter().scalar("k", 8, b"\xed\xa0\x80").finish(),
    "utf8 above max": lambda: go.RawWriter().scalar("k", 8, b"\xf4\x90\x80\x80").finish(),
    "metadata type 13": lambda: go.RawWriter().raw_meta(go._str("k") + struct.pack("<I", 13)).finish(),
    "nested array": lambda: go.RawWriter().raw_meta(go._str("k") + struct.pack("<IIQ", 9, 9, 1)
                                                     + struct.pack("<IQ", 4, 0)).finish(),
    "array elem type 13": lambda: go.RawWriter().raw_meta(go._str("k") + struct.pack("<IIQ", 9, 13, 1)).finish(),
    "rank 0": lambda: _one_tensor(rank=0, dims=(), data=b"").finish(),
    "rank 5": lambda: _one_tensor(dims=(32, 1, 1, 1, 1)).finish(),
    "zero dim": lambda: _one_tensor(dims=(32, 0), data=b"").finish(),
    "element overflow": lambda: _one_tensor(dims=(2 ** 32, 2 ** 32, 2), data=b"").finish(),
    "type Q4_1": lambda: _one_tensor(ttype=3, data=b"").finish(),
    "type 15": lambda: _one_tensor(ttype=15, data=b"").finish(),
    "q4 not block multiple": lambda: _one_tensor(dims=(33,), data=b"").finish(),
    "q6 not block multiple": lambda: _one_tensor(ttype=Q6_K, dims=(128,), data=b"").finish(),
    "unaligned offset": lambda: _one_tensor(offset=16).finish(),
    "alignment 64": lambda: _one_tensor().scalar("general.alignment", 4, 64).finish(),
    "alignment text": lambda: _one_tensor().scalar("general.alignment", 8, "32 ").finish(),
    "outside the file": lambda: _one_tensor(dims=(32, 4), data=b"\x11" * 36).finish(),
    "byte size overflow": lambda: _one_tensor(ttype=F32, dims=(2 ** 62, 4), data=b"").finish(),
    "overlap": lambda: go.RawWriter().tensor("a", [32, 2], Q4_0, 0, b"\1" * 36)
                                     .tensor("b", [32], Q4_0, 32, b"\2" * 18).finish(),
}


@pytest.mark.parametrize("case", sorted(REJECTS))
def test_rejected_like_the_reference(case):
    data = REJECTS[case]()
    with pytest.raises(go.GgufReject):
        go.parse(data)
    agree(data)


def test_alignment_forms_accepted():
    for t, v in [(4, 32), (8, "32"), (8, "+32"), (10, 32), (6, 32.0)]:
        data = _one_tensor().scalar("general.alignment", t, v).finish()
        assert agree(data) is None, (t, v)


def test_every_strict_prefix_is_rejected():
    data = sample_file(np.random.default_rng(2))
    for n in range(0, len(data)):
        with pytest.raises(OperatorError):
            GgufModel.from_bytes(data[:n])


def test_mutation_fuzz_agrees_with_restatement():
    """Random corruptions of a valid file: the product reader and the
    restatement must agree on accept / reject and, when accepted, on content."""
    r = np.random.default_rng(3)
    base = bytearray(sample_file(r))
    header_end = go.parse(bytes(base))["data_start"]
    outcomes = {"accepted": 0, "rejected": 0}
    for trial in range(1500):
        data = bytearray(base)
        kind = trial % 4
        if kind == 0:  # flip bytes in the header
            for _ in range(int(r.integers(1, 4))):
                data[int(r.integers(0, header_end))] ^= int(r.integers(1, 256))
        elif kind == 1:  # overwrite a little-endian length / count / offset field with a nearby value
            at = int(r.integers(0, header_end - 8))
            v = struct.unpack_from("<Q", data, at)[0]
            struct.pack_into("<Q", data, at, (v + int(r.integers(-40, 40))) % 2 ** 64)
        elif kind == 2:  # set a u32 to a small random value (types, ranks)
            at = int(r.integers(0, header_end - 4))
            struct.pack_into("<I", data, at, int(r.integers(0, 20)))
        else:  # truncate or extend
            data = data[:int(r.integers(0, len(data)))] if r.random() < 0.5 else data + bytes(int(r.integers(1, 64)))
        outcomes["accepted" if agree(bytes(data)) is None else "rejected"] += 1
    assert outcomes["accepted"] > 50 and outcomes["rejected"] > 500, outcomes
