"""CPU checks of the C ABI: the library loads, exports exactly what
include/atlas_hip_ops.h and include/atlas_gguf.h declare, behaves like MetalError::NoDevice when no
GPU is present, and its host-only helpers (RoPE tables) agree bit-for-bit
with the oracle.  No kernel is launched here."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import atlas_amd
from atlas_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("atlas_hip_ops.h", "atlas_gguf.h")]


def declared_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
        names |= set(re.findall(r"\b(atlas_(?:hip|ops|rope|gguf)_\w+)\s*\(", text))
    return sorted(names)


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    return {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert len(names) >= 50
    exported = exported_symbols()
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    lib = atlas_amd.load()
    for n in names:
        assert hasattr(lib, n)
    # the Python binding declares a signature for every C entry point
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_library_has_no_oracle_or_cpu_fallback_symbols():
    exported = exported_symbols()
    assert not [s for s in exported if s.startswith("oracle_")]
    out = subprocess.run(["ldd", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    assert "liboracle" not in out


def test_gfx950_code_object_present():
    sections = subprocess.run(["readelf", "-S", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    assert ".hip_fatbin" in sections
    assert b"amdgcn-amd-amdhsa--gfx950" in open(_lib.LIB_PATH, "rb").read()


def _has_gpu():
    n = ctypes.c_int(0)
    atlas_amd.load().atlas_hip_device_count(ctypes.byref(n))
    return n.value > 0


def test_no_device_and_null_context_errors():
    lib = atlas_amd.load()
    if _has_gpu():
        pytest.skip("a GPU is visible; NoDevice path not reachable")
    ctx = ctypes.c_void_p()
    assert lib.atlas_hip_init(0, ctypes.byref(ctx)) == atlas_amd.ATLAS_ERR_NO_DEVICE
    with pytest.raises(atlas_amd.OperatorError) as e:
        atlas_amd.NeuralOps()
    assert e.value.kind == "NoDevice"
    # a null context is invalid input, never a crash
    assert lib.atlas_hip_sync(None) == atlas_amd.ATLAS_ERR_INVALID_INPUT
    assert lib.atlas_hip_rms_norm_f32(None, None, None, None, 1, 1, 1e-5) == atlas_amd.ATLAS_ERR_INVALID_INPUT
    assert lib.atlas_hip_set_reduction(None, 0) == atlas_amd.ATLAS_ERR_INVALID_INPUT


def test_host_rope_tables_match_oracle(ora):
    pos = np.array([0, 1, 2, 100, 4095, 65536, 131071], np.uint32)
    for pairs, rot, theta in [(128, 256, 1e4), (128, 256, 1e6), (256, 512, 1e6), (256, 256, 1e4), (64, 128, 1e4)]:
        a = atlas_amd.rope_tables_gemma4(pos, pairs, rot, theta)
        b = ora.rope_tables_gemma4(pos, pairs, rot, theta)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    ff = np.linspace(1, 3, 128).astype(np.float32)
    a = atlas_amd.rope_tables_gemma4(pos, 128, 256, 1e6, ff)
    b = ora.rope_tables_gemma4(pos, 128, 256, 1e6, ff)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    for d, theta in [(64, 1e4), (64, 130000.0)]:
        a = atlas_amd.rope_tables_llama(pos, d, theta)
        b = ora.rope_tables_llama(pos, d, theta)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    with pytest.raises(atlas_amd.OperatorError):
        atlas_amd.rope_tables_llama(pos, 63, 1e4)
