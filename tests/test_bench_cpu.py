"""bench.py's CPU baseline (the C oracle timed on host threads): the fields
the bench line carries, on a short budget.  Runs without a GPU."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from atlas_amd import workloads as wl  # noqa: E402


def test_cpu_baseline_fields_single_and_threaded():
    out = bench.cpu_baseline(wl, budget_s=0.3, max_threads=2)
    assert set(out) >= {"value", "unit", "cores", "kind", "sample", "single_thread"}
    assert out["unit"] == "tokens/s" and out["kind"] == "port"
    assert 1 <= out["cores"] <= 2
    assert out["value"] > 0 and out["single_thread"] > 0
    if out["cores"] == 1:
        assert out["value"] == out["single_thread"]


def test_stream_floor_library_exports():
    """The measurement-only floor library bench.py loads: built, loadable
    without a GPU, and exporting the entry points bench.py binds."""
    import ctypes
    path = os.path.join(ROOT, "atlas_amd", "libatlas_stream_floor.so")
    assert os.path.exists(path), "run __graft_entry__.build() first"
    lib = ctypes.CDLL(path)
    for name in ("atlas_floor_stream_kind", "atlas_floor_kinds", "atlas_floor_launch"):
        assert hasattr(lib, name), name
    assert lib.atlas_floor_kinds() == 3
