"""bench.py's CPU baseline (the C oracle timed on host threads): the fields
the bench line carries, on a short budget.  Runs without a GPU."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from atlas_amd import workloads as wl  # noqa: E402


def test_cpu_baseline_fields_single_and_threaded():
    """On small inputs (the field layout does not depend on the sizes)."""
    import numpy as np
    L, Q = wl.GemmaLayerShape(), wl.QuantGatherShape()
    T, H, D, QH, F = L.tokens, L.hidden, L.head_dim, L.q_heads, L.ffn
    r = wl.rng(1)
    ple_row = Q.ple_layers * Q.ple_width
    vocab = Q.vocab
    # full-vocabulary tables are large; a table of 512 rows with ids below 512 exercises the same calls
    host = {"q4": wl.q4_0_table(r, 512, H), "q6": wl.q6_k_table(r, 512, H), "ple": wl.q4_0_table(r, 512, ple_row),
            "ids": wl.token_ids(r, T, 512), "w": wl.normal(r, H, 1.0, 0.1), "qw": wl.normal(r, D, 1.0, 0.1),
            "kw": wl.normal(r, D, 1.0, 0.1), "x": wl.normal(r, T * H), "res": wl.normal(r, T * H),
            "q": wl.normal(r, T * QH * D), "k": wl.normal(r, T * D), "gate": wl.normal(r, T * F),
            "up": wl.normal(r, T * F), "proj": wl.normal(r, T * ple_row)}
    assert vocab >= 512 and host["ids"].max() < 512
    out = bench.cpu_baseline(wl, budget_s=0.05, max_threads=2, host=host)
    assert set(out) >= {"value", "unit", "cores", "kind", "sample", "single_thread", "ops"}
    assert out["unit"] == "tokens/s" and out["kind"] == "port"
    assert 1 <= out["cores"] <= 2
    assert out["value"] > 0 and out["single_thread"] > 0
    assert set(out["ops"]) == {"embed_q4_0", "embed_q6_k", "ple_q4_0", "rms_norm", "qk_norm_rope", "rms_residual",
                               "geglu"}
    for op in out["ops"].values():
        assert op["GB/s_1core"] > 0 and np.isfinite(op["tokens_per_s_1core"])


def test_stream_floor_library_exports():
    """The measurement-only floor library bench.py loads: built, loadable
    without a GPU, and exporting the entry points bench.py binds."""
    import ctypes
    path = os.path.join(ROOT, "atlas_amd", "libatlas_stream_floor.so")
    assert os.path.exists(path), "run __graft_entry__.build() first"
    lib = ctypes.CDLL(path)
    for name in ("atlas_floor_stream_kind", "atlas_floor_kinds", "atlas_floor_launch", "atlas_floor_gather",
                 "atlas_floor_stream_policy", "atlas_floor_policy_count"):
        assert hasattr(lib, name), name
    assert lib.atlas_floor_kinds() == 3


def test_division_check_library_exports():
    """The test-only enumeration library the GPU division test loads: built
    and exporting its entry point (no call without a GPU)."""
    import ctypes
    path = os.path.join(ROOT, "atlas_amd", "libatlas_division_check.so")
    assert os.path.exists(path), "run __graft_entry__.build() first"
    assert hasattr(ctypes.CDLL(path), "atlas_division_check")


def test_buffer_sets_carved_from_one_arena():
    """Every op's rotating sets are views into one arena allocation: each
    tensor 4 KiB aligned, tensors and sets disjoint, set 0 uploaded and the
    others copied from it, and a request larger than the arena refused."""
    import numpy as np

    class View:
        def __init__(self, ptr, nbytes, dtype):
            self.ptr, self.nbytes, self.dtype = ptr, nbytes, np.dtype(dtype)
            self.uploaded = None

        def offset(self, off, dtype=None):
            return View(self.ptr + off, self.nbytes - off, dtype if dtype is not None else self.dtype)

        def upload(self, host):
            self.uploaded = host.nbytes
            return self

    class FakeRuntime:
        def __init__(self):
            self.copies = []

        def alloc(self, nbytes, dtype=np.float32):
            return View(1 << 20, nbytes, dtype)

        def copy(self, dst, src, nbytes):
            self.copies.append((dst.ptr, src.ptr, nbytes))

        def sync(self):
            pass

    ops = object.__new__(bench.Ops)
    ops.host = {"x": np.zeros(1000, np.float32), "ids": np.zeros(7, np.uint32)}
    ops.table = {"op": (["x", "ids"], {"y": 5000}, 0, None)}
    rt = FakeRuntime()
    per_set = ops.sets_bytes(["op"], 1)
    arena = bench.Arena(rt, ops.sets_bytes(["op"], 3))
    sets = ops.build_sets(rt, ["op"], 3, arena)
    spans = []
    for i, s in enumerate(sets):
        for k, v in s.items():
            assert (v.ptr - arena.buf.ptr) % 4096 == 0
            size = ops.host[k].nbytes if k in ops.host else 5000 * 4
            spans.append((v.ptr, v.ptr + size))
            assert arena.buf.ptr + i * per_set <= v.ptr and v.ptr + size <= arena.buf.ptr + (i + 1) * per_set
        assert s["ids"].dtype == np.uint32 and s["y"].dtype == np.float32
    spans.sort()
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))
    assert sets[0]["x"].uploaded == 4000 and sets[0]["ids"].uploaded == 28
    assert len(rt.copies) == 2 * 2 and all(n in (4000, 28) for _, _, n in rt.copies)
    try:
        ops.build_sets(rt, ["op"], 4, arena)
    except RuntimeError:
        pass
    else:
        raise AssertionError("a request beyond the arena must be refused")


def test_bound_launches_make_the_same_library_calls():
    """bench.py times each op through bind_launch: the runtime method runs
    once against a recorder, and the timed loop replays the recorded C-ABI
    calls (same entry point, same converted arguments, return codes still
    checked); a launcher that makes no library call is refused."""
    import ctypes

    import pytest

    from atlas_amd.runtime import HipRuntime, _ptr

    made = []

    class Entry:
        argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_float]

        def __call__(self, *args):
            made.append(args)
            return 0

    class Lib:
        atlas_hip_rms_norm_f32 = Entry()

    class FakeRuntime(HipRuntime):
        def __init__(self):  # no device: only what the recorder reads
            self.lib, self.ctx = Lib(), ctypes.c_void_p(0x1000)

        def probe(self, x, n, eps):
            self._check(self.lib.atlas_hip_rms_norm_f32(self.ctx, _ptr(x), n, eps))

    rt = FakeRuntime()
    calls = bench.bind_launch(rt, lambda r, s: r.probe(s["x"], 7, 1e-6), {"x": 0x2000})
    assert len(calls) == 1 and made == []          # recorded, not made
    fn, args = calls[0]
    assert fn is Lib.atlas_hip_rms_norm_f32
    assert [type(a) for a in args] == Entry.argtypes
    assert args[1].value == 0x2000 and args[2].value == 7 and abs(args[3].value - 1e-6) < 1e-12
    bench.run_bound(rt, calls)
    bench.run_bound(rt, calls)
    assert len(made) == 2 and all(a is b for a, b in zip(made[0], made[1]))   # the same converted arguments
    with pytest.raises(RuntimeError):
        bench.bind_launch(rt, lambda r, s: None, {})
