"""The no-allocation soft cap + argmax entry point
(atlas_hip_softcap_argmax_f32_noalloc) through the C ABI: on two calls in a
row, the second smaller, its outputs equal atlas_hip_softcap_argmax_f32's
bit for bit (capped logits) and exactly (selected ids); sizes beyond its
static scratch are rejected with InvalidInput."""
import ctypes
import sys

import numpy as np
import pytest

from atlas_amd import OperatorError
from atlas_amd import workloads as wl

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-noalloc] {msg}", flush=True)
    sys.stdout.flush()


def _both(rt, logits, rows, count, cap, capped_out=True):
    """(capped, selected) from the existing entry point and from the variant."""
    lg = rt.upload(logits)
    out = []
    for name in ("atlas_hip_softcap_argmax_f32", "atlas_hip_softcap_argmax_f32_noalloc"):
        capped = rt.empty(rows * count) if capped_out else None
        sel = rt.empty(rows, np.uint32)
        rt.memset(sel, 0xFF, rows * 4)
        fn = getattr(rt.lib, name)
        cptr = ctypes.c_void_p(capped.ptr) if capped is not None else None
        rt._check(fn(rt.ctx, ctypes.c_void_p(lg.ptr), cptr, ctypes.c_void_p(sel.ptr), rows, count, cap))
        rt.sync()
        out.append((capped.download(rows * count) if capped is not None else None, sel.download(rows, np.uint32)))
    return out


def test_noalloc_softcap_argmax_matches_existing_entry_point(rt):
    r = wl.rng(909)
    calls = [(256, 262144, True),     # the C5 decode tail: exactly fills the scratch
             (7, 50001, True),        # second call, smaller and ragged (scalar path)
             (1, 262144, False),      # one token, argmax only
             (33, 4096, True)]
    for rows, count, keep in calls:
        logits = wl.normal(r, rows * count, 0.0, 10.0)
        logits[::997] = logits.max() + 1.0                   # ties of the maximum: the later index wins
        say(f"softcap+argmax rows={rows} count={count} capped={keep}")
        (ca, sa), (cb, sb) = _both(rt, logits, rows, count, 30.0, keep)
        assert np.array_equal(sa, sb), (rows, count)
        if keep:
            assert np.array_equal(ca.view(np.uint32), cb.view(np.uint32)), (rows, count)


def test_noalloc_rejects_sizes_beyond_its_scratch(rt):
    rows, count = 512, 262144
    say("softcap+argmax beyond the scratch")
    lg, sel = rt.empty(rows * count), rt.empty(rows, np.uint32)
    with pytest.raises(OperatorError) as e:
        rt.softcap_argmax_noalloc(lg, None, sel, rows, count, 30.0)
    assert e.value.kind == "InvalidInput"
    with pytest.raises(OperatorError) as e:
        rt.softcap_argmax_noalloc(lg, None, sel, 1, 16, 0.0)   # the cap must be finite and positive
    assert e.value.kind == "InvalidInput"


def test_noalloc_allocates_nothing_and_replays_in_a_graph(rt):
    """The entry point's defining property: the library's allocation count
    and resident bytes do not move across calls, eager or recorded into a
    HIP graph; the recorded call replays (with eager work between the
    replays) to the existing entry point's results every time."""
    rows, count, cap = 64, 262144, 30.0
    logits = wl.normal(wl.rng(910), rows * count, 0.0, 10.0)
    lg = rt.upload(logits)
    ref_c, ref_s = rt.empty(rows * count), rt.empty(rows, np.uint32)
    rt.softcap_argmax(lg, ref_c, ref_s, rows, count, cap)
    rt.sync()
    exp_c, exp_s = ref_c.download(rows * count), ref_s.download(rows, np.uint32)
    capped, sel = rt.empty(rows * count), rt.empty(rows, np.uint32)

    def held(t):
        return t.allocations, t.resident_bytes

    say("noalloc eager: telemetry")
    before = held(rt.telemetry())
    rt.softcap_argmax_noalloc(lg, capped, sel, rows, count, cap)
    rt.sync()
    assert held(rt.telemetry()) == before
    assert np.array_equal(sel.download(rows, np.uint32), exp_s)
    say("noalloc recorded into a graph")
    rt.graph_begin()
    rt.softcap_argmax_noalloc(lg, capped, sel, rows, count, cap)
    g = rt.graph_end()
    assert held(rt.telemetry()) == before
    try:
        for i in range(3):
            rt.memset(capped, 0, rows * count * 4)
            rt.memset(sel, 0xFF, rows * 4)
            rt.sync()
            say(f"graph replay {i}")
            rt.graph_launch(g)
            rt.sync()
            assert np.array_equal(sel.download(rows, np.uint32), exp_s), i
            assert np.array_equal(capped.download(rows * count).view(np.uint32), exp_c.view(np.uint32)), i
    finally:
        rt.graph_destroy(g)
    assert held(rt.telemetry()) == before


def test_noalloc_rows_of_one_workgroup_at_any_count(rt):
    """Rows that fit one workgroup use no scratch slots, so more rows than
    one launch's 65535 are accepted (two launches) and match the existing
    entry point."""
    rows, count = 65537, 1024
    say(f"softcap+argmax rows={rows} count={count}")
    logits = wl.normal(wl.rng(911), rows * count, 0.0, 10.0)
    (ca, sa), (cb, sb) = _both(rt, logits, rows, count, 30.0, True)
    assert np.array_equal(sa, sb)
    assert np.array_equal(ca.view(np.uint32), cb.view(np.uint32))
