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
