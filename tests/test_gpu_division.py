"""Exhaustive GPU check of the activations' in-range division
(device_common.hpp, div_inrange; enumeration in division_check.hip).

GELU's tanh and SiLU divide with a four-operation reciprocal form in their
straight-line (in-range) branches instead of the IEEE division.  That form is
not correctly rounded for every operand pair, so each product helper is run on
every binary32 input of the domain its branch admits, once with the IEEE
division and once with the in-range one, and the bits must agree everywhere.
Two planted mistakes run beside it: without the correction step every domain
must show differences, and without the sign step SiLU must (silu(-0) is -0),
so the comparison is able to see a wrong quotient."""
import ctypes
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# inputs per domain: every finite float; every float with a finite GELU
# argument (|x| below ~1.9e12); every float with |x| < 87
FINITE = (1 << 32) - 2 * (1 << 23)
BELOW_87 = 2 * int(np.array([87.0], np.float32).view(np.uint32)[0])


def _lib():
    path = os.path.join(ROOT, "atlas_amd", "libatlas_division_check.so")
    if not os.path.exists(path):
        raise RuntimeError("libatlas_division_check.so is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    lib.atlas_division_check.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_uint64)]
    lib.atlas_division_check.restype = ctypes.c_int
    return lib


def _gelu_domain_size():
    """Floats whose argument 0.7978845608 * (x + 0.044715 x^3) is finite, in
    float32 as the kernel evaluates it: the largest such |x| is found by
    bisection over the bit patterns (the argument grows with |x|)."""
    def finite(bits):
        x = np.array([bits], np.uint32).view(np.float32)
        with np.errstate(over="ignore", invalid="ignore"):
            a = np.float32(0.7978845608) * (x + np.float32(0.044715) * x * x * x)
        return bool(np.isfinite(a[0]))
    lo, hi = 0, 0x7F800000  # finite(lo), not finite(hi)
    while hi - lo > 1:
        mid = (lo + hi) // 2
        lo, hi = (mid, hi) if finite(mid) else (lo, mid)
    return 2 * (lo + 1)


@pytest.mark.gpu
@pytest.mark.parametrize("domain,name", [(0, "tanh"), (1, "gelu"), (2, "silu")])
def test_in_range_division_is_ieee_on_whole_domain(domain, name):
    counts = (ctypes.c_uint64 * 4)()
    print(f"division check: {name}", flush=True)
    rc = _lib().atlas_division_check(domain, counts)
    assert rc == 0, f"atlas_division_check({domain}) returned {rc}"
    inputs, bad, bad_product, bad_sign = (int(c) for c in counts)
    expected = {0: FINITE, 1: _gelu_domain_size(), 2: BELOW_87}[domain]
    assert inputs == expected, (name, inputs, expected)
    assert bad == 0, f"{name}: {bad} inputs differ from the IEEE division"
    assert bad_product > 1000, (name, bad_product)   # planted: no correction step
    if domain == 2:
        assert bad_sign >= 1, (name, bad_sign)       # planted: silu(-0) loses its sign
