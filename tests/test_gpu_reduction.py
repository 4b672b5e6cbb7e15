"""GPU tests of the library's default reduction (ATLAS_REDUCTION_AUTO) through
the C ABI.

AUTO sums a row's squares as a tree where the output is a plain scaled row:
RMSNorm (f32, f16) and the y output of the pre-norm add+RMSNorm.  There the
contract is north_star's floating-point tolerance against the reference CPU
operator (crates/atlas-ops/tests/phase_02_operators.rs:223-242):

  * f32: every element within 1e-5 relative of the sequential CPU fold.  On
    rows where the sequential fold itself carries a systematic rounding error
    (constant-magnitude rows) an element also passes when it lies within
    2e-6 relative of the float64 RMSNorm, i.e. closer to the exact value
    than the CPU operator is;
  * f16: within one f16 ulp of the CPU operator's output (the only rounding
    that can move is the final one);
  * the stored residual stream (add-norm's residual_out) does not depend on
    the reduction and stays bit-identical.

Where an epilogue can cancel (post-norm residual add, PLE add-scale) AUTO
keeps the sequential fold, and those outputs stay bit-identical.
"""
import sys

import numpy as np
import pytest

import cases
from atlas_amd import ATLAS_REDUCTION_AUTO, ATLAS_REDUCTION_WIDE
from cases import adversarial_f16_rows, adversarial_rows, assert_bits

pytestmark = pytest.mark.gpu
f32 = np.float32
REL = 1e-5          # north_star: norm ops within 1e-5 relative of the CPU operator
REL_F64 = 2e-6      # or closer to the exact float64 value than that


def say(msg):
    print(f"[gpu-reduction] {msg}", flush=True)
    sys.stdout.flush()


def rms_f64(x, w, rows, hidden, eps):
    x64 = x.astype(np.float64).reshape(rows, hidden)
    with np.errstate(over="ignore", invalid="ignore"):
        inv = 1.0 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + eps)
        return (x64 * inv * w.astype(np.float64)).reshape(-1)


def assert_rms_tolerance(name, got, exp, exact):
    """Elementwise: NaN where the oracle has NaN, equal infinities and zeros,
    otherwise within REL of the oracle or within REL_F64 of float64."""
    got, exp = np.asarray(got, np.float64), np.asarray(exp, np.float64)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan), f"{name}: NaN positions differ"
    inf = np.isinf(exp)
    assert np.array_equal(got[inf], exp[inf]), f"{name}: infinities differ"
    fin = ~nan & ~inf
    g, e, x = got[fin], exp[fin], exact[fin]
    with np.errstate(invalid="ignore", divide="ignore"):
        rel = np.where(e == 0, np.abs(g), np.abs(g - e) / np.abs(e))
        rel64 = np.where(x == 0, np.abs(g), np.abs(g - x) / np.abs(x))
    bad = (rel > REL) & ~(rel64 <= REL_F64)
    if bad.any():
        j = int(np.nonzero(bad)[0][0])
        raise AssertionError(f"{name}: {int(bad.sum())} of {g.size} elements beyond tolerance; first: gpu={g[j]!r} "
                             f"oracle={e[j]!r} f64={x[j]!r} rel={rel[j]:.3e}")
    return float(rel.max()) if rel.size else 0.0


@pytest.mark.parametrize("name", ["c1_rms_norm", "c3_rms_norm"])
def test_auto_rms_golden_within_tolerance(rt_auto, ora, name):
    """BASELINE C1 [128, 576] and C3 [4096, 1536] (two rows per wavefront)."""
    build, _ = cases.golden_cases()[name]
    inp, m = build()
    say(f"auto {name} {m}")
    got = cases.rms_gpu(rt_auto, inp, m)[0]
    exp = cases.rms_oracle(ora, inp, m)[0]
    worst = assert_rms_tolerance(name, got, exp, rms_f64(inp["x"], inp["w"], m["rows"], m["hidden"], m["eps"]))
    # on the configs' Gaussian rows the tree sum is within a few ulps of the fold
    assert worst < 3e-6, worst


@pytest.mark.parametrize("rows,hidden", [(1, 4), (3, 7), (5, 576), (33, 2048), (256, 1536), (17, 2304), (2, 8192),
                                         (4093, 1536), (4096, 1536), (4097, 1536), (2050, 2048), (4100, 576),
                                         (8192, 260)])
@pytest.mark.parametrize("mode", ["plain", "addnorm"])
def test_auto_tree_modes_ragged(rt_auto, ora, rows, hidden, mode):
    """The tree engine (one or two rows per wavefront, ragged columns and the
    odd last row), the scalar wide engine for unaligned widths and > 2048."""
    inp, m = cases.rms_case(rows, hidden, 1e-6, 1000 + rows + hidden, mode)
    say(f"auto rms {mode} rows={rows} hidden={hidden}")
    got = cases.rms_gpu(rt_auto, inp, m)
    exp = cases.rms_oracle(ora, inp, m)
    if mode == "plain":
        assert_rms_tolerance("plain", got[0], exp[0], rms_f64(inp["x"], inp["w"], rows, hidden, 1e-6))
    else:
        assert_bits("residual_out", [got[0]], [exp[0]])
        assert_rms_tolerance("add-norm y", got[1], exp[1], rms_f64(exp[0], inp["w"], rows, hidden, 1e-6))


@pytest.mark.parametrize("rows", [4096 + 48, 1024 + 16])
@pytest.mark.parametrize("hidden", [1536, 2048, 576, 260])
def test_auto_tree_adversarial_rows(rt_auto, ora, rows, hidden):
    """The exact-fold stress rows (ties, binade crossings, zeros, subnormal and
    overflowing squares, inf, NaN, constant rows) through the tree engine."""
    inp, m = cases.rms_case(rows, hidden, 1e-6, 4000 + hidden, "plain")
    inp["x"] = adversarial_rows(rows, hidden, 5000 + hidden)
    say(f"auto rms adversarial rows={rows} hidden={hidden}")
    got = cases.rms_gpu(rt_auto, inp, m)[0]
    exp = cases.rms_oracle(ora, inp, m)[0]
    assert_rms_tolerance("adversarial plain", got, exp, rms_f64(inp["x"], inp["w"], rows, hidden, 1e-6))


@pytest.mark.parametrize("mode", ["residual", "addscale"])
@pytest.mark.parametrize("rows,hidden", [(4096, 1536), (256, 1536), (33, 576)])
def test_auto_cancelling_epilogues_stay_bit_exact(rt_auto, ora, mode, rows, hidden):
    """AUTO keeps the sequential fold where the epilogue can cancel."""
    inp, m = cases.rms_case(rows, hidden, 1e-6, 3000 + rows + hidden, mode)
    say(f"auto rms {mode} rows={rows} hidden={hidden}")
    assert_bits(f"auto {mode}", cases.rms_gpu(rt_auto, inp, m), cases.rms_oracle(ora, inp, m))


def test_auto_in_place_and_aliased(rt_auto, ora):
    """x == out for the plain norm and residual_out == x for the add-norm, at
    the two-rows-per-wavefront size (row w + G is loaded before row w is
    stored)."""
    rows, h, eps = 4096, 1536, 1e-6
    inp, m = cases.rms_case(rows, h, eps, 4242, "addnorm")
    exact = rms_f64(inp["x"], inp["w"], rows, h, eps)
    say("auto rms in place")
    work, w = rt_auto.upload(inp["x"]), rt_auto.upload(inp["w"])
    rt_auto.rms_norm(work, w, work, rows, h, eps)
    rt_auto.sync()
    assert_rms_tolerance("in place", work.download(rows * h), ora.rms_norm(inp["x"], inp["w"], rows, h, eps), exact)
    say("auto add+norm with residual_out == x")
    a, res, y = rt_auto.upload(inp["x"]), rt_auto.upload(inp["res"]), rt_auto.empty(rows * h)
    rt_auto.add_rms_norm(a, res, w, a, y, rows, h, eps)
    rt_auto.sync()
    rs_exp, y_exp = ora.add_rms_norm(inp["x"], inp["res"], inp["w"], rows, h, eps)
    assert_bits("residual_out in place", [a.download(rows * h)], [rs_exp])
    assert_rms_tolerance("y", y.download(rows * h), y_exp, rms_f64(rs_exp, inp["w"], rows, h, eps))


def _assert_f16_within_one_ulp(name, got, exp):
    g, e = got.view(np.float16).astype(np.float64), exp.view(np.float16).astype(np.float64)
    nan = np.isnan(e)
    assert np.array_equal(np.isnan(g), nan), f"{name}: NaN positions differ"
    fin = ~nan & np.isfinite(e)
    assert np.array_equal(g[~nan & ~fin], e[~nan & ~fin]), f"{name}: infinities differ"
    ulp = np.spacing(np.abs(e[fin]).astype(np.float16)).astype(np.float64)
    bad = np.abs(g[fin] - e[fin]) > ulp
    if bad.any():
        j = int(np.nonzero(bad)[0][0])
        raise AssertionError(f"{name}: {int(bad.sum())} of {bad.size} beyond one f16 ulp; first gpu={g[fin][j]!r} "
                             f"oracle={e[fin][j]!r}")
    return float(np.mean(g[fin] != e[fin]))


def test_auto_f16_golden_c2(rt_auto, ora):
    """BASELINE C2 [2048, 2048] FP16 add+RMSNorm: residual_out bit-exact, y
    within one f16 ulp (and equal on all but a few near-tie elements)."""
    build, _ = cases.golden_cases()["c2_add_rms_norm_f16"]
    inp, m = build()
    say(f"auto c2 f16 {m}")
    got, exp = cases.f16_norm_gpu(rt_auto, inp, m), cases.f16_norm_oracle(ora, inp, m)
    assert_bits("residual_out", [got[0]], [exp[0]])
    differ = _assert_f16_within_one_ulp("add+norm y", got[1], exp[1])
    assert differ < 1e-2, differ
    _assert_f16_within_one_ulp("norm y", got[2], exp[2])


@pytest.mark.parametrize("rows,hidden", [(1, 8), (33, 576), (2050, 2048), (4096, 2048), (7, 4096), (19, 2056),
                                         (5, 1000), (3, 8200), (4100, 64)])
def test_auto_f16_shapes(rt_auto, ora, rows, hidden):
    inp, m = cases.f16_norm_case(rows, hidden, 1e-5, 7000 + rows + hidden)
    say(f"auto f16 norms rows={rows} hidden={hidden}")
    got, exp = cases.f16_norm_gpu(rt_auto, inp, m), cases.f16_norm_oracle(ora, inp, m)
    assert_bits("residual_out", [got[0]], [exp[0]])
    _assert_f16_within_one_ulp("add+norm y", got[1], exp[1])
    _assert_f16_within_one_ulp("norm y", got[2], exp[2])


@pytest.mark.parametrize("rows,hidden", [(2048 + 37, 2048), (4096 + 3, 2048), (300, 4096), (77, 1536)])
def test_auto_f16_adversarial_rows(rt_auto, ora, rows, hidden):
    inp, m = cases.f16_norm_case(rows, hidden, 1e-5, 7100 + rows + hidden)
    inp["x"] = adversarial_f16_rows(rows, hidden, 7200 + hidden)
    say(f"auto f16 adversarial rows={rows} hidden={hidden}")
    got, exp = cases.f16_norm_gpu(rt_auto, inp, m), cases.f16_norm_oracle(ora, inp, m)
    g16, e16 = got[0].view(np.float16), exp[0].view(np.float16)
    same = (got[0] == exp[0]) | (np.isnan(g16) & np.isnan(e16))
    assert same.all(), f"residual_out: {int((~same).sum())} of {same.size} differ"
    _assert_f16_within_one_ulp("add+norm y", got[1], exp[1])
    _assert_f16_within_one_ulp("norm y", got[2], exp[2])


def test_wide_tree_epilogues_normwise(rt_auto, ora):
    """ATLAS_REDUCTION_WIDE takes the tree engine for the cancelling epilogues
    too: the normalised row stays within 1e-5 relative per element, the
    epilogue outputs within 1e-6 normwise (an elementwise bound is not
    meaningful where residual + n cancels)."""
    rt_auto.set_reduction(ATLAS_REDUCTION_WIDE)
    try:
        for rows in (4096, 300):
            for mode in ("residual", "addscale"):
                inp, m = cases.rms_case(rows, 1536, 1e-6, 6100 + rows, mode)
                say(f"wide {mode} rows={rows}")
                got, exp = cases.rms_gpu(rt_auto, inp, m), cases.rms_oracle(ora, inp, m)
                if mode == "residual":
                    assert_rms_tolerance("wide normalized", got[0], exp[0],
                                         rms_f64(inp["x"], inp["w"], rows, 1536, 1e-6))
                assert np.linalg.norm(got[-1] - exp[-1]) / np.linalg.norm(exp[-1]) <= 1e-6
    finally:
        rt_auto.set_reduction(ATLAS_REDUCTION_AUTO)


@pytest.mark.parametrize("width,groups", [(256, 35), (250, 9), (2000, 5)])
def test_wide_groups_stable(rt_auto, ora, width, groups):
    """ATLAS_REDUCTION_WIDE sums the stable group norm's squares as a tree
    (the PLE projection always does): within 1e-6 relative of the
    sequential oracle per element; an all-zero group stays exactly zero."""
    r = np.random.default_rng(88 + width)
    v = r.standard_normal((groups, width)).astype(np.float32)
    v[1] = 0.0
    w = (1 + 0.1 * r.standard_normal(width)).astype(np.float32)
    rt_auto.set_reduction(ATLAS_REDUCTION_WIDE)
    try:
        say(f"wide groups stable width={width}")
        vb = rt_auto.upload(v)
        rt_auto.rms_norm_groups_stable(vb, rt_auto.upload(w), width, groups, 1e-6)
        rt_auto.sync()
        got = vb.download(v.size).reshape(groups, width)
    finally:
        rt_auto.set_reduction(ATLAS_REDUCTION_AUTO)
    exp = ora.rms_norm_groups_stable(v, w, width, groups, 1e-6).reshape(groups, width)
    assert np.all(got[1] == 0.0)
    assert np.max(np.abs(got - exp) / np.maximum(np.abs(exp), 1e-30)) <= 1e-6
