"""Pin the CPU oracle before it is trusted as the parity checker.

Each oracle function is checked against the reference's own known-answer
values (tests/golden/kats.json, transcribed from the reference tests), and
against what mathematics fixes: float64 evaluations, closed forms,
invariants and exhaustive / brute-force sweeps.  The checks are chosen so a
plausible mistake (dropped epsilon, wrong divisor, swapped pair, wrong nibble
or scale index, missing rounding step) fails at least one of them.
"""
import json
import os

import numpy as np
import pytest

import matvec_cases as mc

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "kats.json")))
f32 = np.float32


def ulp_err(actual, exact):
    actual = np.asarray(actual, np.float64)
    exact = np.asarray(exact, np.float64)
    spacing = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    return np.abs(actual - exact) / spacing


# --------------------------------------------------------------------- f16

def test_f16_decode_exhaustive(ora):
    codes = np.arange(65536, dtype=np.uint16)
    got = ora.f16_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_encode_is_ieee_rne(ora):
    r = np.random.default_rng(7)
    vals = np.concatenate([
        r.standard_normal(200000).astype(f32) * f32(100),
        r.uniform(-70000, 70000, 20000).astype(f32),
        (r.standard_normal(20000) * 1e-6).astype(f32),          # f16 subnormal range
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25, 1.0009765625 + 2.0 ** -11], f32),
    ])
    got = ora.f32_to_f16(vals)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    # Atlas's converter rounds 1.9999999 to 1.0 (carry bug); IEEE RNE gives 2.0.
    assert ora.f32_to_f16(np.array([1.9999999], f32))[0] == 0x4000


# --------------------------------------------------------------- exp / act

def test_expf_faithful_against_float64(ora):
    r = np.random.default_rng(3)
    xs = np.concatenate([r.uniform(-87, 88, 30000), r.uniform(-1, 1, 10000),
                         np.array([0.0, 1.0, -1.0, 0.5, -0.5, 88.0, -87.0])]).astype(f32)
    got = ora.expf(xs)
    err = ulp_err(got, np.exp(xs.astype(np.float64)))
    assert err.max() < 1.0, err.max()
    assert ora.expf(np.array([0.0], f32))[0] == 1.0
    assert np.isinf(ora.expf(np.array([89.5], f32))[0])
    assert ora.expf(np.array([-105.0], f32))[0] == 0.0
    sub = ora.expf(np.array([-100.0], f32))[0]            # subnormal result
    assert 0 < sub < np.finfo(np.float32).tiny
    assert abs(float(sub) - np.exp(-100.0)) <= 2.0 ** -149


def test_tanh_silu_against_float64(ora):
    lib = ora.lib()
    r = np.random.default_rng(5)
    xs = np.concatenate([r.uniform(-12, 12, 20000), r.uniform(-0.01, 0.01, 2000)]).astype(f32)
    t = np.array([lib.oracle_tanhf(float(x)) for x in xs], np.float64)
    assert np.max(np.abs(t - np.tanh(xs.astype(np.float64)))) < 2.5e-7
    s = ora.silu(xs).astype(np.float64)
    x64 = xs.astype(np.float64)
    exact = x64 / (1.0 + np.exp(-x64))
    assert ulp_err(s, exact).max() <= 4.0
    assert ora.silu(np.array([-200.0], f32))[0] == 0.0


def test_gelu_reference_extremes_and_formula(ora):
    kat = KATS["gelu_extremes"]
    x = np.array(kat["input"], f32)
    got = ora.gelu(x)
    assert np.all(np.isfinite(got))
    # phase_00_bootstrap.rs:137-141: CPU tanh formula, abs <= 1e-5
    a = f32(0.7978846) * (x + f32(0.044715) * x * x * x)
    exp_cpu = (f32(0.5) * x * (f32(1.0) + np.tanh(a))).astype(f32)
    assert np.max(np.abs(got - exp_cpu)) <= kat["tolerance"]
    r = np.random.default_rng(11)
    xs = r.uniform(-8, 8, 50000).astype(f32)
    x64 = xs.astype(np.float64)
    exact = 0.5 * x64 * (1 + np.tanh(0.7978845608 * (x64 + 0.044715 * x64 ** 3)))
    assert np.max(np.abs(ora.gelu(xs) - exact)) < 2e-6
    # the inf guard: x large negative -> 0, large positive -> x
    assert ora.gelu(np.array([-1e20], f32))[0] == 0.0
    assert ora.gelu(np.array([1e20], f32))[0] == f32(1e20)


def test_glu_is_activation_times_up(ora):
    r = np.random.default_rng(2)
    g, u = r.standard_normal(4096).astype(f32), r.standard_normal(4096).astype(f32)
    assert np.array_equal(ora.swiglu(g, u), ora.silu(g) * u)
    assert np.array_equal(ora.geglu(g, u), ora.gelu(g) * u)
    ple = r.standard_normal((3, 5 * 64)).astype(f32)
    gate = r.standard_normal((3, 64)).astype(f32)
    got = ora.geglu_offset(gate, ple, 2 * 64, 5 * 64, 64, 3).reshape(3, 64)
    assert np.array_equal(got, ora.gelu(gate).reshape(3, 64) * ple[:, 128:192])


# ----------------------------------------------------------------- RMSNorm

def rms_f64(x, w, eps):
    x64 = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
    return x64 * inv * w.astype(np.float64)


def test_rms_norm_reference_kat(ora):
    k = KATS["rms_norm"]
    x, w = np.array(k["input"], f32), np.array(k["weight"], f32)
    got = ora.rms_norm(x, w, k["rows"], k["hidden"], k["epsilon"]).reshape(2, 4)
    exact = rms_f64(x.reshape(2, 4), w, k["epsilon"])
    assert np.max(np.abs(got - exact)) <= k["tolerance"]
    assert np.max(np.abs(got - exact) / np.abs(exact)) < 1e-6


def test_rms_norm_math_and_invariants(ora):
    r = np.random.default_rng(4)
    rows, h = 64, 1536
    x = r.standard_normal((rows, h)).astype(f32)
    w = (1 + 0.1 * r.standard_normal(h)).astype(f32)
    y = ora.rms_norm(x, w, rows, h, 1e-6).reshape(rows, h)
    assert np.max(np.abs(y - rms_f64(x, w, 1e-6)) / np.abs(rms_f64(x, w, 1e-6))) < 5e-6
    # scale invariance (eps negligible) and unit RMS of y / w
    y2 = ora.rms_norm(x * f32(8), w, rows, h, 1e-6).reshape(rows, h)
    assert np.max(np.abs(y2 - y) / np.abs(y)) < 1e-5
    assert np.allclose(np.sqrt(np.mean((y / w).astype(np.float64) ** 2, axis=1)), 1.0, atol=1e-5)
    # sequential f32 fold: equal to a float32 cumulative sum in index order
    sq = (x * x).astype(f32)
    seq = np.cumsum(sq, axis=1, dtype=np.float32)[:, -1]
    lib = ora.lib()
    for i in range(4):
        row = np.ascontiguousarray(x[i])
        inv = lib.oracle_inverse_rms(row.ctypes.data, h, f32(1e-6))
        assert inv == f32(1) / np.sqrt(seq[i] / f32(h) + f32(1e-6))


def test_fused_epilogues_equal_unfused_chains(ora):
    r = np.random.default_rng(9)
    rows, h, eps = 16, 1536, 1e-6
    x = r.standard_normal(rows * h).astype(f32)
    w = (1 + 0.1 * r.standard_normal(h)).astype(f32)
    res = r.standard_normal(rows * h).astype(f32)
    n = ora.rms_norm(x, w, rows, h, eps)
    # post-norm residual epilogue == rms_norm then vector_add
    nn, out = ora.rms_norm_residual(x, w, res, rows, h, eps)
    assert np.array_equal(nn, n) and np.array_equal(out, res + n)
    # pre-norm add + norm == vector_add then rms_norm
    rs, y = ora.add_rms_norm(x, res, w, rows, h, eps)
    assert np.array_equal(rs, x + res)
    assert np.array_equal(y, ora.rms_norm(x + res, w, rows, h, eps))
    # PLE epilogue == norm, add, scale
    st = ora.rms_norm_add_scale(x, w, res, f32(0.37), rows, h, eps)
    assert np.array_equal(st, ((res + n) * f32(0.37)).astype(f32))


def test_groups_stable(ora):
    r = np.random.default_rng(12)
    width, groups = 256, 20
    v = r.standard_normal((groups, width)).astype(f32)
    v[3] = 0.0
    v[5] *= f32(1e30)   # x*x would overflow without the max scaling
    w = (1 + 0.1 * r.standard_normal(width)).astype(f32)
    got = ora.rms_norm_groups_stable(v, w, width, groups, 1e-6).reshape(groups, width)
    assert np.all(got[3] == 0.0)
    assert np.all(np.isfinite(got))
    exact = rms_f64(v.astype(np.float64), w, 1e-6)
    ok = np.arange(groups) != 3
    assert np.max(np.abs(got[ok] - exact[ok]) / np.maximum(np.abs(exact[ok]), 1e-30)) < 5e-6


def test_f16_norms_are_widen_compute_round(ora):
    r = np.random.default_rng(13)
    rows, h = 8, 2048
    x = r.standard_normal(rows * h).astype(np.float16).view(np.uint16)
    res = r.standard_normal(rows * h).astype(np.float16).view(np.uint16)
    w = (1 + 0.1 * r.standard_normal(h)).astype(np.float16).view(np.uint16)
    got = ora.rms_norm_f16(x, w, rows, h, 1e-5)
    ref = ora.f32_to_f16(ora.rms_norm(ora.f16_to_f32(x), ora.f16_to_f32(w), rows, h, 1e-5))
    assert np.array_equal(got, ref)
    rs, y = ora.add_rms_norm_f16(x, res, w, rows, h, 1e-5)
    stored = ora.f32_to_f16(ora.f16_to_f32(x) + ora.f16_to_f32(res))
    assert np.array_equal(rs, stored)
    assert np.array_equal(y, ora.f32_to_f16(ora.rms_norm(ora.f16_to_f32(stored), ora.f16_to_f32(w), rows, h, 1e-5)))
    g = r.standard_normal(4096).astype(np.float16).view(np.uint16)
    u = r.standard_normal(4096).astype(np.float16).view(np.uint16)
    assert np.array_equal(ora.swiglu_f16(g, u), ora.f32_to_f16(ora.swiglu(ora.f16_to_f32(g), ora.f16_to_f32(u))))


# -------------------------------------------------------------------- RoPE

def test_rope_reference_kat(ora):
    k = KATS["rope"]
    x = np.array(k["input"], f32)
    c, s = np.array(k["cos"], f32), np.array(k["sin"], f32)
    got = ora.rope_interleaved(x, k["rows"], k["hidden"], c, s)
    x64 = x.reshape(2, 2, 2).astype(np.float64)
    exp = np.stack([x64[..., 0] * c - x64[..., 1] * s, x64[..., 0] * s + x64[..., 1] * c], -1).reshape(-1)
    assert np.max(np.abs(got - exp)) <= k["tolerance"]


def test_rope_angle_kats(ora):
    k = KATS["rope_angle"]
    n = k["normal"]
    assert ora.rope_angle(n["position"], n["pair"], n["rotary"], n["theta"], n["factor"]) == n["expected"]
    sp = k["suppressed"]
    assert abs(ora.rope_angle(sp["position"], sp["pair"], sp["rotary"], sp["theta"], sp["factor"])) < sp["abs_below"]
    o = k["outside_partial_width"]
    assert ora.rope_angle(o["position"], o["pair"], o["rotary"], o["theta"], o["factor"]) == o["expected"]
    c, s = ora.rope_tables_gemma4(np.array([0, 8], np.uint32), 128, 256, 1e6)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    assert c[1, 0] == np.float32(np.cos(np.float32(8.0)))
    c2, s2 = ora.rope_tables_llama(np.array([0, 5], np.uint32), 64, 1e4)
    assert np.all(c2[0] == 1.0) and np.all(s2[0] == 0.0)


def _angle_closed_form(pos, pairs, rotary, theta, factors):
    """theta_p = pos / theta^(2p/rotary) / factor_p in float64
    (gemma4_executor.rs:622-633; executor.rs:632-647 with rotary = head_dim)."""
    p = np.arange(pairs, dtype=np.float64)
    ang = pos.astype(np.float64)[:, None] / np.power(np.float64(theta), 2.0 * p / rotary)[None, :]
    return ang / factors.astype(np.float64)[None, :]


def _check_tables(cos, sin, pos, pairs, rotary, theta, factors):
    """Angles within 2 f32 ulp of the closed form on every pair 1..rotary/2-1;
    cos/sin within 1e-6 of float64 cos/sin of the table's own f32 angle."""
    exact = _angle_closed_form(pos, pairs, rotary, theta, factors)[:, 1:]
    # recover the f32 angle the table was built from: the closed form rounded to
    # f32 is within 2 ulp of it, so check cos/sin of that angle and of its
    # neighbours, and the angle itself through the closed form
    a32 = exact.astype(np.float32)
    spacing = np.spacing(np.abs(a32)).astype(np.float64)
    c, s = cos[:, 1:].astype(np.float64), sin[:, 1:].astype(np.float64)
    best = np.full(exact.shape, np.inf)
    for k in range(-2, 3):
        cand = a32.astype(np.float64) + k * spacing
        err = np.maximum(np.abs(c - np.cos(cand)), np.abs(s - np.sin(cand)))
        best = np.minimum(best, err)
    return float(best.max())


def test_rope_tables_angle_against_float64_closed_form(ora):
    """Pins the angle exponent (2p/rotary) on every pair > 0, which the pair-0
    KATs cannot see: table entries equal cos/sin of an f32 angle within 2 ulp
    of pos / theta^(2p/rotary) / factor (float64), at positions up to 131071,
    theta 1e4 / 1e6 / 130000, rotary 128 / 256 / 512, unit and non-unit
    per-pair factors.  A planted exponent p/rotary must fail the same check."""
    r = np.random.default_rng(41)
    pos = np.concatenate([np.array([1, 2, 3, 7, 100, 4095, 65535, 131071]),
                          r.integers(0, 131072, 24)]).astype(np.uint32)
    for rotary in (128, 256, 512):
        pairs = rotary // 2
        for theta in (1e4, 1e6, 130000.0):
            for factors in (np.ones(pairs, f32), r.uniform(0.5, 40.0, pairs).astype(f32)):
                c, s = ora.rope_tables_gemma4(pos, pairs, rotary, theta, factors)
                assert _check_tables(c, s, pos, pairs, rotary, theta, factors) < 1e-6, (rotary, theta)
        c, s = ora.rope_tables_llama(pos, rotary, 130000.0)
        assert _check_tables(c, s, pos, pairs, rotary, 130000.0, np.ones(pairs, f32)) < 1e-6
    # planted mistake: exponent p/rotary instead of 2p/rotary
    pairs, rotary, theta = 128, 256, 1e6
    p = np.arange(pairs, dtype=np.float32)
    wrong = pos.astype(np.float32)[:, None] / np.power(np.float32(theta), p / np.float32(rotary))[None, :]
    assert _check_tables(np.cos(wrong), np.sin(wrong), pos, pairs, rotary, theta, np.ones(pairs, f32)) > 1e-2
    # planted mistake: factor multiplied instead of divided
    ff = r.uniform(0.5, 40.0, pairs).astype(f32)
    c, s = ora.rope_tables_gemma4(pos, pairs, rotary, theta, np.ones(pairs, f32))
    ang = _angle_closed_form(pos, pairs, rotary, theta, np.ones(pairs, f32)) * ff.astype(np.float64)[None, :]
    assert _check_tables(np.cos(ang), np.sin(ang), pos, pairs, rotary, theta, ff) > 1e-2


def test_rope_angle_scalar_matches_closed_form(ora):
    """The scalar angle (the decode path's per-token entry) is within 2 f32
    ulp of the float64 closed form on pairs > 0 and is 0 from rotary/2 up."""
    r = np.random.default_rng(43)
    for _ in range(400):
        rotary = int(r.choice([128, 256, 512]))
        pair = int(r.integers(1, rotary // 2))
        pos = int(r.integers(0, 131072))
        theta = float(r.choice([1e4, 1e6, 130000.0]))
        factor = float(np.float32(r.uniform(0.5, 40.0)))
        got = ora.rope_angle(pos, pair, rotary, theta, factor)
        exact = pos / theta ** (2.0 * pair / rotary) / factor
        assert abs(got - exact) <= 2 * np.spacing(np.float32(abs(exact))), (pos, pair, rotary, theta, factor)
        assert ora.rope_angle(pos, rotary // 2 + pair % 7, rotary, theta, factor) == 0.0


def test_rope_half_equals_reference_three_kernel_chain(ora):
    """rope_half_to_interleaved -> rope_f32 -> rope_interleaved_to_half (kernels.metal:940-994)."""
    r = np.random.default_rng(14)
    tokens, heads, d = 5, 3, 64
    x = r.standard_normal((tokens, heads, d)).astype(f32)
    c, s = ora.rope_tables_llama(np.arange(tokens, dtype=np.uint32) * 7, d, 130000.0)
    got = ora.rope_half(x, c, s, tokens, heads, d, d // 2).reshape(tokens, heads, d)
    for t in range(tokens):
        inter = np.empty((heads, d), f32)
        inter[:, 0::2], inter[:, 1::2] = x[t, :, : d // 2], x[t, :, d // 2:]
        rot = ora.rope_interleaved(inter, heads, d, c[t], s[t]).reshape(heads, d)
        back = np.concatenate([rot[:, 0::2], rot[:, 1::2]], axis=1)
        assert np.array_equal(got[t], back)
    # pair norm preserved; identity at position 0
    n_in = x[..., : d // 2] ** 2 + x[..., d // 2:] ** 2
    n_out = got[..., : d // 2] ** 2 + got[..., d // 2:] ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5)
    assert np.array_equal(got[0], x[0])


def _np_rope_half_f16(x16, c, s, tokens, heads, d, stride):
    """numpy restatement: widen f16 exactly, rotate with separately rounded f32
    products and one f32 add/subtract, round once to f16 (IEEE RNE)."""
    x = x16.view(np.float16).astype(f32).reshape(tokens, heads, d)
    cc = c.reshape(tokens, stride)[:, None, : d // 2].astype(f32)
    ss = s.reshape(tokens, stride)[:, None, : d // 2].astype(f32)
    x0, x1 = x[..., : d // 2], x[..., d // 2:]
    with np.errstate(invalid="ignore", over="ignore"):
        lo = (x0 * cc).astype(f32) - (x1 * ss).astype(f32)
        hi = (x0 * ss).astype(f32) + (x1 * cc).astype(f32)
    return np.concatenate([lo, hi], -1).astype(np.float16).view(np.uint16).reshape(-1)


def test_rope_half_f16_is_widen_rotate_round(ora):
    """oracle_rope_half_f16 == f32_to_f16(rope_half(f16_to_f32(x))) bit for bit
    at the C2 shape [2048, 32, 64] (theta 130000), and equals an independent
    numpy restatement of the same steps.  The f32 rotation it composes is
    pinned by the reference three-kernel chain and the cpu_rope KAT above.
    Planted mistakes (products rounded to f16 before the subtraction; the
    pair partner taken from the wrong half) must fail."""
    r = np.random.default_rng(19)
    tokens, heads, d = 2048, 32, 64
    x16 = r.standard_normal(tokens * heads * d).astype(np.float16).view(np.uint16)
    # adversarial rows: exact cancellation, f16 subnormals, the f16 max, inf, nan
    x16[:64] = np.float16(1.0).view(np.uint16)
    x16[64:128] = np.array([6.0e-8, -6.0e-8, 65504.0, -65504.0] * 16, np.float16).view(np.uint16)
    x16[128:130] = np.array([np.inf, np.nan], np.float16).view(np.uint16)
    c, s = ora.rope_tables_llama(np.arange(tokens, dtype=np.uint32), d, 130000.0)
    got = ora.rope_half_f16(x16, c, s, tokens, heads, d, d // 2)
    composed = ora.f32_to_f16(ora.rope_half(ora.f16_to_f32(x16), c, s, tokens, heads, d, d // 2))
    assert np.array_equal(got, composed)
    ref = _np_rope_half_f16(x16, c, s, tokens, heads, d, d // 2)
    nan = np.isnan(ref.view(np.float16))
    assert np.array_equal(np.isnan(got.view(np.float16)), nan)
    assert np.array_equal(got[~nan], ref[~nan])
    # within one f16 ulp of the float64 rotation of the same f32 tables, plus
    # the f32 arithmetic's own bound (2^-23 of the operand magnitudes) where
    # the two products cancel
    x64 = x16.view(np.float16).astype(np.float64).reshape(tokens, heads, d)
    c64 = c.astype(np.float64)[:, None, :]
    s64 = s.astype(np.float64)[:, None, :]
    with np.errstate(invalid="ignore", over="ignore"):
        a0, a1 = x64[..., :32], x64[..., 32:]
        exact = np.concatenate([a0 * c64 - a1 * s64, a0 * s64 + a1 * c64], -1)
        mag = np.concatenate([np.abs(a0 * c64) + np.abs(a1 * s64), np.abs(a0 * s64) + np.abs(a1 * c64)], -1)
        g = got.view(np.float16).astype(np.float64).reshape(exact.shape)
        fin = np.isfinite(exact) & (np.abs(exact) < 65504)
        bound = np.spacing(np.abs(exact[fin]).astype(np.float16)).astype(np.float64) + 2.0 ** -23 * mag[fin]
    assert np.all(np.abs(g[fin] - exact[fin]) <= bound)
    with np.errstate(invalid="ignore", over="ignore"):
        # planted: each product rounded to f16 before the subtraction
        x = x16.view(np.float16).astype(f32).reshape(tokens, heads, d)
        cc, ss = c[:, None, :].astype(f32), s[:, None, :].astype(f32)
        r16 = lambda v: v.astype(np.float16).astype(f32)
        lo = r16(x[..., :32] * cc) - r16(x[..., 32:] * ss)
        hi = r16(x[..., :32] * ss) + r16(x[..., 32:] * cc)
        planted = np.concatenate([lo, hi], -1).astype(np.float16).view(np.uint16).reshape(-1)
        assert not np.array_equal(got[~nan], planted[~nan])
        # planted: interleaved partner (x[2p], x[2p+1]) instead of the half split
        xi = x.reshape(tokens, heads, 32, 2)
        lo = xi[..., 0] * cc - xi[..., 1] * ss
        hi = xi[..., 0] * ss + xi[..., 1] * cc
        planted = np.concatenate([lo, hi], -1).astype(np.float16).view(np.uint16).reshape(-1)
        assert not np.array_equal(got[~nan], planted[~nan])


def test_qk_norm_rope_equals_norm_then_rope(ora):
    r = np.random.default_rng(15)
    tokens, qh, d, eps = 6, 8, 256, 1e-6
    q = r.standard_normal((tokens, qh, d)).astype(f32)
    k = r.standard_normal((tokens, 1, d)).astype(f32)
    qw = (1 + 0.1 * r.standard_normal(d)).astype(f32)
    kw = (1 + 0.1 * r.standard_normal(d)).astype(f32)
    c, s = ora.rope_tables_gemma4(np.arange(tokens, dtype=np.uint32) + 100, 128, 256, 1e4)
    qo, ko = ora.qk_norm_rope(q, k, qw, kw, c, s, tokens, qh, True, d, 128, eps)
    qn = ora.rms_norm(q.reshape(-1, d), qw, tokens * qh, d, eps)
    kn = ora.rms_norm(k.reshape(-1, d), kw, tokens, d, eps)
    assert np.array_equal(qo, ora.rope_half(qn, c, s, tokens, qh, d, 128))
    assert np.array_equal(ko, ora.rope_half(kn, c, s, tokens, 1, d, 128))


# ---------------------------------------------------------- dequant/gathers

def test_q4_0_reference_kat(ora):
    k = KATS["q4_0"]
    block = np.zeros(18, np.uint8)
    block[0:2] = np.array([k["scale_bits"]], np.uint16).view(np.uint8)
    for i in range(16):
        block[2 + i] = (i & 15) | ((15 - i) << 4)
    got = ora.dequant_q4_0_block(block)
    for i in range(16):
        assert got[i] == i - 8.0 and got[i + 16] == 7.0 - i


def _q6k_kat_block():
    b = np.zeros(210, np.uint8)
    b[208:210] = np.array([0x3800], np.uint16).view(np.uint8)
    for index in range(256):
        value = index % 64
        half, within = index // 128, index % 128
        stream, lane = within // 32, within % 32
        ql = half * 64 + lane + (32 if stream % 2 == 1 else 0)
        b[ql] |= ((value & 0x0F) << 4) if stream >= 2 else (value & 0x0F)
        b[128 + half * 32 + lane] |= ((value >> 4) & 3) << (stream * 2)
    b[192:208] = 1
    return b


def test_q6_k_reference_kat_and_independent_decoder(ora):
    k = KATS["q6_k"]
    b = _q6k_kat_block()
    got = ora.dequant_q6_k_block(b)
    for idx, val in k["expected"].items():
        assert got[int(idx)] == val
    assert np.array_equal(got, ora.dequant_q6_k_block(b, llama_order=True))
    # the KAT layout encodes value = index % 64 -> (code - 32) * 1 * 0.5
    assert np.array_equal(got, ((np.arange(256) % 64) - 32).astype(f32) * f32(0.5))
    r = np.random.default_rng(16)
    for _ in range(200):
        blk = np.frombuffer(r.bytes(210), np.uint8).copy()
        blk[208:210] = np.array([np.float16(r.uniform(1e-4, 1))]).view(np.uint8)
        assert np.array_equal(ora.dequant_q6_k_block(blk), ora.dequant_q6_k_block(blk, llama_order=True))


def test_q8_0_reference_round_trip_and_brute_force(ora):
    """q4_and_q8_blocks_round_trip_without_full_dequantization
    (crates/atlas-core/tests/phase_11a_gguf.rs:33-54): values (i-16)/7 encoded
    to Q8_0 and decoded stay within 0.03.  Then every int8 code under random
    f16 scales equals the exact product int8 * f16 (gguf.rs:431-435), and a
    planted unsigned-byte decode fails."""
    vals = ((np.arange(32) - 16.0) / 7.0).astype(f32)
    block = np.zeros(34, np.uint8)
    ora.lib().oracle_encode_q8_0_block(vals.ctypes.data, block.ctypes.data)
    dec = ora.dequant_q8_0_block(block)
    assert np.max(np.abs(dec - vals)) <= 0.03
    r = np.random.default_rng(31)
    codes = np.arange(256, dtype=np.uint8)
    for _ in range(40):
        d = np.float16(r.uniform(1e-4, 4.0) * r.choice([-1, 1]))
        for chunk in range(8):
            b = np.zeros(34, np.uint8)
            b[0:2] = np.array([d]).view(np.uint8)
            b[2:] = codes[32 * chunk: 32 * chunk + 32]
            got = ora.dequant_q8_0_block(b)
            exact = b[2:].view(np.int8).astype(np.float64) * float(d)
            assert np.array_equal(got.astype(np.float64), exact)
            unsigned = b[2:].astype(np.float64) * float(d)
            if chunk >= 4:   # codes 128..255: the signed reading differs
                assert not np.array_equal(got.astype(np.float64), unsigned)
    # the gather: rows by id, ids >= vocab untouched, one rounding by the scale
    vocab, h = 9, 64
    table = np.frombuffer(r.bytes(vocab * 2 * 34), np.uint8).copy()
    table.reshape(vocab, 2, 34)[:, :, 0:2] = np.array([0.125], np.float16).view(np.uint8)
    ids = np.array([3, 9, 0, 8], np.uint32)
    got = ora.embed_q8_0(table, ids, vocab, h, 1.5, out=np.full(ids.size * h, -1.0, f32)).reshape(ids.size, h)
    rows = table.reshape(vocab, 2, 34)[:, :, 2:].view(np.int8).reshape(vocab, h).astype(f32) * f32(0.125)
    assert np.array_equal(got[0], rows[3] * f32(1.5)) and np.array_equal(got[2], rows[0] * f32(1.5))
    assert np.all(got[1] == -1.0)
    assert np.array_equal(got[3], rows[8] * f32(1.5))


def test_dequant_brute_force_every_code(ora):
    r = np.random.default_rng(17)
    for d in [np.float16(1.0), np.float16(0.0137), np.float16(-2.5), np.float16(6e-5)]:
        for nib in range(16):
            block = np.zeros(18, np.uint8)
            block[0:2] = np.array([d]).view(np.uint8)
            block[2:] = nib | (nib << 4)
            got = ora.dequant_q4_0_block(block)
            assert np.all(got == np.float64(nib - 8) * np.float64(d))  # exact in f32
    for _ in range(20):
        d = np.float16(r.uniform(-1, 1))
        sc = int(r.integers(-128, 128))
        for code in range(64):
            b = np.zeros(210, np.uint8)
            b[208:210] = np.array([d]).view(np.uint8)
            b[192:208] = np.array([sc], np.int8).view(np.uint8)[0]
            low, high = code & 15, code >> 4
            b[0:64] = low | (low << 4)
            b[64:128] = low | (low << 4)
            b[128:192] = high | (high << 2) | (high << 4) | (high << 6)
            got = ora.dequant_q6_k_block(b)
            assert np.all(got == np.float64(code - 32) * sc * np.float64(d))


def test_embedding_kat_and_gathers(ora):
    k = KATS["embedding"]
    got = ora.embed_f32(np.array(k["table"], f32), np.array(k["ids"], np.uint32), k["vocab"], k["hidden"])
    assert np.max(np.abs(got - np.array(k["expected"], f32))) <= k["tolerance"]
    assert np.array_equal(got, np.array(k["expected"], f32))  # a gather is a copy
    zero = ora.embed_f32(np.array(k["table"], f32), np.array([7], np.uint32), 3, 4)
    assert np.all(zero == 0.0)
    from atlas_amd import workloads as wl
    r = wl.rng(18)
    vocab, h, t = 64, 512, 9
    for q6 in (False, True):
        table = wl.q6_k_table(r, vocab, h) if q6 else wl.q4_0_table(r, vocab, h)
        ids = wl.token_ids(r, t, vocab)
        ids[2] = vocab + 5  # untouched row
        scale = wl.f32_sqrt(h)
        fn = ora.embed_q6_k if q6 else ora.embed_q4_0
        sentinel = np.full(t * h, 123.0, f32)
        got = fn(table, ids, vocab, h, scale, out=sentinel).reshape(t, h)
        rb = wl.q_row_bytes(h, q6)
        qk, bb = (256, 210) if q6 else (32, 18)
        for i, tok in enumerate(ids):
            if tok >= vocab:
                assert np.all(got[i] == 123.0)
                continue
            row = table[tok * rb:(tok + 1) * rb]
            deq = np.concatenate([
                (ora.dequant_q6_k_block if q6 else ora.dequant_q4_0_block)(row[b * bb:(b + 1) * bb])
                for b in range(h // qk)])
            assert np.array_equal(got[i], deq * scale)


def test_ple_combine_kat_and_chain(ora):
    k = KATS["ple_combine"]
    got = ora.combine_ple(np.array(k["identity"], f32), np.array(k["context"], f32))
    exp = np.array([6 / np.sqrt(2), -2 / np.sqrt(2)])
    assert np.max(np.abs(got - exp)) < k["tolerance"]
    from atlas_amd import workloads as wl
    assert np.float32(0.70710677) == wl.SQRT_2_RECIP
    r = wl.rng(19)
    vocab, layers, width, t = 32, 3, 256, 5
    for q6 in (False, True):
        table = wl.q6_k_table(r, vocab, layers * width) if q6 else wl.q4_0_table(r, vocab, layers * width)
        ids = wl.token_ids(r, t, vocab)
        proj = wl.normal(r, (t, layers, width))
        got = ora.ple(table, ids, proj, vocab, layers, width, f32(16.0), wl.SQRT_2_RECIP, q6=q6)
        lookup = (ora.embed_q6_k if q6 else ora.embed_q4_0)(table, ids, vocab, layers * width, 1.0)
        chain = ora.combine_ple(ora.scale(lookup, f32(16.0)), proj.reshape(-1))
        assert np.array_equal(got, chain)


# ------------------------------------------------- planted-mistake controls

def test_pins_catch_planted_mistakes(ora):
    """Run the same pins against deliberately wrong CPU variants; each must fail."""
    k = KATS["rms_norm"]
    x, w = np.array(k["input"], f32).reshape(2, 4), np.array(k["weight"], f32)
    exact = rms_f64(x, w, k["epsilon"])
    wrong_div = x / np.sqrt(np.sum(x * x, 1, keepdims=True) / 3 + f32(1e-5)) * w   # h-1 divisor
    assert np.max(np.abs(wrong_div - exact)) > k["tolerance"]
    kr = KATS["rope"]
    xr = np.array(kr["input"], f32).reshape(2, 2, 2)
    c, s = np.array(kr["cos"], f32), np.array(kr["sin"], f32)
    good = ora.rope_interleaved(xr, 2, 4, c, s)
    swapped_sign = np.stack([xr[..., 0] * c + xr[..., 1] * s, xr[..., 0] * s - xr[..., 1] * c], -1).reshape(-1)
    assert np.max(np.abs(good - swapped_sign)) > kr["tolerance"]
    b = _q6k_kat_block()
    wrong_scale_index = b.copy()
    wrong_scale_index[192] = 2  # scale of group 0 only: a wrong index must change values
    assert not np.array_equal(ora.dequant_q6_k_block(b), ora.dequant_q6_k_block(wrong_scale_index))


# ------------------------------------------------ RMS-folded Q4_0 projections

def test_matvec_q4_0_oracles_pinned(ora):
    """The f64 oracle equals an independent numpy decode + float64 matvec; the
    f32 reference-test oracle (normalise, then sequential matvec) stays within
    the sequential-accumulation bound of it; a one-hot input has a closed form."""
    import matvec_cases as mc
    r = np.random.default_rng(31)
    n, rows, eps = 256, 40, 1e-6
    x = r.standard_normal(n).astype(f32)
    w = (1.0 + 0.1 * r.standard_normal(n)).astype(f32)
    W = mc.random_q4_0(r, rows, n)
    deq = mc.q4_0_dequant_numpy(W, rows, n)
    inv = 1.0 / np.sqrt(np.sum(x.astype(np.float64) ** 2) / n + eps)
    exp = (deq @ (x.astype(np.float64) * w.astype(np.float64))) * inv
    got64, mag = ora.matvec_q4_0_rms_f64(x, W, w, n, rows, eps)
    np.testing.assert_allclose(got64, exp, rtol=1e-12, atol=1e-12 * float(mag.max()))
    ref32 = ora.matvec_q4_0_rms_ref(x, W, w, n, rows, eps)
    # sequential f32: |err| <= (n + 4) * 2^-24 * sum|terms| (sum|terms| <= mag / 2)
    assert np.all(np.abs(ref32 - got64) <= (n + 8) * 2.0 ** -24 * mag)
    # plain matvec (no RMS weight) and a one-hot input: output = deq column exactly
    k = 77
    e = np.zeros(n, f32)
    e[k] = 1.0
    col, _ = ora.matvec_q4_0_rms_f64(e, W, None, n, rows, eps)
    assert np.array_equal(col, deq[:, k])
    assert np.array_equal(ora.matvec_q4_0_rms_ref(e, W, None, n, rows, eps), deq[:, k].astype(f32))
    # one-hot with RMS: x = c e_k -> inv = 1/sqrt(c^2/n + eps), y_k = c w_k
    c = f32(3.0)
    got, _ = ora.matvec_q4_0_rms_f64(c * e, W, w, n, rows, eps)
    np.testing.assert_allclose(got, deq[:, k] * float(c) * float(w[k]) / np.sqrt(9.0 / n + eps), rtol=1e-12)


def test_ple_projection_f16_pinned(ora):
    """The decode PLE projection (matvec_f16 * scale, then the stable group
    norm; gemma4_executor.rs:4184-4214): against numpy's float64 matmul of the
    exactly widened F16 weights and the group norm in float64, within the
    sequential f32 dot's bound carried through the norm; a one-hot input
    selects one weight column exactly (the dot has no rounding); a zero group
    stays zero; and a reversed column order (a planted mistake) is caught."""
    r = np.random.default_rng(41)
    hidden, width, groups, eps, scale = 96, 32, 4, 1e-6, 0.125
    x = r.standard_normal(hidden).astype(f32)
    Wh = (0.1 * r.standard_normal((groups * width, hidden))).astype(np.float16)
    Wh[width:2 * width] = 0                                   # group 1 all zero
    W = Wh.view(np.uint16).reshape(-1)
    nw = (1.0 + 0.1 * r.standard_normal(width)).astype(f32)

    def exact(xv, Wm):
        p = (Wm.astype(np.float64) @ xv.astype(np.float64)) * scale
        mag = (np.abs(Wm.astype(np.float64)) @ np.abs(xv.astype(np.float64))) * scale
        out = np.zeros_like(p)
        for g in range(groups):
            v = p[g * width:(g + 1) * width]
            m = np.max(np.abs(v))
            if m > 0:
                out[g * width:(g + 1) * width] = v * ((1 / np.sqrt(np.sum((v / m) ** 2) / width + eps / m / m)) / m) * nw
        return p, mag, out

    got = ora.ple_projection_f16(x, W, nw, hidden, width, groups, scale, eps)
    p, mag, out = exact(x, Wh)
    assert np.all(got[width:2 * width] == 0.0)
    for g in (0, 2, 3):
        sl = slice(g * width, (g + 1) * width)
        # sequential f32 dot: |err| <= (hidden + 2) * 2^-24 * mag; through the
        # scale-free norm about twice that, normwise, plus the norm's roundings
        rel = np.linalg.norm(got[sl] - out[sl]) / np.linalg.norm(out[sl])
        assert rel <= 2 * (hidden + 2) * 2.0 ** -24 * np.linalg.norm(mag[sl]) / np.linalg.norm(p[sl]) + 1e-6
    # one-hot input: p = scale * W[:, k] exactly, so each group is W[:, k] normalised
    k = 17
    e = np.zeros(hidden, f32)
    e[k] = 1.0
    got1 = ora.ple_projection_f16(e, W, nw, hidden, width, groups, scale, eps)
    _, _, out1 = exact(e, Wh)
    np.testing.assert_allclose(got1, out1, rtol=2e-6, atol=1e-30)
    # planted mistake: the weights' columns reversed must not pass
    wrong = ora.ple_projection_f16(x, Wh[:, ::-1].copy().view(np.uint16).reshape(-1), nw, hidden, width, groups,
                                   scale, eps)
    assert np.linalg.norm(wrong[:width] - out[:width]) > 0.1 * np.linalg.norm(out[:width])


def test_reference_matvec_generators():
    """The restated reference-test generators reproduce the LCG and the weight
    pattern of matvec_rms_fused_parity.rs:16-49."""
    import matvec_cases as mc
    lcg = mc.Lcg(0x9E3779B9)
    assert lcg.next_u32() == (0x9E3779B9 * 1664525 + 1013904223) & 0xFFFFFFFF
    v = mc.reference_fill_f32(1000, mc.Lcg(1))
    assert v.dtype == np.float32 and v.min() >= -1.0 and v.max() < 1.0
    W = mc.reference_q4_weights(3, 2).reshape(6, 18)
    for i in range(6):
        bits = int(round((0.005 + (i % 101) * 0.0003) * 32768.0))
        assert W[i, 0] | (W[i, 1] << 8) == bits
        for j in range(16):
            nib = (i * 7 + j * 13) % 16
            assert W[i, 2 + j] == nib | (nib << 4)


# ------------------------------------------- KV append: Q8_0 / Q4_0 encoders

def _np_encode_q8_0(v):
    """Independent vectorised restatement of kv_append_decode_q8_0's block encoder
    (kernels.metal:1222-1231) in float32 numpy: [n, 32] -> [n, 34] bytes."""
    v = v.astype(f32)
    m = np.max(np.abs(v), axis=1)
    scale = np.where(m == 0, f32(0), m / f32(127)).astype(f32)
    safe = np.where(scale == 0, f32(1), scale)
    q = np.clip(v / safe[:, None], f32(-127), f32(127))
    code = np.where(scale[:, None] == 0, 0, np.sign(q) * np.floor(np.abs(q) + 0.5)).astype(np.int8)
    out = np.zeros((v.shape[0], 34), np.uint8)
    out[:, 0:2] = scale.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = code.view(np.uint8)
    return out


def _np_encode_q4_0(v):
    """kv_append_decode_q4_0's block encoder (kernels.metal:1247-1256): the first
    index of the largest |v| gives the signed maximum."""
    v = v.astype(f32)
    first = np.argmax(np.abs(v), axis=1)             # argmax returns the first occurrence
    smax = v[np.arange(v.shape[0]), first]
    m = np.abs(smax)
    scale = np.where(m == 0, f32(0), smax / f32(-8)).astype(f32)
    safe = np.where(scale == 0, f32(1), scale)
    t = (v / safe[:, None]).astype(f32) + f32(8.5)
    code = np.where(t >= 15, 15, np.where(t > 0, np.trunc(t), 0)).astype(np.int64)
    code[scale == 0] = 0
    out = np.zeros((v.shape[0], 18), np.uint8)
    out[:, 0:2] = scale.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = (code[:, :16] | (code[:, 16:] << 4)).astype(np.uint8)
    return out


def _adversarial_blocks(r):
    blocks = [r.standard_normal(32), np.zeros(32), (r.integers(-20, 20, 32) / 4.0),   # exact halves: rounding ties
              np.full(32, -3.0), np.where(np.arange(32) % 2 == 0, 2.5, -2.5),          # |max| tie, signs differ
              r.standard_normal(32) * 1e30, r.standard_normal(32) * 1e-30, np.arange(32) - 16.0]
    b = np.array(blocks, f32)
    b[3, 5] = 3.0                                          # equal |max| with the opposite sign later
    return b


def test_kv_encoders_pinned(ora):
    """The C encoders equal an independent numpy restatement on random and
    adversarial blocks, and satisfy the reference's own round-trip KAT
    (phase_11a_gguf.rs:33-55: values (i-16)/7, |v - deq| <= 0.35 Q4_0, 0.03 Q8_0)."""
    r = np.random.default_rng(41)
    v = np.concatenate([r.standard_normal((500, 32)).astype(f32) * f32(3), _adversarial_blocks(r)])
    got8 = np.array([ora.encode_q8_0_block(b) for b in v])
    got4 = np.array([ora.encode_q4_0_block(b) for b in v])
    assert np.array_equal(got8, _np_encode_q8_0(v))
    assert np.array_equal(got4, _np_encode_q4_0(v))
    kat = ((np.arange(32) - 16.0) / 7.0).astype(f32)
    dq4 = ora.dequant_q4_0_block(ora.encode_q4_0_block(kat))
    assert np.all(np.abs(dq4 - kat) <= 0.35)
    b8 = ora.encode_q8_0_block(kat)
    d8 = np.frombuffer(b8[:2].tobytes(), np.float16).astype(np.float64)[0]
    dq8 = b8[2:].view(np.int8).astype(np.float64) * d8
    assert np.all(np.abs(dq8 - kat) <= 0.03)


def test_kv_encoder_tie_rules_known_answers(ora):
    """The oracle's encoders give the hand-derived bytes of kv_tie_blocks, and
    the same check rejects encoders with the other tie rules (planted
    mistakes: round-half-even quotients, the last largest |v|)."""
    q8, want8, q4, want4 = mc.kv_tie_blocks()
    assert bytes(ora.encode_q8_0_block(q8)) == want8
    assert bytes(ora.encode_q4_0_block(q4)) == want4
    # planted: round half to even (numpy's rint) instead of half away from zero
    even = np.rint(q8 / f32(1.0)).astype(np.int8)
    assert bytes([0x00, 0x3C]) + even.view(np.uint8).tobytes() != want8
    # planted: the last index of the largest |v| gives the signed maximum
    last = 31 - int(np.argmax(np.abs(q4)[::-1]))
    scale = f32(q4[last] / f32(-8))
    codes = np.clip(np.trunc(q4 / scale + f32(8.5)), 0, 15).astype(np.uint8)
    planted = np.array([scale], np.float16).view(np.uint8).tobytes() + bytes(int(codes[i]) | (int(codes[i + 16]) << 4) for i in range(16))
    assert planted != want4


def test_kv_encoder_error_bounds(ora):
    """Round trip of random blocks within half a step plus the f16 scale rounding;
    the block maximum maps to code -127/127 (Q8_0) and to code 0 (Q4_0)."""
    r = np.random.default_rng(43)
    for _ in range(300):
        v = (r.standard_normal(32) * r.uniform(0.01, 100)).astype(f32)
        b8 = ora.encode_q8_0_block(v)
        s = float(np.max(np.abs(v))) / 127.0
        d = float(np.frombuffer(b8[:2].tobytes(), np.float16)[0])
        codes = b8[2:].view(np.int8).astype(np.float64)
        assert np.all(np.abs(codes * d - v) <= s / 2 + 127 * abs(d - s) + 1e-6 * s)
        assert abs(codes[np.argmax(np.abs(v))]) == 127
        b4 = ora.encode_q4_0_block(v)
        dq = ora.dequant_q4_0_block(b4).astype(np.float64)
        s4 = abs(float(v[np.argmax(np.abs(v))])) / 8.0
        d4 = abs(float(np.frombuffer(b4[:2].tobytes(), np.float16)[0]))
        # codes clamp at 15 (value +7 * scale): the positive side of a negative
        # signed maximum saturates, so bound only the unclamped values
        ok = np.abs(v.astype(np.float64)) <= 7 * s4
        assert np.all(np.abs(dq - v)[ok] <= s4 / 2 + 8 * abs(d4 - s4) + 1e-6 * s4)


def test_kv_append_layout_and_vnorm(ora):
    """Cache rows land at [K | V][position]; positions >= capacity are skipped;
    the V norm scales each row by 1/sqrt(mean v^2 + eps) (float64 check)."""
    r = np.random.default_rng(47)
    w, cap, T = 64, 6, 5
    key, value = r.standard_normal((T, w)).astype(f32), r.standard_normal((T, w)).astype(f32)
    pos = np.array([4, 0, 9, 2, 6], np.uint32)     # 9 and 6 are outside the cache
    cache = np.full(2 * cap * w * 4, 0xAB, np.uint8)
    out = ora.kv_append("f32", key, value, cache, w, cap, pos, True, 1e-6).view(f32).reshape(2, cap, w)
    for t, p in enumerate(pos):
        if p >= cap:
            continue
        assert np.array_equal(out[0, p], key[t])
        inv = 1.0 / np.sqrt(np.mean(value[t].astype(np.float64) ** 2) + 1e-6)
        np.testing.assert_allclose(out[1, p], value[t] * inv, rtol=2e-6)
    untouched = [1, 3, 5]
    raw = cache.view(f32).reshape(2, cap, w)
    assert np.array_equal(out[:, untouched].view(np.uint32), raw[:, untouched].view(np.uint32))


# ------------------------------------------------------------ logits tail

def test_tanh_precise_against_float64(ora):
    """The soft cap's tanh: dense sweep of binary32 inputs against float64
    (softcap with cap 1 is tanh itself: x/1 and 1*t are exact)."""
    bits = np.arange(0, 0x7F800000, 61, dtype=np.uint32)
    x = bits.view(f32)
    got = ora.softcap(x, 1.0)
    err = ulp_err(got, np.tanh(x.astype(np.float64)))
    assert float(err.max()) < 1.4, f"tanh worst {float(err.max()):.3f} ulp"
    # odd symmetry, signed zero, saturation, NaN, subnormals pass through
    assert np.array_equal(ora.softcap(-x[:200000], 1.0).view(np.uint32),
                          (-got[:200000]).view(np.uint32))
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 10.0, 1e30], f32)
    s = ora.softcap(special, 1.0)
    assert s[0] == 0 and not np.signbit(s[0]) and s[1] == 0 and np.signbit(s[1])
    assert s[2] == 1 and s[3] == -1 and np.isnan(s[4])
    assert s[5] == special[5] and s[6] == special[6] and s[7] == 1 and s[8] == 1


def test_softcap_kat_and_cpu_form(ora):
    k = KATS["softcap"]
    v = ora.softcap(np.array(k["logits"], f32), k["cap"])
    assert np.all(np.abs(v) <= k["cap"])
    assert np.all(np.diff(v) > 0)
    assert abs(float(v[2])) < np.finfo(f32).eps
    # the reference CPU form cap * (x / cap).tanh() in binary32 (numpy's tanh
    # standing in for Rust's libm): within the operator tolerance of 4 ulp
    r = np.random.default_rng(31)
    x = np.concatenate([r.normal(0, 10, 200000), r.normal(0, 100, 50000), r.uniform(-1e4, 1e4, 50000)]).astype(f32)
    cap = f32(30.0)
    got = ora.softcap(x, cap)
    cpu_form = (cap * np.tanh(x / cap)).astype(f32)
    assert float(ulp_err(got, cpu_form).max()) <= 4.0
    exact = 30.0 * np.tanh(x.astype(np.float64) / 30.0)
    assert float(ulp_err(got, exact).max()) <= 2.5


def _reference_argmax_kernel(values):
    """The reference kernel's structure, step by step (kernels.metal:2033-2066):
    256 lanes scan their stride with `>=` from (-inf, 0), then the tree."""
    vals = [float(v) for v in values]
    best = [(-np.inf, 0)] * 256
    for lane in range(256):
        bv, bi = -np.inf, 0
        for i in range(lane, len(vals), 256):
            if vals[i] >= bv:
                bv, bi = vals[i], i
        best[lane] = (bv, bi)
    stride = 128
    while stride:
        for lane in range(stride):
            ov, oi = best[lane + stride]
            cv, ci = best[lane]
            if ov > cv or (ov == cv and oi >= ci):
                best[lane] = (ov, oi)
        stride >>= 1
    return best[0][1]


def test_argmax_kat_and_kernel_structure(ora):
    k = KATS["argmax"]
    v = np.full(k["count"], k["fill"], f32)
    for i, val in k["set"]:
        v[i] = val
    assert ora.argmax(v) == k["expected"]
    r = np.random.default_rng(5)
    pool = np.array([-1.0, 0.0, -0.0, 1.0, 2.0, -np.inf, np.inf, np.nan], f32)
    for trial in range(300):
        n = int(r.integers(1, 700))
        vals = pool[r.integers(0, len(pool) - (0 if trial % 3 else 2), n)]
        assert ora.argmax(vals) == _reference_argmax_kernel(vals), vals
    for vals in (np.full(5, np.nan, f32), np.full(300, -np.inf, f32), np.array([-0.0, 0.0, -0.0], f32)):
        assert ora.argmax(vals) == _reference_argmax_kernel(vals)
    # NaN-free rows without signed-zero ties: also the CPU executor's argmax
    # (max_by over total_cmp keeps the last maximum, atlas-model/src/lib.rs:1469-1476)
    for _ in range(50):
        vals = r.integers(-20, 20, int(r.integers(1, 5000))).astype(f32)
        vals[vals == 0] = 1.0
        assert ora.argmax(vals) == len(vals) - 1 - int(np.argmax(vals[::-1]))


def test_softcap_argmax_rows_is_the_composition(ora):
    r = np.random.default_rng(9)
    rows, count = 5, 3001
    x = r.normal(0, 20, rows * count).astype(f32)
    capped, sel = ora.softcap_argmax_rows(x, rows, count, 30.0)
    assert np.array_equal(capped.view(np.uint32), ora.softcap(x, 30.0).view(np.uint32))
    for i in range(rows):
        assert sel[i] == ora.argmax(capped[i * count:(i + 1) * count])
    plain, sel0 = ora.softcap_argmax_rows(x, rows, count, 0.0)
    assert np.array_equal(plain.view(np.uint32), x.view(np.uint32))
    assert all(sel0[i] == ora.argmax(x[i * count:(i + 1) * count]) for i in range(rows))
