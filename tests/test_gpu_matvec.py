"""GPU tests of the RMS-folded Q4_0 decode projections (matvec, fused QKV,
fused gate/up) through the C ABI.

Parity is floating-point, so two tolerances are asserted:
  * the reference's own contract (crates/atlas-metal/tests/
    matvec_rms_fused_parity.rs): max |gpu - oracle| < 1e-3 against the f32
    normalise-then-matvec oracle, on the reference test's own seeded inputs;
  * a normwise bound against the float64 oracle: |gpu - exact| <= 1e-5 *
    magnitude, where magnitude = inv_rms * sum_k 16 |x_k w_k d_k| bounds every
    partial sum an f32 evaluation forms (TOL below).
"""
import sys

import numpy as np
import pytest

import matvec_cases as mc
from atlas_amd import OperatorError

pytestmark = pytest.mark.gpu
f32 = np.float32
EPS = 1e-6
TOL = 1e-5       # normwise, against the float64 oracle
REF_TOL = 1e-3   # the reference's max-abs contract against its f32 oracle


def say(msg):
    print(f"[gpu-matvec] {msg}", flush=True)
    sys.stdout.flush()


def check(name, got, ora, x, W, w, n, rows, ref_contract=False):
    exact, mag = ora.matvec_q4_0_rms_f64(x, W, w, n, rows, EPS)
    err = np.abs(got.astype(np.float64) - exact)
    worst = float(np.max(err / np.maximum(mag, 1e-300)))
    assert np.all(err <= TOL * mag), f"{name}: normwise error {worst:.3e} > {TOL}"
    if ref_contract:
        ref = ora.matvec_q4_0_rms_ref(x, W, w, n, rows, EPS)
        max_abs = float(np.max(np.abs(got - ref)))
        assert max_abs < REF_TOL, f"{name}: max_abs {max_abs:.3e} against the reference oracle"
    return worst


def run_qkv(rt, x, qw, kw, vw, w, n, qn, kvn):
    dx, dw = rt.upload(x), (rt.upload(w) if w is not None else None)
    dq, dk, dv = rt.upload(qw), rt.upload(kw), rt.upload(vw)
    oq, ok, ov = rt.empty(qn), rt.empty(kvn), rt.empty(kvn)
    rt.matmul_q4_0_qkv_rms(dx, dq, dk, dv, oq, ok, ov, n, qn, kvn, dw, EPS)
    rt.sync()
    return oq.download(qn), ok.download(kvn), ov.download(kvn)


def run_gate_up(rt, x, gw, uw, w, n, m):
    dx, dw = rt.upload(x), (rt.upload(w) if w is not None else None)
    dg, du = rt.upload(gw), rt.upload(uw)
    og, ou = rt.empty(m), rt.empty(m)
    rt.matmul_q4_0_gate_up_rms(dx, dg, du, og, ou, n, m, dw, EPS)
    rt.sync()
    return og.download(m), ou.download(m)


def run_matvec(rt, x, W, w, n, m, weight_offset=0):
    dx, dw = rt.upload(x), (rt.upload(w) if w is not None else None)
    raw = np.zeros(W.size + weight_offset, np.uint8)
    raw[weight_offset:] = W
    dW = rt.upload(raw)
    out = rt.empty(m)
    rt.matvec_q4_0_rms(dx, dW.ptr + weight_offset, out, n, m, dw, EPS)
    rt.sync()
    return out.download(m)


def test_qkv_reference_test_inputs(rt, ora):
    """qkv_32row_mv_rms_matches_cpu_oracle (matvec_rms_fused_parity.rs:106-198):
    same LCG stream, widths and weight builder."""
    lcg = mc.Lcg(0x9E3779B9)
    for n in (128, 256, 2048):
        x = mc.reference_fill_f32(n, lcg)
        w = mc.reference_fill_rms_weight(n, lcg)
        for qn, kvn in ((96, 96), (128, 128), (512, 128), (513, 129)):
            say(f"qkv reference inputs n={n} q={qn} kv={kvn}")
            qw, kw, vw = (mc.reference_q4_weights(r, n // 32) for r in (qn, kvn, kvn))
            q, k, v = run_qkv(rt, x, qw, kw, vw, w, n, qn, kvn)
            check("q", q, ora, x, qw, w, n, qn, True)
            check("k", k, ora, x, kw, w, n, kvn, True)
            check("v", v, ora, x, vw, w, n, kvn, True)


def test_gate_up_reference_test_inputs(rt, ora):
    """gate_up_32row_mv_rms_matches_cpu_oracle (matvec_rms_fused_parity.rs:200-267)."""
    lcg = mc.Lcg(0x9E3779B9)
    for n in (128, 256, 2048):
        x = mc.reference_fill_f32(n, lcg)
        w = mc.reference_fill_rms_weight(n, lcg)
        for m in (96, 512, 513, 129):
            say(f"gate_up reference inputs n={n} out={m}")
            gw, uw = mc.reference_q4_weights(m, n // 32), mc.reference_q4_weights(m, n // 32)
            g, u = run_gate_up(rt, x, gw, uw, w, n, m)
            check("gate", g, ora, x, gw, w, n, m, True)
            check("up", u, ora, x, uw, w, n, m, True)


@pytest.mark.parametrize("n,qn,kvn", [(1536, 2048, 256), (1536, 4096, 512), (2048, 2048, 512), (576, 576, 192),
                                      (32, 17, 1), (4096, 64, 16), (1024, 1000, 33)])
def test_qkv_shapes(rt, ora, n, qn, kvn):
    """Gemma-4-E2B (1536 -> 8x256 / 1x256; full layers 1536 -> 8x512 / 1x512),
    SmolLM2 (2048, 576) and edge widths (one block, 4096, ragged tiles)."""
    r = np.random.default_rng(100 + n + qn)
    x = r.standard_normal(n).astype(f32)
    w = (1.0 + 0.1 * r.standard_normal(n)).astype(f32)
    qw, kw, vw = mc.random_q4_0(r, qn, n), mc.random_q4_0(r, kvn, n), mc.random_q4_0(r, kvn, n)
    say(f"qkv shapes n={n} q={qn} kv={kvn}")
    q, k, v = run_qkv(rt, x, qw, kw, vw, w, n, qn, kvn)
    worst = max(check("q", q, ora, x, qw, w, n, qn), check("k", k, ora, x, kw, w, n, kvn),
                check("v", v, ora, x, vw, w, n, kvn))
    say(f"  worst normwise error {worst:.2e}")


@pytest.mark.parametrize("n,m", [(1536, 6144), (2048, 8192), (576, 1536), (4096, 100), (64, 3)])
def test_gate_up_shapes(rt, ora, n, m):
    r = np.random.default_rng(200 + n + m)
    x = r.standard_normal(n).astype(f32)
    w = (1.0 + 0.1 * r.standard_normal(n)).astype(f32)
    gw, uw = mc.random_q4_0(r, m, n), mc.random_q4_0(r, m, n)
    say(f"gate_up shapes n={n} out={m}")
    g, u = run_gate_up(rt, x, gw, uw, w, n, m)
    check("gate", g, ora, x, gw, w, n, m)
    check("up", u, ora, x, uw, w, n, m)


@pytest.mark.parametrize("rms", [True, False])
@pytest.mark.parametrize("offset", [0, 2, 18])
def test_matvec_single_and_unaligned_weights(rt, ora, rms, offset):
    """matvec_q4_0_16row_mv_rms and the plain matvec (no RMS weight); weights at
    2-byte (not 16-byte) aligned addresses take the narrow staging path."""
    r = np.random.default_rng(300 + offset)
    n, m = 1536, 777
    x = (3.0 * r.standard_normal(n)).astype(f32)
    w = (1.0 + 0.1 * r.standard_normal(n)).astype(f32) if rms else None
    W = mc.random_q4_0(r, m, n)
    say(f"matvec rms={rms} weight offset={offset}")
    got = run_matvec(rt, x, W, w, n, m, offset)
    check("matvec", got, ora, x, W, w, n, m)


def test_matvec_deterministic(rt, ora):
    r = np.random.default_rng(9)
    n, m = 1536, 2048
    x, w, W = r.standard_normal(n).astype(f32), r.standard_normal(n).astype(f32), mc.random_q4_0(r, m, n)
    say("matvec run-to-run determinism")
    a = run_matvec(rt, x, W, w, n, m)
    b = run_matvec(rt, x, W, w, n, m)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_matvec_invalid_input(rt):
    """InvalidInput before any device work (widths, alignment, epsilon, null buffers)."""
    say("matvec invalid input")
    x, out = rt.empty(4096 + 64), rt.empty(64)
    W = rt.empty(64 * 8)
    w = rt.empty(4096)
    for bad in (lambda: rt.matvec_q4_0_rms(x, W, out, 100, 4, w, EPS),           # not a multiple of 32
                lambda: rt.matvec_q4_0_rms(x, W, out, 4096 + 32, 4, w, EPS),     # wider than 4096
                lambda: rt.matvec_q4_0_rms(x, W, out, 0, 4, w, EPS),
                lambda: rt.matvec_q4_0_rms(x, W, out, 64, 0, w, EPS),
                lambda: rt.matvec_q4_0_rms(x.ptr + 4, W, out, 64, 4, w, EPS),    # misaligned input
                lambda: rt.matvec_q4_0_rms(x, W.ptr + 1, out, 64, 4, w, EPS),    # odd weight address
                lambda: rt.matvec_q4_0_rms(x, W, out, 64, 4, w, 0.0),            # epsilon
                lambda: rt.matvec_q4_0_rms(x, None, out, 64, 4, w, EPS)):
        with pytest.raises(OperatorError) as e:
            bad()
        assert e.value.kind == "InvalidInput"


def _gelu64(x):
    a = 0.7978845608 * (x + 0.044715 * x ** 3)
    return 0.5 * x * (1.0 + np.tanh(a))


@pytest.mark.parametrize("n,m,layers", [(1536, 256, 35), (2048, 64, 3), (32, 5, 2), (4096, 300, 1)])
def test_ple_gate_gelu(rt, ora, n, m, layers):
    """gemma4_ple_gate_gelu_f32 (kernels.metal:803-881): gelu(W . state) * ple[offset + o]
    for each layer's slice.  The projection error (<= TOL * magnitude, as above) passes
    through GELU (|gelu'| < 1.13) and the f32 GELU adds a few ulp of |x|."""
    r = np.random.default_rng(500 + n + m)
    x = (0.3 * r.standard_normal(n)).astype(f32)
    W = mc.random_q4_0(r, m, n)
    ple = r.standard_normal(layers * m).astype(f32)
    dx, dW, dp, out = rt.upload(x), rt.upload(W), rt.upload(ple), rt.empty(m)
    g64, mag = ora.matvec_q4_0_rms_f64(x, W, None, n, m, EPS)
    for layer in range(layers):
        say(f"ple gate n={n} out={m} layer={layer}")
        rt.ple_gate_gelu(dx, dW, dp, layer * m, out, n, m)
        rt.sync()
        got = out.download(m).astype(np.float64)
        p = ple[layer * m:(layer + 1) * m].astype(np.float64)
        exact = _gelu64(g64) * p
        bound = (1.2 * TOL * mag + 8 * 2.0 ** -24 * (np.abs(g64) + 1.0)) * np.abs(p) + 2.0 ** -23 * np.abs(exact)
        assert np.all(np.abs(got - exact) <= bound), float(np.max(np.abs(got - exact) / bound))


def test_ple_gate_invalid_input(rt):
    say("ple gate invalid input")
    x, W, p, out = rt.empty(1536), rt.empty(4096), rt.empty(256), rt.empty(256)
    for bad in (lambda: rt.ple_gate_gelu(x, W, None, 0, out, 1536, 256),
                lambda: rt.ple_gate_gelu(x, W, p, 0, out, 1000, 256),
                lambda: rt.ple_gate_gelu(x, W, p, 0, out, 1536, 0)):
        with pytest.raises(OperatorError) as e:
            bad()
        assert e.value.kind == "InvalidInput"


# ---- the PLE projection with its stable group norm (matvec_f16 + scale +
# rms_norm_groups_in_place_stable_f32, kernels.metal:731-740, 897-917;
# gemma4_executor.rs:4184-4214) ----------------------------------------------

def _ple_projection64(x, W16, nw, hidden, width, groups, scale, eps):
    """float64 of the same steps: exact dots (numpy matmul), the scale, the
    stable norm; also mag = |scale| * sum_k |x_k W[o, k]|, the scale of any
    f32 evaluation's rounding error in the dot."""
    Wf = W16.view(np.float16).astype(np.float64).reshape(groups * width, hidden)
    xd = x.astype(np.float64)
    p = (Wf @ xd) * float(scale)
    mag = (np.abs(Wf) @ np.abs(xd)) * abs(float(scale))
    out = np.zeros_like(p)
    for g in range(groups):
        v = p[g * width:(g + 1) * width]
        m = np.max(np.abs(v))
        if m == 0:
            continue
        inv = (1.0 / np.sqrt(np.sum((v / m) ** 2) / width + eps / (m * m))) / m
        out[g * width:(g + 1) * width] = v * inv * nw.astype(np.float64)
    return p, mag, out


def _check_ple_projection(name, got, p64, mag, out64, width, groups):
    """Per group: the f32 dots are within TOL * mag of the exact ones, so the
    normalised group (out = p w / rms(p), scale-free) moves by at most about
    twice their normwise relative error; plus a few ulp for the norm's own
    roundings.  An all-zero group is exactly zero."""
    for g in range(groups):
        sl = slice(g * width, (g + 1) * width)
        pn = np.linalg.norm(p64[sl])
        if pn == 0:
            assert np.array_equal(got[sl], np.zeros(width, f32)), f"{name} group {g}: zero group not zero"
            continue
        kappa = np.linalg.norm(mag[sl]) / pn
        err = np.linalg.norm(got[sl].astype(np.float64) - out64[sl]) / np.linalg.norm(out64[sl])
        assert err <= 2 * TOL * kappa + 1e-6, f"{name} group {g}: normwise {err:.3e} (kappa {kappa:.1f})"


def _ple_case(r, hidden, width, groups, zero_group=None):
    x = (0.5 * r.standard_normal(hidden)).astype(f32)
    W = (0.05 * r.standard_normal((groups * width, hidden))).astype(np.float16)
    if zero_group is not None:
        W[zero_group * width:(zero_group + 1) * width] = 0
    nw = (1.0 + 0.1 * r.standard_normal(width)).astype(f32)
    return x, W.view(np.uint16).reshape(-1), nw


@pytest.mark.parametrize("hidden,width,groups", [(1536, 256, 35), (64, 16, 1), (1000, 32, 5), (4096, 1024, 3),
                                                 (8, 16, 2), (2560, 128, 9)])
def test_ple_projection_f16(rt, ora, hidden, width, groups):
    """Gemma-4-E2B's decode shape (hidden 1536, 35 groups of 256), a width of
    16 and of 1024, ragged hidden widths (1000: the last 512-column chunk is
    partial; 8), against float64 and against the f32 restatement; one group
    all zero; two calls in a row with different inputs."""
    r = np.random.default_rng(900 + hidden + width + groups)
    scale = float(hidden) ** -0.5
    for call in range(2):
        x, W, nw = _ple_case(r, hidden, width, groups, zero_group=(groups - 1 if groups > 1 else None))
        say(f"ple projection hidden={hidden} width={width} groups={groups} call {call}")
        dx, dW, dn, out = rt.upload(x), rt.upload(W), rt.upload(nw), rt.empty(groups * width)
        rt.ple_projection_f16(dx, dW, dn, out, hidden, width, groups, scale, EPS)
        rt.sync()
        got = out.download(groups * width)
        p64, mag, out64 = _ple_projection64(x, W, nw, hidden, width, groups, scale, EPS)
        _check_ple_projection(f"call {call}", got, p64, mag, out64, width, groups)
        ref = ora.ple_projection_f16(x, W, nw, hidden, width, groups, scale, EPS)
        _check_ple_projection(f"call {call} (oracle)", ref, p64, mag, out64, width, groups)


def test_ple_projection_graph_replays(rt):
    """Captured once (both of its launches), replayed three times with a new
    input written eagerly before each replay."""
    hidden, width, groups = 1536, 256, 35
    r = np.random.default_rng(77)
    x, W, nw = _ple_case(r, hidden, width, groups)
    dx, dW, dn, out = rt.upload(x), rt.upload(W), rt.upload(nw), rt.empty(groups * width)
    scale = hidden ** -0.5
    rt.graph_begin()
    try:
        rt.ple_projection_f16(dx, dW, dn, out, hidden, width, groups, scale, EPS)
    finally:
        g = rt.graph_end()
    try:
        for i in range(3):
            xi = (0.5 * r.standard_normal(hidden)).astype(f32)
            dx.upload(xi)
            say(f"ple projection graph replay {i}")
            rt.graph_launch(g)
            rt.sync()
            p64, mag, out64 = _ple_projection64(xi, W, nw, hidden, width, groups, scale, EPS)
            _check_ple_projection(f"replay {i}", out.download(groups * width), p64, mag, out64, width, groups)
    finally:
        rt.graph_destroy(g)


def test_ple_projection_invalid_input(rt):
    say("ple projection invalid input")
    x, W, n, out = rt.empty(1536), rt.empty(1 << 20), rt.empty(256), rt.empty(8960)
    for bad in (lambda: rt.ple_projection_f16(x, W, n, out, 1000 + 4, 256, 35, 1.0, EPS),   # hidden % 8
                lambda: rt.ple_projection_f16(x, W, n, out, 8192, 256, 1, 1.0, EPS),        # hidden > 4096
                lambda: rt.ple_projection_f16(x, W, n, out, 1536, 250, 35, 1.0, EPS),       # width % 16
                lambda: rt.ple_projection_f16(x, W, n, out, 1536, 2048, 1, 1.0, EPS),       # width > 1024
                lambda: rt.ple_projection_f16(x, W, n, out, 1536, 256, 0, 1.0, EPS),
                lambda: rt.ple_projection_f16(x, W, n, out, 1536, 256, 2000, 1.0, EPS),     # groups > 1024
                lambda: rt.ple_projection_f16(x, W, n, out, 1536, 256, 35, float("nan"), EPS),
                lambda: rt.ple_projection_f16(x, W, n, out, 1536, 256, 35, 1.0, 0.0),
                lambda: rt.ple_projection_f16(x, None, n, out, 1536, 256, 35, 1.0, EPS)):
        with pytest.raises(OperatorError) as e:
            bad()
        assert e.value.kind == "InvalidInput"
