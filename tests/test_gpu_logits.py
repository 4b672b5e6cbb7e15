"""GPU tests of the decode tail: the logit soft cap and the greedy argmax
(softcap_f32 / argmax_f32, crates/atlas-metal/src/kernels.metal:931-934,
2033-2066; caller gemma4_executor.rs:4678-4688), through the C ABI.

Bar: bit-exact against the CPU oracle.  The soft cap's tanh is this build's
(the reference's Metal/libm bits are not reproducible here); the oracle pins
it against float64 and the reference CPU form, so the GPU is held to the
oracle's bits.  The argmax is an index: exact, with the reference's tie rule
(the largest index of the maximum), NaN never selected, +0 == -0.
"""
import sys

import numpy as np
import pytest

from atlas_amd import OperatorError

pytestmark = pytest.mark.gpu
f32 = np.float32
CAP = 30.0  # Gemma 4's final_logit_softcapping


def say(msg):
    print(f"[gpu-logits] {msg}", flush=True)
    sys.stdout.flush()


def same_bits(a, b):
    return np.array_equal(np.asarray(a, f32).view(np.uint32), np.asarray(b, f32).view(np.uint32))


def logits(r, rows, count, scale=20.0):
    return (r.standard_normal(rows * count) * scale).astype(f32)


def run_fused(rt, x, rows, count, cap, capped=True):
    dx = rt.upload(x)
    sel = rt.empty(rows, np.uint32)
    rt.softcap_argmax(dx, dx if capped else None, sel, rows, count, cap)
    rt.sync()
    return dx.download(rows * count), sel.download(rows, np.uint32)


def test_argmax_reference_kat(rt):
    say("argmax KAT 65537 (crates/atlas-metal/src/lib.rs:2217-2230)")
    v = np.full(65537, -10.0, f32)
    v[7], v[31111], v[65536] = 3.5, 9.0, 9.0
    sel = rt.empty(1, np.uint32)
    rt.argmax(rt.upload(v), sel, 1, v.size)
    rt.sync()
    assert int(sel.download(1, np.uint32)[0]) == 65536


@pytest.mark.parametrize("rows,count", [(1, 1), (1, 3), (1, 4), (2, 5), (1, 1023), (3, 1024), (2, 1025), (1, 4097),
                                        (1, 262144), (7, 65537), (256, 262144)])
def test_softcap_argmax_matches_oracle(rt, ora, rows, count):
    say(f"softcap_argmax rows={rows} count={count}")
    r = np.random.default_rng(rows * 1000003 + count)
    x = logits(r, rows, count)
    # plant ties on the maximum in a few rows: the larger index must win
    for i in range(min(rows, 3)):
        if count > 2:
            row = x[i * count:(i + 1) * count]
            j, k = sorted(r.choice(count, 2, replace=False))
            row[j] = row[k] = np.float32(1e4)
    exp_capped, exp_sel = ora.softcap_argmax_rows(x, rows, count, CAP)
    got_capped, got_sel = run_fused(rt, x, rows, count, CAP)
    assert same_bits(got_capped, exp_capped)
    assert np.array_equal(got_sel, exp_sel)
    # argmax alone over the uncapped logits
    sel = rt.empty(rows, np.uint32)
    rt.argmax(rt.upload(x), sel, rows, count)
    rt.sync()
    _, exp_plain = ora.softcap_argmax_rows(x, rows, count, 0.0)
    assert np.array_equal(sel.download(rows, np.uint32), exp_plain)


def test_softcap_values_and_special_inputs(rt, ora):
    say("softcap special inputs")
    r = np.random.default_rng(77)
    x = np.concatenate([
        logits(r, 1, 100000, 5.0), logits(r, 1, 100000, 100.0), r.uniform(-1e30, 1e30, 1000).astype(f32),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 18.75, -18.75, 18.7499, 30.0, 1e38], f32),
    ]).astype(f32)
    for offset in (0, 1):  # 16-byte aligned vector path, then the scalar path
        n = x.size - offset
        src = rt.upload(x)
        dst = rt.empty(x.size)
        rt.softcap(src.ptr + 4 * offset, dst.ptr + 4 * offset, n, CAP)
        rt.sync()
        got = dst.download(x.size)[offset:]
        exp = ora.softcap(x[offset:], CAP)
        assert same_bits(got, exp), f"offset {offset}"


def test_argmax_ties_nan_signed_zero_rows(rt, ora):
    say("argmax NaN / -inf / signed zero rows")
    count = 5000
    rows = [
        np.full(count, np.nan, f32),                                        # all NaN -> 0
        np.full(count, -np.inf, f32),                                       # all -inf -> last
        np.where(np.arange(count) % 3 == 0, np.nan, -np.inf).astype(f32),  # NaN never wins
        np.zeros(count, f32),
        np.full(count, 2.0, f32),
    ]
    rows[3][::7] = -0.0  # +0 and -0 tie: the last index wins
    rows[4][[10, 4000, 4999]] = 3.0
    rows[4][4998] = np.nan
    x = np.concatenate(rows)
    n = len(rows)
    sel = rt.empty(n, np.uint32)
    rt.argmax(rt.upload(x), sel, n, count)
    rt.sync()
    got = sel.download(n, np.uint32)
    exp = [ora.argmax(row) for row in rows]
    assert list(got) == exp
    assert exp[0] == 0 and exp[1] == count - 1 and exp[4] == 4999


def test_softcap_argmax_without_store_and_repeated_calls(rt, ora):
    say("softcap_argmax capped=NULL, back-to-back calls on the workspace")
    r = np.random.default_rng(123)
    rows, count = 3, 262144
    dx = rt.empty(rows * count)
    sel = rt.empty(rows, np.uint32)
    for trial in range(4):
        x = logits(r, rows, count, 10.0 + 20 * trial)
        dx.upload(x)
        rt.softcap_argmax(dx, None, sel, rows, count, CAP)
        rt.sync()
        _, exp = ora.softcap_argmax_rows(x, rows, count, CAP)
        assert np.array_equal(sel.download(rows, np.uint32), exp), f"trial {trial}"
        assert same_bits(dx.download(rows * count), x)  # input untouched without a store


def test_more_rows_than_one_launch(rt, ora):
    say("softcap_argmax rows beyond one launch's workspace slots (two launches, scalar path)")
    r = np.random.default_rng(4100)
    rows, count = 300, 262143  # odd width: 256 workgroups per row, 256 rows per launch
    x = logits(r, rows, count)
    exp_capped, exp_sel = ora.softcap_argmax_rows(x, rows, count, CAP)
    got_capped, got_sel = run_fused(rt, x, rows, count, CAP)
    assert np.array_equal(got_sel, exp_sel)
    assert same_bits(got_capped, exp_capped)


def test_softcap_argmax_graph_replays(rt, ora):
    say("softcap_argmax captured in a HIP graph, replayed with new logits")
    r = np.random.default_rng(5)
    rows, count = 4, 262144
    dx = rt.empty(rows * count)
    sel = rt.empty(rows, np.uint32)
    rt.graph_begin()
    rt.softcap_argmax(dx, dx, sel, rows, count, CAP)
    graph = rt.graph_end()
    try:
        for trial in range(3):
            x = logits(r, rows, count, 5.0 + trial)
            dx.upload(x)
            rt.graph_launch(graph)
            rt.sync()
            exp_capped, exp_sel = ora.softcap_argmax_rows(x, rows, count, CAP)
            assert np.array_equal(sel.download(rows, np.uint32), exp_sel), f"replay {trial}"
            assert same_bits(dx.download(rows * count), exp_capped), f"replay {trial}"
    finally:
        rt.graph_destroy(graph)


def test_logits_invalid_input(rt):
    say("invalid inputs")
    x = rt.empty(16)
    sel = rt.empty(2, np.uint32)
    for cap in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(OperatorError):
            rt.softcap(x, x, 16, cap)
        with pytest.raises(OperatorError):
            rt.softcap_argmax(x, x, sel, 1, 16, cap)
    with pytest.raises(OperatorError):
        rt.argmax(x, sel, 1, 0)
    with pytest.raises(OperatorError):
        rt.argmax(x, sel, 0, 16)
    with pytest.raises(OperatorError):
        rt.argmax(x, None, 1, 16)
    with pytest.raises(OperatorError):
        rt.softcap(x, x, 0, CAP)
