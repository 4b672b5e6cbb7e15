"""GPU tests of the KV-cache append (f32, Q8_0, Q4_0; decode and batched;
with and without the fused V RMSNorm) through the C ABI.  The whole cache is
compared byte for byte with the CPU restatement of the Metal kernels.  Widths
256, 512 and 1024 run the row engine (two wavefronts per token); the others
run the per-value engine."""
import sys

import numpy as np
import pytest

import matvec_cases as mc
from atlas_amd import OperatorError

pytestmark = pytest.mark.gpu
f32 = np.float32
EPS = 1e-6


def say(msg):
    print(f"[gpu-kv] {msg}", flush=True)
    sys.stdout.flush()


def run(rt, ora, fmt, key, value, w, cap, pos, vnorm, fill=0x5A):
    row = ora.kv_row_bytes(fmt, w)
    cache0 = np.full(2 * cap * row, fill, np.uint8)
    dk, dv, dp = rt.upload(key), rt.upload(value), rt.upload(np.asarray(pos, np.uint32))
    dc = rt.upload(cache0)
    rt.kv_append(fmt, dk, dv, dc, w, cap, dp, len(pos), vnorm, EPS)
    rt.sync()
    got = dc.download(cache0.size, np.uint8)
    exp = ora.kv_append(fmt, key, value, cache0, w, cap, pos, vnorm, EPS)
    return got, exp, dv.download(value.size, np.float32)


def assert_cache(name, got, exp, fmt=None):
    if fmt == "f32":
        # f32 caches: a NaN equals any NaN (payload bits are not part of the contract)
        g, e = got.view(np.float32), exp.view(np.float32)
        both_nan = np.isnan(g) & np.isnan(e)
        got = np.where(both_nan, np.float32(0), g).view(np.uint8)
        exp = np.where(both_nan, np.float32(0), e).view(np.uint8)
    if not np.array_equal(got, exp):
        j = int(np.nonzero(got != exp)[0][0])
        raise AssertionError(f"{name}: {int((got != exp).sum())} of {exp.size} cache bytes differ; first at {j}: "
                             f"gpu={got[j]} oracle={exp[j]}")


@pytest.mark.parametrize("fmt,seed", [("f32", 0x1F2A3B4C), ("q8_0", 0x5A6B7C8D), ("q4_0", 0x9E10A1B2)])
def test_kv_append_reference_test_inputs(rt, ora, fmt, seed):
    """kv_append_vnorm_fused_parity.rs:200-283: widths 64/128/256, positions 0 and 2,
    capacity 8, the test's LCG stream; fused V norm and plain append."""
    lcg = mc.Lcg(seed)
    for w in (64, 128, 256):
        for p in (0, 2):
            key, value = mc.reference_fill_f32(w, lcg), mc.reference_fill_f32(w, lcg)
            for vnorm in (True, False):
                say(f"kv {fmt} reference inputs w={w} position={p} vnorm={vnorm}")
                got, exp, v_after = run(rt, ora, fmt, key, value, w, 8, [p], vnorm)
                assert_cache(f"{fmt} w={w} p={p}", got, exp)
                assert np.array_equal(v_after.view(np.uint32), value.view(np.uint32)), "V input was modified"


def _values(r, tokens, w, kind):
    v = r.standard_normal((tokens, w)).astype(f32)
    if kind == "adversarial":
        v[0::5] = 0.0                                        # all-zero rows and blocks
        v[1::5] = (r.integers(-40, 40, (len(v[1::5]), w)) / 4.0).astype(f32)   # rounding ties
        v[2::5, ::7] = np.float32(1e30)
        v[3::5] = np.where(np.arange(w) % 2 == 0, f32(2.5), f32(-2.5))        # |max| ties, mixed signs
        v[4::5] *= f32(1e-20)                                # subnormal squares in the V norm
    elif kind == "nan":
        nan = f32(np.nan)
        v[0::4, :32] = nan                                   # an all-NaN block: scale 0, codes 0
        v[1::4, 5] = nan                                     # one NaN: with the V norm the whole row is NaN
        v[2::4] = nan                                        # an all-NaN row
        v[3::4, ::3] = nan                                   # NaN beside finite values in every block
    elif kind == "band":
        # quotients on, just inside and just outside the row engine's band of
        # 2^-12 around half-integers (where it recomputes with a division):
        # even rows open every block with -8 (Q4_0 scale 1), odd rows with 127
        # (Q8_0 scale 1), so value = quotient
        offs = np.array([0.0, 2.0 ** -13, -2.0 ** -13, 2.0 ** -11, -2.0 ** -11, 2.0 ** -20, -2.0 ** -20, 0.25])
        idx = np.arange(tokens * w).reshape(tokens, w)
        half = r.integers(-8, 8, (tokens, w)) + 0.5
        half[1::2] = r.integers(-126, 126, (len(half[1::2]), w)) + 0.5
        v = (half + offs[idx % 8]).astype(f32)
        v[0::2, ::32] = f32(-8.0)
        v[1::2, ::32] = f32(127.0)
    return v


@pytest.mark.parametrize("fmt", ["f32", "q8_0", "q4_0"])
@pytest.mark.parametrize("w,tokens,cap", [(256, 1, 64), (512, 1, 4096), (256, 4096, 4096), (256, 301, 512),
                                          (32, 9, 16), (4096, 3, 4), (96, 33, 40), (1024, 130, 128)])
@pytest.mark.parametrize("kind", ["normal", "adversarial", "nan", "band"])
def test_kv_append_shapes(rt, ora, fmt, w, tokens, cap, kind):
    """Decode (one token at a random position), prefill batches (eight f32 /
    four quantised tokens per workgroup with the V norm at width 256, a
    ragged last workgroup at 301 tokens), ragged widths,
    positions past the capacity (skipped), adversarial blocks, NaN blocks
    and rows (the encoders' maximum starts at 0, as the reference's does),
    and quotients at and beside half-integers (the exact recompute)."""
    r = np.random.default_rng(w * 7 + tokens + cap)
    key, value = _values(r, tokens, w, kind), _values(r, tokens, w, kind)
    pos = r.permutation(max(cap, tokens))[:tokens].astype(np.uint32) if tokens > 1 else \
        np.array([r.integers(0, cap)], np.uint32)
    if tokens > 2:
        pos[1] = cap + 3                                     # outside the cache: skipped
    for vnorm in (True, False):
        say(f"kv {fmt} w={w} tokens={tokens} capacity={cap} {kind} vnorm={vnorm}")
        got, exp, _ = run(rt, ora, fmt, key, value, w, cap, pos, vnorm)
        assert_cache(f"{fmt} w={w} tokens={tokens}", got, exp, fmt)


def test_kv_append_invalid_input(rt):
    say("kv invalid input")
    k, v, c, p = rt.empty(8192), rt.empty(8192), rt.empty(1 << 16), rt.upload(np.zeros(4, np.uint32))
    for bad in (lambda: rt.kv_append("q8_0", k, v, c, 48, 4, p, 1, False, EPS),   # not a multiple of 32
                lambda: rt.kv_append("q4_0", k, v, c, 0, 4, p, 1, False, EPS),
                lambda: rt.kv_append("f32", k, v, c, 4097, 4, p, 1, False, EPS),
                lambda: rt.kv_append("f32", k, v, c, 6, 4, p, 1, True, EPS),      # V norm needs % 4
                lambda: rt.kv_append("f32", k, v, c, 64, 0, p, 1, False, EPS),
                lambda: rt.kv_append("f32", k, v, c, 64, 4, p, 0, False, EPS),
                lambda: rt.kv_append("q4_0", k, v, c, 64, 4, p, 1, True, 0.0),
                lambda: rt.kv_append("q4_0", k, None, c, 64, 4, p, 1, False, EPS)):
        with pytest.raises(OperatorError) as e:
            bad()
        assert e.value.kind == "InvalidInput"


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0"])
def test_kv_append_tie_rules_known_answers(rt, ora, fmt):
    """The hand-derived blocks of matvec_cases.kv_tie_blocks (quotients on
    half-integers for Q8_0's half-away rounding, +-4 as the largest |v| for
    Q4_0's first-maximum rule) tiled over a K and a V row: every block of the
    device cache equals the hand-derived bytes, on the row engine (width 256)
    and the per-value engine (width 64)."""
    q8, want8, q4, want4 = mc.kv_tie_blocks()
    blk, want = (q8, want8) if fmt == "q8_0" else (q4, want4)
    for w in (256, 64):
        row = np.tile(blk, w // 32).astype(f32)
        say(f"kv {fmt} tie-rule blocks w={w}")
        got, exp, _ = run(rt, ora, fmt, row, row.copy(), w, 2, [1], False)
        assert_cache(f"{fmt} tie blocks w={w}", got, exp)
        rb = ora.kv_row_bytes(fmt, w)
        for side in (0, 1):  # K and V rows of position 1
            r = got[(side * 2 + 1) * rb:(side * 2 + 2) * rb]
            assert r.tobytes() == want * (w // 32), (fmt, w, side)
