"""CPU model of the KV row engine's encoder shortcuts (kv_kernels.hip,
encode_items and div127).  The reference encodes y (the K row, or the V row
times the V norm's inverse RMS) with codes taken from the correctly rounded
quotient q = fl(y / scale) (kernels.metal:1212-1264).  The row engine:

  * takes the block maximum of y = fl(v inv) as fl(max|v| inv);
  * divides the Q8_0 maximum by 127 with Markstein's correction;
  * takes the quotient as v * fl(inv rcp(scale)) (v * rcp(scale) for K rows)
    and keeps it only when it lies more than 2^-12 from every half-integer
    and the scale and that factor are normal floats.

These tests check the claims behind each step, with the reciprocal anywhere
within one ulp of 1/scale (v_rcp_f32's bound).  Blocks are random, scaled
over many binades, and built so that quotients fall on, beside and just
outside the band."""
import numpy as np

f32 = np.float32
BAND = f32(2.0 ** -12)


def rn(x):
    return np.asarray(x).astype(f32)


def div127_markstein(a):
    """The kernel's steps: q0 = a c, r = fma(-q0, 127, a), q = fma(r, c, q0),
    with each fma's exact value formed in float64 and rounded once.  The
    second fma's exact value can need more than 53 bits, so it is rounded to
    float64 first and checked not to sit on a float32 halfway point, where
    that double rounding could differ from a single one."""
    c = f32(1) / f32(127)
    q0 = rn(a * c)
    r64 = a.astype(np.float64) - 127.0 * q0.astype(np.float64)      # exact (31-bit product)
    r = rn(r64)
    assert np.array_equal(r.astype(np.float64), r64), "the residual must be exact"
    s = q0.astype(np.float64) + r.astype(np.float64) * np.float64(c)
    q = rn(s)
    assert not (np.abs(s - q) == np.spacing(np.abs(q)).astype(np.float64) / 2).any()
    return q


def test_div127_every_float_of_one_binade():
    """RN(a / 127) for all 2^23 floats in [1, 2); every step scales exactly
    by powers of two, so this covers the kernel's range [2^-100, 2^100]."""
    a = (np.arange(1 << 23, dtype=np.uint32) | np.uint32(127 << 23)).view(f32)
    ref = rn(a / f32(127))
    assert np.array_equal(div127_markstein(a), ref)
    # control: the uncorrected product is wrong for many of them
    assert int((rn(a * (f32(1) / f32(127))) != ref).sum()) > 100000


def test_norm_block_max_is_scaled_raw_max():
    """max |fl(v inv)| == fl(max|v| inv) for finite values and inv: rounding
    is monotonic, so the largest |v| gives the largest |y|."""
    r = np.random.default_rng(5)
    v = (r.standard_normal((1 << 15, 32)) * 2.0 ** r.integers(-120, 120, (1 << 15, 1))).astype(f32)
    v[::7, 3] = v[::7, 5] * f32(1 + 2 ** -23)            # near-ties that rounding can merge
    inv = rn(2.0 ** r.uniform(-60, 60, (1 << 15, 1)))
    with np.errstate(over="ignore", under="ignore"):
        y = rn(v * inv)
        fast = rn(np.max(np.abs(v), axis=1, keepdims=True) * inv)
    finite = np.isfinite(fast[:, 0])
    assert finite.mean() > 0.9
    assert np.array_equal(np.max(np.abs(y), axis=1)[finite], fast[finite, 0])


def scales(fmt, y):
    """Per-block scale of the values y, the encoders' own steps (float32)."""
    amax = np.max(np.abs(y), axis=1)
    if fmt == "q8_0":
        s = np.where(amax == 0, f32(0), rn(amax / f32(127)))
    else:
        first = np.argmax(np.abs(y) == amax[:, None], axis=1)
        smax = y[np.arange(len(y)), first]
        s = np.where(amax == 0, f32(0), rn(smax * f32(-0.125)))
    return rn(s)


def code_exact(fmt, y, s):
    with np.errstate(divide="ignore", invalid="ignore"):
        q = rn(y / s)
    q = np.where(s == 0, f32(0), q)   # the reference's select: no quotient at scale 0
    if fmt == "q8_0":
        c = np.clip(np.where(np.isnan(q), f32(-127), q), f32(-127), f32(127)).astype(np.float64)  # fmaxf drops NaN
        return np.where(s == 0, 0, (np.sign(c) * np.floor(np.abs(c) + 0.5)).astype(np.int64))
    t = rn(q + f32(8.5))
    code = np.where(t >= 15, 15, np.where(t > 0, np.trunc(np.where(t > 0, t, 0)), 0)).astype(np.int64)
    return np.where(s == 0, 0, code)


def code_fast(fmt, qa):
    if fmt == "q8_0":
        return np.rint(np.clip(qa, f32(-127), f32(127))).astype(np.int64)
    return np.trunc(np.clip(rn(qa + f32(8.5)), f32(0), f32(15))).astype(np.int64)


def normal(x):
    a = np.abs(x)
    return (a >= f32(2.0 ** -126)) & (a <= f32(2.0 ** 126))


def kept(qa, s, factor):
    frac = rn(qa - np.floor(qa))
    return normal(s) & normal(factor) & (np.abs(frac - f32(0.5)) > BAND)


def blocks_under_test(r, n):
    """n blocks of 32: random normal values over binades 2^-100..2^100, and
    blocks whose quotients sit on or near half-integers."""
    b = r.standard_normal((n, 32)).astype(f32)
    b *= (2.0 ** r.integers(-100, 100, (n, 1))).astype(f32)
    m = n // 2
    # quotient-targeted blocks: value = (k + 0.5 + off) * unit with max |v| = 127 * unit (Q8_0)
    # or 8 * unit (Q4_0), unit a random normal float
    unit = (r.uniform(0.5, 1.0, (m, 1)) * 2.0 ** r.integers(-90, 90, (m, 1))).astype(f32)
    offs = np.array([0.0, 2.0 ** -13, -2.0 ** -13, 2.0 ** -12, -2.0 ** -12, 2.0 ** -11, -2.0 ** -11, 2.0 ** -22])
    lim = np.where(r.random((m, 1)) < 0.5, 126, 7)
    k = np.floor(r.random((m, 32)) * (2 * lim)) - lim
    q = k + 0.5 + offs[r.integers(0, len(offs), (m, 32))]
    b[:m] = (q * unit).astype(f32)
    b[:m, 0] = np.where(lim[:, 0] == 126, 127.0, -8.0) * unit[:, 0]
    return b


def check(fmt, seed, norm, n=1 << 16):
    """Every kept product gives the reference's code, for the reciprocal at
    RN(1/scale) and one ulp either side.  With `norm` the values are scaled
    by a per-block inverse RMS first (by the kernel's factor for the
    quotient, by y = fl(v inv) for the reference)."""
    r = np.random.default_rng(seed)
    v = blocks_under_test(r, n)
    inv = rn(2.0 ** r.uniform(-30, 30, (n, 1))) if norm else np.ones((n, 1), f32)
    with np.errstate(over="ignore", under="ignore"):
        y = rn(v * inv)
    s = scales(fmt, y)
    exact = code_exact(fmt, y, s[:, None])
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        r0 = rn(f32(1) / s)
    kept_random = 0
    for r1 in (np.nextafter(r0, f32(-np.inf)), r0, np.nextafter(r0, f32(np.inf))):
        with np.errstate(over="ignore", under="ignore", invalid="ignore"):
            factor = rn(inv[:, 0] * r1) if norm else r1
            qa = rn(v * factor[:, None])
            keep = kept(qa, s[:, None], factor[:, None])
            fast = code_fast(fmt, np.where(keep, qa, f32(0)))
        bad = keep & (fast != exact)
        assert not bad.any(), (fmt, norm, v[bad][:4], s[np.nonzero(bad)[0][:4]])
        kept_random += int(keep[n // 2:].sum())
    return kept_random, (n - n // 2) * 32 * 3


def test_band_shortcut_q8_0():
    kept_n, total = check("q8_0", 11, norm=False)
    assert kept_n > 0.99 * total     # on random blocks the shortcut is the common case


def test_band_shortcut_q4_0():
    kept_n, total = check("q4_0", 12, norm=False)
    assert kept_n > 0.99 * total


def test_band_shortcut_with_v_norm():
    for fmt, seed in (("q8_0", 14), ("q4_0", 15)):
        kept_n, total = check(fmt, seed, norm=True)
        assert kept_n > 0.98 * total


def test_band_catches_planted_error():
    """Keeping every product (no band) must fail on the half-integer blocks:
    the check above is able to see a wrong code."""
    global BAND
    saved = BAND
    BAND = f32(-1.0)
    try:
        failed = False
        try:
            check("q8_0", 13, norm=False, n=1 << 12)
        except AssertionError:
            failed = True
        assert failed
    finally:
        BAND = saved
