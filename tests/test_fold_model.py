"""CPU model of the exact wave-parallel fold (fold_chunk_exact in
atlas_amd/csrc/device_common.hpp) and its proof by exhaustion on sample rows.

The reference CPU operator folds a row's squares left to right in f32
(crates/atlas-ops/tests/phase_02_operators.rs:233).  The GPU register engine
folds the first 256 squares in order and then each chunk of 64 lanes x S
consecutive squares (S = 4: one float4 column chunk; at decode batches the
whole continuation as one run, S = 4(J - 1) = 20 for 1536 values) without the
dependent add chain:

  * a running sum s >= 0 lies in a binade [2^E, 2^(E+1)); there every
    partial sum is an integer k of ulps u = 2^(E-23), and s + a rounds to
    (k + rint(a/u)) u unless a/u is an exact tie m + 1/2 (round-half-even then
    looks at the parity of k) or the result leaves the binade;
  * per lane, the S addends are converted to ulp counts, a prefix scan over
    the lanes gives every lane its running count, and the lanes before the
    first *event* (a lane holding a tie or an addend of >= 2^21 ulps, or the
    lane whose prefix reaches the next binade) are applied as one integer add
    to the bit pattern of s;
  * the event lane is folded value by value in f32, and the scan is reused
    (same binade) or recomputed (new binade); sums below 2^-100 or above
    2^124, inf and NaN fold lane by lane.

This file restates those steps in numpy and checks, row by row, that they
reproduce the sequential f32 fold bit for bit on Gaussian rows, FP16-valued
rows and the adversarial rows of the GPU tests (ties, binade crossings,
zeros, subnormal and overflowing squares, inf, NaN, constant and geometric
rows).  Planted mistakes (ignoring ties, ignoring binade crossings) must fail.

The decode engines fold the first 256 squares by candidate segments
(head_fold_candidates); its model at the end of this file is checked the same
way, with windows narrow enough to force the in-order fallback, and with a
planted mistake (the nearest candidate taken instead of the exact one).
"""
import numpy as np
import pytest

import cases

f32 = np.float32
u32 = np.uint32


def sequential_fold(sq):
    return np.cumsum(sq, dtype=f32)[-1] if sq.size else f32(0)


def _bits(x):
    return int(np.array([x], f32).view(u32)[0])


def _from_bits(b):
    return np.array([b], u32).view(f32)[0]


def exact_fold_model(sq, S, head=256, ties=True, crossings=True):
    """fold_chunk_exact_from's steps (device_common.hpp) on one row's squares
    (f32 array): `head` values in order, then chunks of 64 lanes x S values
    (lane l holds values [lS, lS + S) of the chunk, zero-padded past the row).
    Arithmetic as on the device: q = v * 2^(23-E), m = rint(q), the lane's
    ulp count summed in f32, an event where that count is not below 2^21 or a
    value sits exactly halfway (|q - m| == 1/2)."""
    s = sequential_fold(sq[:head]) if head else f32(0)
    rest = sq[head:]
    width = 64 * S
    for c0 in range(0, rest.size, width):
        ch = np.zeros(width, f32)
        ch[:min(width, rest.size - c0)] = rest[c0:c0 + width]
        lanes = ch.reshape(64, S)
        l0 = 0
        while l0 < 64:
            sb = _bits(s)
            ex = sb >> 23                                  # biased exponent (inf / NaN: >= 255)
            if ex < 27 or ex > 251:
                for a in lanes[l0]:                        # one lane in f32, then look again
                    s = f32(s + a)
                l0 += 1
                continue
            inv_ulp = _from_bits((277 - ex) << 23)         # 2^(23-E)
            with np.errstate(invalid="ignore", over="ignore"):
                q = (lanes * inv_ulp).astype(f32)
                m = np.rint(q).astype(f32)
                dev = np.max(np.abs(q - m), axis=1)
                ul = np.zeros(64, f32)
                for i in range(S):
                    ul = (ul + m[:, i]).astype(f32)
            bad = ~(ul < f32(2097152.0))
            if ties:
                bad |= dev == f32(0.5)
            inc = np.where(bad, 0, ul).astype(np.int64)
            incl = np.cumsum(inc)
            base = int(incl[l0 - 1]) if l0 else 0
            while True:
                sb = _bits(s)
                room = (1 << 23) - (sb & 0x7FFFFF)         # ulps to the next power of two
                reach = (incl - base) >= room if crossings else np.zeros(64, bool)
                ev = reach | bad
                ev[:l0] = False
                if not ev.any():
                    s = _from_bits(sb + int(incl[63]) - base)
                    l0 = 64
                    break
                lc = int(np.argmax(ev))
                s = _from_bits(sb + int(incl[lc] - inc[lc]) - base)   # lanes [l0, lc): one integer add
                for a in lanes[lc]:                                     # the event lane in f32
                    s = f32(s + a)
                base = int(incl[lc])
                l0 = lc + 1
                if l0 >= 64 or (_bits(s) >> 23) != ex:
                    break                                               # rescan in the new binade
    return s


def _rows():
    r = np.random.default_rng(77)
    out = [("gaussian", r.standard_normal((300, 1536)).astype(f32)),
           ("gaussian_2048", r.standard_normal((120, 2048)).astype(f32)),
           ("f16_values", r.standard_normal((200, 2048)).astype(np.float16).astype(f32))]
    for hidden in (1536, 2048, 576):
        out.append((f"adversarial_{hidden}", cases.adversarial_rows(160, hidden, 5000 + hidden).reshape(160, hidden)))
    out.append(("adversarial_f16", cases.adversarial_f16_rows(140, 2048, 7200).view(np.float16)
                .astype(f32).reshape(140, 2048)))
    return out


@pytest.mark.parametrize("S", [4, 8, 20])
def test_model_reproduces_the_sequential_fold(S):
    checked = 0
    with np.errstate(over="ignore", invalid="ignore"):
        for name, x in _rows():
            for row in x:
                sq = (row * row).astype(f32)
                want, got = sequential_fold(sq), exact_fold_model(sq, S)
                same = _bits(want) == _bits(got) or (np.isnan(want) and np.isnan(got))
                assert same, (name, S, want, got)
                checked += 1
    assert checked > 1000


def test_planted_mistakes_fail():
    """Ignoring ties or binade crossings breaks the fold on rows built for it."""
    x = cases.adversarial_rows(160, 1536, 5000 + 1536).reshape(160, 1536)
    with np.errstate(over="ignore", invalid="ignore"):
        sq_rows = [(row * row).astype(f32) for row in x]
        for kw in ({"ties": False}, {"crossings": False}):
            wrong = sum(_bits(sequential_fold(sq)) != _bits(exact_fold_model(sq, 4, **kw))
                        for sq in sq_rows if np.isfinite(sequential_fold(sq)))
            assert wrong > 0, kw


# ---------------------------------------------------------------------------
# The head by candidate segments (head_fold_candidates in device_common.hpp):
# the first 256 squares as four segments of 64; segment 0 folds from 0,
# segment k from the 2 * window + 1 consecutive floats around an estimate of
# its start, and the exact start of segment k (the selected fold of segment
# k - 1) selects the candidate that started there, or folds the segment in
# order from it when none did (a miss).
# ---------------------------------------------------------------------------
def _fold_from(starts, vals):
    """In-order f32 fold of vals from every start at once."""
    s = np.asarray(starts, f32).copy()
    for a in vals:
        s = (s + a).astype(f32)
    return s


def candidate_head_model(sq256, window=10, exact=True):
    seg = sq256.reshape(4, 64)
    lanes = sq256.reshape(64, 4)
    part = ((lanes[:, 0] + lanes[:, 1]) + (lanes[:, 2] + lanes[:, 3])).astype(f32)
    pre = np.cumsum(part, dtype=f32)  # an estimate: any order would do
    s = _fold_from([0.0], seg[0])[0]
    misses = 0
    for k in range(1, 4):
        est = _bits(pre[16 * k - 1])
        starts = (np.arange(est - window, est + window + 1, dtype=np.int64) & 0xFFFFFFFF).astype(u32)
        res = _fold_from(starts.view(f32), seg[k])
        want = _bits(s)
        hit = np.nonzero(starts == want)[0]
        if exact:
            if hit.size:
                s = res[hit[0]]
            else:
                s = _fold_from([s], seg[k])[0]
                misses += 1
        else:  # planted mistake: the nearest candidate, exact or not
            s = res[int(np.argmin(np.abs(starts.astype(np.int64) - want)))]
    return s, misses


def _heads():
    for name, x in _rows():
        for row in x:
            if row.size >= 256:
                yield name, (row[:256] * row[:256]).astype(f32)


@pytest.mark.parametrize("window", [10, 5, 1])
def test_candidate_head_reproduces_the_sequential_fold(window):
    checked = misses = 0
    with np.errstate(over="ignore", invalid="ignore"):
        for name, sq in _heads():
            want = sequential_fold(sq)
            got, m = candidate_head_model(sq, window)
            assert _bits(want) == _bits(got) or (np.isnan(want) and np.isnan(got)), (name, window, want, got)
            checked += 1
            misses += m
    assert checked > 1000
    if window == 1:
        assert misses > 0  # the in-order fallback was exercised


def test_candidate_head_planted_mistake_fails():
    """Taking the nearest candidate instead of the exact start's gives wrong bits."""
    wrong = 0
    with np.errstate(over="ignore", invalid="ignore"):
        for name, sq in _heads():
            want = sequential_fold(sq)
            if not np.isfinite(want):
                continue
            got, _ = candidate_head_model(sq, 1, exact=False)
            wrong += _bits(want) != _bits(got)
    assert wrong > 0
