"""The Q6_K gather computes the reference's ((q - 32) * sc) * d
(crates/atlas-core/src/gguf.rs:384-413) as (q - 32) * (sc * d), with sc * d
formed once per super-block pass (atlas_amd/csrc/gather_kernels.hip,
q6_k_decode4).  The two groupings are the same float32 value whenever both
inner products are exact, which holds for every operand the format can
hold: this test checks it exhaustively in IEEE float32 -- every q - 32 in
[-32, 31], every int8 sub-scale and every f16 bit pattern of d (zeros of
both signs, subnormals, infinities and NaNs) -- bit for bit, NaNs equal to
NaNs.  A grouping whose inner product rounds (here: a scale of 1/3 in
place of d) must fail the same comparison."""
import numpy as np

f32 = np.float32


def _regroup_mismatches(dvals):
    sc = np.arange(-128, 128, dtype=np.int64).astype(f32)
    sd = np.multiply.outer(sc, dvals)                          # sc * d, once per pass
    bad = 0
    for q in range(-32, 32):
        qf = f32(q)
        ref = np.multiply.outer(qf * sc, dvals)                 # (q * sc) * d
        got = qf * sd                                           # q * (sc * d)
        both_nan = np.isnan(ref) & np.isnan(got)
        bad += int(np.count_nonzero((ref.view(np.uint32) != got.view(np.uint32)) & ~both_nan))
    return bad


def test_q6k_regrouping_is_exact_for_every_f16_scale():
    with np.errstate(all="ignore"):
        d = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(f32)
        assert _regroup_mismatches(d) == 0


def test_q6k_regrouping_check_sees_a_rounding_inner_product():
    # planted: d = 1/3 * 2^k has a 24-bit significand, so sc * d rounds and
    # the two groupings differ for some (q, sc)
    with np.errstate(all="ignore"):
        d = (f32(1.0) / f32(3.0)) * np.exp2(np.arange(-4, 4, dtype=f32))
        assert _regroup_mismatches(d.astype(f32)) > 0
