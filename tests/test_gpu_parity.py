"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Default mode (sequential reduction) must be bit-identical to the oracle for
every op -- gathers and dequant by construction, norms / RoPE / activations
because the kernels keep the reference's f32 operation order and share the
oracle's exp algorithm.  Bit-identity is asserted on the raw bytes; the
seeded golden cases additionally match the committed SHA-256 digests.
"""
import json
import os
import sys

import numpy as np
import pytest

import cases
from cases import assert_bits, assert_bits_nan_equal
from atlas_amd import OperatorError, rope_tables_gemma4, rope_tables_llama
from atlas_amd import workloads as wl

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = json.load(open(os.path.join(HERE, "golden", "golden.json")))["cases"]
f32 = np.float32


def say(msg):
    print(f"[gpu-parity] {msg}", flush=True)
    sys.stdout.flush()


def run_golden(rt, ora, name, gpu_fn):
    build, orc = cases.golden_cases()[name]
    inp, meta = build()
    say(f"{name} {meta}")
    exp = orc(ora, inp, meta)
    assert cases.digest(exp) == GOLDEN[name]["sha256"], f"oracle drifted from the golden digest for {name}"
    got = gpu_fn(rt, inp, meta)
    assert_bits(name, got, exp)
    assert cases.digest(got) == GOLDEN[name]["sha256"]


# ------------------------------------------------------------- golden cases

@pytest.mark.parametrize("name", ["c1_rms_norm", "c3_rms_norm", "c3_rms_residual"])
def test_golden_rms(rt, ora, name):
    run_golden(rt, ora, name, cases.rms_gpu)


@pytest.mark.parametrize("name", ["c1_swiglu", "c3_geglu"])
def test_golden_glu(rt, ora, name):
    run_golden(rt, ora, name, cases.glu_gpu)


@pytest.mark.parametrize("name", ["c3_qk_norm_rope_local", "c3_qk_norm_rope_global"])
def test_golden_qk_norm_rope(rt, ora, name):
    def gpu(rt_, inp, m):
        tables = rope_tables_gemma4(inp["pos"], m["rope_stride"], m["head_dim"], m["theta"])
        return cases.qk_gpu(rt_, inp, m, tables)
    run_golden(rt, ora, name, gpu)


@pytest.mark.parametrize("name", ["c1_rope_q", "c1_rope_k", "c2_rope_f16"])
def test_golden_rope_half(rt, ora, name):
    def gpu(rt_, inp, m):
        return cases.rope_half_gpu(rt_, inp, m, rope_tables_llama(inp["pos"], m["head_dim"], m["theta"]))
    run_golden(rt, ora, name, gpu)


def test_golden_embed_f32(rt, ora):
    run_golden(rt, ora, "c1_embed_f32", cases.embed_f32_gpu)


@pytest.mark.parametrize("name", ["c4_embed_q4_0", "c4_embed_q6_k"])
def test_golden_embed_quant(rt, ora, name):
    run_golden(rt, ora, name, cases.embed_q_gpu)


def test_golden_ple(rt, ora):
    run_golden(rt, ora, "c4_ple_q4_0", cases.ple_gpu)


def test_golden_f16(rt, ora):
    run_golden(rt, ora, "c2_add_rms_norm_f16", cases.f16_norm_gpu)
    run_golden(rt, ora, "c2_swiglu_f16", cases.swiglu_f16_gpu)


# ------------------------------------------------- shapes, modes, edge cases

@pytest.mark.parametrize("rows,hidden", [(1, 4), (3, 7), (5, 576), (33, 2048), (256, 1536), (17, 2304), (2, 8192),
                                         (4093, 1536), (2050, 2048), (4100, 576)])
@pytest.mark.parametrize("mode", ["plain", "residual", "addnorm", "addscale"])
def test_rms_modes_ragged(rt, ora, rows, hidden, mode):
    inp, m = cases.rms_case(rows, hidden, 1e-6, 1000 + rows + hidden, mode)
    say(f"rms {mode} rows={rows} hidden={hidden}")
    assert_bits(f"rms_{mode}", cases.rms_gpu(rt, inp, m), cases.rms_oracle(ora, inp, m))


def test_rms_aliasing_like_reference_call_sites(rt, ora):
    """gemma4_executor.rs:4492-4506 binds x=work, normalized=work, residual=out=state;
    :3952 normalises work in place; :4101 adds with out == lhs."""
    rows, h, eps = 64, 1536, 1e-6
    inp, m = cases.rms_case(rows, h, eps, 77, "residual")
    n_exp, out_exp = ora.rms_norm_residual(inp["x"], inp["w"], inp["res"], rows, h, eps)
    say("rms residual aliased")
    work, state, w = rt.upload(inp["x"]), rt.upload(inp["res"]), rt.upload(inp["w"])
    rt.rms_norm_residual(work, w, state, work, state, rows, h, eps)
    rt.sync()
    assert_bits("aliased residual", [work.download(rows * h), state.download(rows * h)], [n_exp, out_exp])
    say("rms in place")
    work = rt.upload(inp["x"])
    rt.rms_norm(work, w, work, rows, h, eps)
    rt.sync()
    assert_bits("in-place rms", [work.download(rows * h)], [ora.rms_norm(inp["x"], inp["w"], rows, h, eps)])
    say("add+norm with residual_out == input")
    a, res = rt.upload(inp["x"]), rt.upload(inp["res"])
    y = rt.empty(rows * h)
    rt.add_rms_norm(a, res, w, a, y, rows, h, eps)
    rt.sync()
    rs_exp, y_exp = ora.add_rms_norm(inp["x"], inp["res"], inp["w"], rows, h, eps)
    assert_bits("aliased add+norm", [a.download(rows * h), y.download(rows * h)], [rs_exp, y_exp])


def test_rms_unaligned_pointer_takes_scalar_path(rt, ora):
    rows, h, eps = 9, 1536, 1e-5
    inp, m = cases.rms_case(rows, h, eps, 78)
    say("rms unaligned")
    buf = rt.empty(rows * h + 4)
    x = buf.offset(4)
    x.upload(inp["x"])
    w = rt.upload(inp["w"])
    y = rt.empty(rows * h + 4).offset(4)
    rt.rms_norm(x, w, y, rows, h, eps)
    rt.sync()
    assert_bits("unaligned rms", [y.download(rows * h)], [ora.rms_norm(inp["x"], inp["w"], rows, h, eps)])


def test_reference_fusion_parity_seeds(rt, ora):
    """The reference's own fused-vs-unfused cases (dispatch_fusion_parity.rs:184-352), LCG inputs."""
    def lcg_fill(n, state):
        out = np.empty(n, f32)
        for i in range(n):
            state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
            out[i] = (f32((state >> 8)) / f32(1 << 24) - f32(0.5)) * f32(2.0)
        return out, state

    state = 0x9E3779B9
    for hidden in [512, 2048, 2304]:
        x, state = lcg_fill(hidden, state)
        w, state = lcg_fill(hidden, state)
        res, state = lcg_fill(hidden, state)
        say(f"rms_residual lcg hidden={hidden}")
        n_exp, out_exp = ora.rms_norm_residual(x, w, res, 1, hidden, 1e-6)
        xb, wb, rb = rt.upload(x), rt.upload(w), rt.upload(res)
        nb, ob = rt.empty(hidden), rt.empty(hidden)
        rt.rms_norm_residual(xb, wb, rb, nb, ob, 1, hidden, 1e-6)
        rt.sync()
        assert_bits("lcg residual", [nb.download(hidden), ob.download(hidden)], [n_exp, out_exp])
    state = 0x853C49E2
    for count in [256, 2048, 8192]:
        g, state = lcg_fill(count, state)
        u, state = lcg_fill(count, state)
        say(f"geglu lcg count={count}")
        gb, ub, ob = rt.upload(g), rt.upload(u), rt.empty(count)
        rt.geglu(gb, ub, ob, count)
        rt.sync()
        assert_bits("lcg geglu", [ob.download(count)], [ora.geglu(g, u)])


@pytest.mark.parametrize("head_dim,rope_stride,q_heads,has_key", [
    (256, 128, 8, True), (256, 256, 8, True), (512, 256, 8, True), (128, 64, 4, True), (256, 128, 8, False),
    (96, 48, 3, True), (64, 32, 2, True)])
@pytest.mark.parametrize("tokens", [37, 300, 600, 1000, 2051])
def test_qk_norm_rope_shapes(rt, ora, head_dim, rope_stride, q_heads, has_key, tokens):
    """Each token engine: a token's units one per wavefront (37 and 300
    tokens; at head_dim 256 each unit folded by candidate segments) or two per
    wavefront (600; odd unit counts leave a last wavefront one unit), one
    token per wavefront (1000) and four per workgroup (2051 tokens: a ragged
    last workgroup)."""
    inp, m = cases.qk_case(tokens, q_heads, head_dim, rope_stride, 1e6, 1e-6, 500 + head_dim, has_key, start=1000)
    tables = rope_tables_gemma4(inp["pos"], rope_stride, head_dim, 1e6)
    say(f"qk_norm_rope {m}")
    assert_bits("qk", cases.qk_gpu(rt, inp, m, tables), cases.qk_oracle(ora, inp, m))


@pytest.mark.parametrize("tokens", [37, 300, 600, 1000])
@pytest.mark.parametrize("head_dim", [256, 128])
def test_qk_norm_rope_exact_fold_adversarial_heads(rt, ora, tokens, head_dim):
    """Heads built to break a reordered or speculative fold (ties, binade
    crossings, zeros, subnormal and overflowing squares, inf and NaN) through
    each token engine: one unit per wavefront (37, 300; at head_dim 256 the
    unit folded by candidate segments, whose misses take the in-order path),
    two units per wavefront (600) and one token per wavefront (1000)."""
    qh = 8
    inp, m = cases.qk_case(tokens, qh, head_dim, head_dim // 2, 1e6, 1e-6, 700 + tokens + head_dim)
    inp["q"] = cases.adversarial_rows(tokens * qh, head_dim, 800 + tokens).reshape(-1)
    inp["k"] = cases.adversarial_rows(tokens, head_dim, 900 + tokens).reshape(-1)
    tables = rope_tables_gemma4(inp["pos"], head_dim // 2, head_dim, 1e6)
    say(f"qk_norm_rope adversarial tokens={tokens} head_dim={head_dim}")
    assert_bits_nan_equal("qk", cases.qk_gpu(rt, inp, m, tables), cases.qk_oracle(ora, inp, m))


def test_qk_norm_rope_in_place_and_decode_positions(rt, ora):
    d, qh, tokens = 256, 8, 256
    r = wl.rng(9)
    q = wl.normal(r, tokens * qh * d)
    k = wl.normal(r, tokens * d)
    qw, kw = wl.normal(r, d, 1, 0.1), wl.normal(r, d, 1, 0.1)
    pos = r.integers(0, 131072, tokens, dtype=np.uint32)
    c, s = rope_tables_gemma4(pos, 128, 256, 1e4)
    say("qk in place, decode positions")
    qb, kb = rt.upload(q), rt.upload(k)
    rt.qk_norm_rope(qb, kb, rt.upload(qw), rt.upload(kw), rt.upload(c), rt.upload(s), qb, kb, tokens, qh, 1, d, 128,
                    1e-6)
    rt.sync()
    qe, ke = ora.qk_norm_rope(q, k, qw, kw, c, s, tokens, qh, True, d, 128, 1e-6)
    assert_bits("qk in place", [qb.download(q.size), kb.download(k.size)], [qe, ke])


def test_rope_tables_match_oracle_tables(ora):
    pos = np.array([0, 1, 7, 4095, 131071], np.uint32)
    for rot, theta in [(256, 1e4), (256, 1e6), (512, 1e6), (128, 1e4)]:
        a = rope_tables_gemma4(pos, 256, rot, theta)
        b = ora.rope_tables_gemma4(pos, 256, rot, theta)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    a, b = rope_tables_llama(pos, 64, 130000.0), ora.rope_tables_llama(pos, 64, 130000.0)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_activations_extremes_and_elementwise(rt, ora):
    r = wl.rng(21)
    x = np.concatenate([np.array([-100.0, -17.29969, -1.0, 0.0, 1.0, 17.29969, 100.0, -1e20, 1e20, -88.9, 88.9,
                                  -104.5, 1e-30, -1e-30], f32), r.uniform(-30, 30, 100003).astype(f32)])
    y = r.standard_normal(x.size).astype(f32)
    n = x.size
    xb, yb, ob = rt.upload(x), rt.upload(y), rt.empty(n)
    for name, fn, exp in [("silu", lambda: rt.silu(xb, ob, n), ora.silu(x)),
                          ("gelu", lambda: rt.gelu(xb, ob, n), ora.gelu(x)),
                          ("swiglu", lambda: rt.swiglu(xb, yb, ob, n), ora.swiglu(x, y)),
                          ("geglu", lambda: rt.geglu(xb, yb, ob, n), ora.geglu(x, y)),
                          ("add", lambda: rt.add(xb, yb, ob, n), ora.add(x, y)),
                          ("multiply", lambda: rt.multiply(xb, yb, ob, n), ora.multiply(x, y)),
                          ("scale", lambda: rt.scale(xb, f32(39.191837), ob, n), ora.scale(x, f32(39.191837)))]:
        say(f"elementwise {name} n={n}")
        fn()
        rt.sync()
        assert_bits(name, [ob.download(n)], [exp])


def test_geglu_offset_ple_slices(rt, ora):
    r = wl.rng(22)
    rows, layers, width = 64, 35, 256
    gate = wl.normal(r, rows * width)
    ple = wl.normal(r, rows * layers * width)
    gb, pb, ob = rt.upload(gate), rt.upload(ple), rt.empty(rows * width)
    for layer in (0, 17, 34):
        say(f"geglu_offset layer={layer}")
        rt.geglu_offset(gb, pb, ob, layer * width, layers * width, width, rows)
        rt.sync()
        assert_bits("geglu_offset", [ob.download(rows * width)],
                    [ora.geglu_offset(gate, ple, layer * width, layers * width, width, rows)])


def test_geglu_offset_extremes_and_scalar_shapes(rt, ora):
    """Overflowing and infinite gates in some wavefronts (the guarded
    GELU form) beside ordinary ones, on each vector form (width 256: one
    value per lane from 16384 values, four per lane below that and from 2^21
    values) and on the scalar one (width 37, offsets not divisible by 4)."""
    r = wl.rng(24)
    for rows, layers, width, layer in [(96, 35, 256, 3), (40, 35, 256, 9), (8200, 2, 256, 1), (50, 7, 37, 5)]:
        gate = r.uniform(-30, 30, rows * width).astype(f32)
        gate[[3, 700, 701, rows * width * 3 // 4]] = [np.inf, -np.inf, f32(-3e13), f32(1e20)]
        gate[rows * width - 1] = f32(-1e20)
        ple = wl.normal(r, rows * layers * width)
        gb, pb, ob = rt.upload(gate), rt.upload(ple), rt.empty(rows * width)
        say(f"geglu_offset extremes rows={rows} width={width} layer={layer}")
        rt.geglu_offset(gb, pb, ob, layer * width, layers * width, width, rows)
        rt.sync()
        assert_bits("geglu_offset extremes", [ob.download(rows * width)],
                    [ora.geglu_offset(gate, ple, layer * width, layers * width, width, rows)])


@pytest.mark.parametrize("width,groups", [(256, 35 * 64), (250, 37), (64, 11), (512, 35), (1024, 9), (1000, 13),
                                          (2000, 7)])
def test_groups_stable(rt, ora, width, groups):
    """Widths held in registers (64, 250: not a multiple of 4, 256, 512,
    1000, 1024) and the general kernel above 1024; an all-zero group and one
    of 1e30 (whose squares overflow without the max scaling)."""
    r = wl.rng(23 + width)
    v = wl.normal(r, (groups, width))
    v[5] = 0.0
    v[9 % groups] *= f32(1e30)
    w = wl.normal(r, width, 1, 0.1)
    say(f"groups stable width={width} groups={groups}")
    vb = rt.upload(v)
    rt.rms_norm_groups_stable(vb, rt.upload(w), width, groups, 1e-6)
    rt.sync()
    assert_bits("groups", [vb.download(v.size)], [ora.rms_norm_groups_stable(v, w, width, groups, 1e-6)])


def test_full_size_gathers_c4(rt, ora):
    S = wl.QuantGatherShape()
    for q6 in (False, True):
        inp, m = cases.embed_q_case(S.vocab, S.hidden, S.tokens, 600 + q6, q6)
        inp["ids"][:4] = [0, S.vocab - 1, S.vocab - 1, 0]      # boundary rows, repeated ids
        say(f"embed full vocab q6={q6}")
        assert_bits("embed", cases.embed_q_gpu(rt, inp, m), cases.embed_q_oracle(ora, inp, m))


@pytest.mark.parametrize("fmt", ["q4_0", "q6_k", "q8_0"])
@pytest.mark.parametrize("hidden,tokens", [(256, 1), (1536, 4097), (2048, 3), (8960, 65), (19968, 9), (20224, 9), (20224, 2049),
                                           (28672, 5), (29184, 5), (65536, 3)])
def test_embed_quant_shapes(rt, ora, fmt, hidden, tokens):
    """Every packed gather format over row widths that keep four rows per
    workgroup in LDS and ones that do not (Q6_K > 19968, Q4_0 > 28672 values),
    ragged grids and the maximum width; ids include the first and last row.
    Q8_0 is the Llama resident embedding (executor.rs:1541-1549) with the
    reference's scale of 1; the others are scaled by sqrt(hidden)."""
    if fmt == "q6_k" and hidden % 256:
        pytest.skip("Q6_K needs hidden % 256 == 0")
    vocab = 257
    inp, m = cases.embed_q_case(vocab, hidden, tokens, 640 + hidden + tokens, fmt == "q6_k", fmt)
    inp["ids"][0] = vocab - 1
    if fmt == "q8_0":
        m["scale"] = 1.0
    say(f"embed {fmt} hidden={hidden} tokens={tokens}")
    assert_bits(f"embed {fmt}", cases.embed_q_gpu(rt, inp, m), cases.embed_q_oracle(ora, inp, m))


# f16 scale patterns: +-0, subnormals, +-max, +-inf and NaNs with payloads
_SPECIAL_D = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x8001, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0xFE00,
                       0x7C01, 0x3C00, 0xBC00], np.uint16)


@pytest.mark.parametrize("fmt", ["q6_k", "q4_0"])
def test_embed_quant_special_scales(rt, ora, fmt):
    """Block scales d cycling through +-0, subnormals, +-max, +-inf and NaNs,
    with zero codes (q = 32 for Q6_K, nibble 8 for Q4_0) and Q6_K sub-scales
    of 0, -128 and 127 in every block: the device gather equals the oracle
    bit for bit, NaNs equal to NaNs (the Q6_K decode forms sc * d once per
    super-block, the reference (q * sc) * d)."""
    vocab, hidden, tokens = 64, 1536, 96
    inp, m = cases.embed_q_case(vocab, hidden, tokens, 727, fmt == "q6_k", fmt)
    step = 210 if fmt == "q6_k" else 18
    t = inp["table"].reshape(-1, step)
    nblk = t.shape[0]
    d = _SPECIAL_D[np.arange(nblk) % _SPECIAL_D.size]
    if fmt == "q6_k":
        t[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
        t[:, 192] = 0                               # sub-scale 0
        t[:, 193] = 0x80                            # -128
        t[:, 194] = 0x7F                            # 127
        t[:, 0] = 0x00                              # ql low nibble 0 ...
        t[:, 128] = 0x02                            # ... with qh bits 2 -> q = 32 (a zero code)
    else:
        t[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        t[:, 2] = 0x88                              # nibbles 8: zero codes
    inp["table"] = t.reshape(-1)
    say(f"embed {fmt} special scales")
    with np.errstate(all="ignore"):
        exp = cases.embed_q_oracle(ora, inp, m)
    cases.assert_bits_nan_equal(f"embed {fmt} special scales", cases.embed_q_gpu(rt, inp, m), exp)


@pytest.mark.parametrize("fmt", ["q4_0", "q6_k", "q8_0"])
def test_embed_quant_table_at_any_offset(rt, ora, fmt):
    """The gather stages a row through the 16-byte-aligned span around it:
    tables starting at every even skew of a 16-byte line (rows then start
    at skews 0-14), and at odd addresses, which take the generic staging,
    give the same bits.  Row widths 1536 (C4) and 8960 (the PLE row); ids
    include the first and last row."""
    vocab, tokens = 97, 70
    for hidden in (1536, 8960):
        inp, m = cases.embed_q_case(vocab, hidden, tokens, 660 + hidden, fmt == "q6_k", fmt)
        inp["ids"][:3] = [0, vocab - 1, 0]
        exp = cases.embed_q_oracle(ora, inp, m)
        table = inp["table"]
        fn = {"q4_0": rt.embed_q4_0, "q6_k": rt.embed_q6_k, "q8_0": rt.embed_q8_0}[fmt]
        ids = rt.upload(inp["ids"])
        n = tokens * hidden
        o = rt.empty(n)
        for off in (0, 2, 4, 6, 10, 14, 1, 7):
            say(f"embed {fmt} hidden={hidden} table offset {off}")
            buf = rt.alloc(table.nbytes + 16, np.uint8)
            t = buf.offset(off, np.uint8).upload(table)
            rt.memset(o, 0, n * 4)
            fn(t, ids, o, vocab, hidden, tokens, m["scale"])
            rt.sync()
            assert_bits(f"embed {fmt} offset {off}", [o.download(n)], exp)
            rt.free(buf)


def test_embed_q8_0_out_of_range_and_scale(rt, ora):
    """Q8_0 ids at and past the vocabulary leave rows untouched
    (kernels.metal:660); a non-unit scale rounds once after the exact dequant."""
    vocab, h = 100, 1536
    ids = np.array([1, 100, 5, 4000000000, 99, 0], np.uint32)
    inp, m = cases.embed_q_case(vocab, h, ids.size, 650, False, "q8_0")
    tb, ib = rt.upload(inp["table"]), rt.upload(ids)
    for scale in (1.0, float(wl.f32_sqrt(h))):
        sentinel = np.full(ids.size * h, 7.0, f32)
        ob = rt.upload(sentinel)
        say(f"embed q8_0 out-of-range ids scale={scale}")
        rt.embed_q8_0(tb, ib, ob, vocab, h, ids.size, scale)
        rt.sync()
        exp = ora.embed_q8_0(inp["table"], ids, vocab, h, scale, out=sentinel)
        assert_bits("q8_0 oob untouched", [ob.download(ids.size * h)], [exp])
        assert np.all(exp.reshape(ids.size, -1)[[1, 3]] == 7.0)
    with pytest.raises(OperatorError) as e:
        rt.embed_q8_0(tb, ib, rt.empty(ids.size * 48), vocab, 48, ids.size)   # hidden % 32 != 0
    assert e.value.kind == "InvalidInput"


def test_full_size_ple_c4(rt, ora):
    S = wl.QuantGatherShape()
    inp, m = cases.ple_case(S.vocab, S.ple_layers, S.ple_width, S.tokens, 610, False)
    say("ple full size q4_0")
    assert_bits("ple", cases.ple_gpu(rt, inp, m), cases.ple_oracle(ora, inp, m))
    inp, m = cases.ple_case(4096, S.ple_layers, S.ple_width, 1024, 611, True)
    say("ple q6_k")
    assert_bits("ple q6", cases.ple_gpu(rt, inp, m), cases.ple_oracle(ora, inp, m))


def test_out_of_range_ids_follow_reference(rt, ora):
    vocab, h, t = 100, 512, 6
    ids = np.array([1, 100, 5, 4000000000, 99, 0], np.uint32)
    for q6 in (False, True):
        inp, m = cases.embed_q_case(vocab, h, t, 620, q6)
        inp["ids"] = ids
        say(f"out-of-range ids q6={q6}")
        tb, ib = rt.upload(inp["table"]), rt.upload(ids)
        sentinel = np.full(t * h, 7.0, f32)
        ob = rt.upload(sentinel)
        (rt.embed_q6_k if q6 else rt.embed_q4_0)(tb, ib, ob, vocab, h, t, m["scale"])
        rt.sync()
        exp = (ora.embed_q6_k if q6 else ora.embed_q4_0)(inp["table"], ids, vocab, h, m["scale"], out=sentinel)
        assert_bits("oob untouched", [ob.download(t * h)], [exp])
        # a table with no rows: every id is out of range and nothing is read or written
        say(f"empty table q6={q6}")
        ob = rt.upload(sentinel)
        (rt.embed_q6_k if q6 else rt.embed_q4_0)(rt.empty(4), ib, ob, 0, h, t, m["scale"])
        rt.sync()
        assert_bits("vocab 0 untouched", [ob.download(t * h)], [sentinel])
    table = wl.normal(wl.rng(1), vocab * h)
    tb, ib, ob = rt.upload(table), rt.upload(ids), rt.empty(t * h)
    rt.embed_f32(tb, ib, ob, vocab, h, t)
    rt.sync()
    assert_bits("oob f32 zeros", [ob.download(t * h)], [ora.embed_f32(table, ids, vocab, h)])


def test_ple_out_of_range_ids_leave_rows_untouched(rt, ora):
    """PLE gather-combine with ids at and far past the vocabulary: those token
    rows keep what the output held (the Q4/Q6 lookups skip them,
    kernels.metal:655,686), the others match the oracle; a row width that is
    not a whole number of 1024-value segments (35 x 256)."""
    vocab, layers, width = 100, 35, 256
    ids = np.array([1, 100, 5, 4000000000, 99, 0, 101, 50], np.uint32)
    for q6 in (False, True):
        inp, m = cases.ple_case(vocab, layers, width, ids.size, 630 + q6, q6)
        inp["ids"] = ids
        n = inp["proj"].size
        sentinel = np.full(n, 7.0, f32)
        say(f"ple out-of-range ids q6={q6}")
        tb, ib, pb, ob = rt.upload(inp["table"]), rt.upload(ids), rt.upload(inp["proj"]), rt.upload(sentinel)
        (rt.ple_q6_k if q6 else rt.ple_q4_0)(tb, ib, pb, ob, vocab, layers, width, ids.size, m["es"], m["os"])
        rt.sync()
        exp = ora.ple(inp["table"], ids, inp["proj"], vocab, layers, width, m["es"], m["os"], q6=q6, out=sentinel)
        assert_bits("ple oob untouched", [ob.download(n)], [exp])
        assert np.all(exp.reshape(ids.size, -1)[[1, 3, 6]] == 7.0)
        # an empty table (vocab 0) is invalid input: no row may be staged from it
        say(f"ple vocab 0 q6={q6}")
        with pytest.raises(OperatorError) as e:
            (rt.ple_q6_k if q6 else rt.ple_q4_0)(tb, ib, pb, ob, 0, layers, width, ids.size, m["es"], m["os"])
        assert e.value.kind == "InvalidInput"


def test_wide_reduction_is_tolerance_level(rt, ora):
    """ATLAS_REDUCTION_WIDE reorders the sum of squares: plain RMSNorm stays
    within 1e-5 relative per element; epilogues that cancel are checked
    normwise (1e-6) since an elementwise bound is not meaningful there."""
    from atlas_amd import ATLAS_REDUCTION_SEQUENTIAL, ATLAS_REDUCTION_WIDE
    rows, h, eps = 512, 1536, 1e-6
    inp, m = cases.rms_case(rows, h, eps, 91)
    rt.set_reduction(ATLAS_REDUCTION_WIDE)
    try:
        say("wide rms")
        got = cases.rms_gpu(rt, inp, m)[0]
        exp = cases.rms_oracle(ora, inp, m)[0]
        assert np.max(np.abs(got - exp) / np.abs(exp)) <= 1e-5
        m2 = dict(m, mode="residual")
        got_n, got_o = cases.rms_gpu(rt, inp, m2)
        exp_n, exp_o = cases.rms_oracle(ora, inp, m2)
        assert np.max(np.abs(got_n - exp_n) / np.abs(exp_n)) <= 1e-5
        assert np.linalg.norm(got_o - exp_o) / np.linalg.norm(exp_o) <= 1e-6
        # every token engine (one or two units per wavefront, one or four
        # tokens per workgroup) at head_dim 256, and head_dim 128 and 512
        for tokens, heads, d in [(64, 8, 256), (300, 8, 256), (600, 8, 256), (1000, 8, 256), (2051, 8, 256),
                                 (37, 4, 128), (300, 8, 512)]:
            qinp, qm = cases.qk_case(tokens, heads, d, d // 2, 1e4, 1e-6, 92 + tokens)
            tables = rope_tables_gemma4(qinp["pos"], d // 2, d, 1e4)
            say(f"wide qk tokens={tokens} heads={heads} head_dim={d}")
            gq = cases.qk_gpu(rt, qinp, qm, tables)
            eq = cases.qk_oracle(ora, qinp, qm)
            for g_, e_ in zip(gq, eq):
                assert np.linalg.norm(g_ - e_) / np.linalg.norm(e_) <= 1e-6
    finally:
        rt.set_reduction(ATLAS_REDUCTION_SEQUENTIAL)


@pytest.mark.parametrize("rows", [2048 + 48, 2048 + 47, 1024 + 16])
@pytest.mark.parametrize("hidden", [1536, 2048, 576, 1024, 260, 1280, 1792])
@pytest.mark.parametrize("mode", ["plain", "residual", "addnorm", "addscale"])
def test_rms_exact_fold_adversarial_rows(rt, ora, rows, hidden, mode):
    """Both folds of the register engine against the oracle's sequential sum on
    rows built to break a reordered or wave-parallel fold.  Below 2048 rows every
    mode uses one row per wavefront and the exact wave-parallel fold with its
    scans computed ahead by a helper wavefront (the walk across binade
    crossings, ties, subnormal, inf and NaN stretches); from 2048 rows up, plain
    RMSNorm keeps the chunked parallel fold and the epilogue modes fold in order
    with two rows per wavefront up to the last chunk, which takes the parallel
    fold (2 to 8 chunks per row; an odd row count leaves the last wavefront
    one row)."""
    inp, m = cases.rms_case(rows, hidden, 1e-6, 4000 + hidden, mode)
    inp["x"] = cases.adversarial_rows(rows, hidden, 5000 + hidden)
    say(f"rms exact fold adversarial {mode} rows={rows} hidden={hidden}")
    assert_bits_nan_equal(f"rms_{mode}", cases.rms_gpu(rt, inp, m), cases.rms_oracle(ora, inp, m))


@pytest.mark.parametrize("rows,hidden", [(1, 8), (33, 576), (2050, 2048), (7, 4096), (19, 2056), (5, 1000),
                                         (3, 8200), (4100, 64)])
def test_f16_norms_shapes(rt, ora, rows, hidden):
    """FP16-storage RMSNorm and add+RMSNorm: register engine (hidden % 8 == 0,
    <= 4096, both row-per-wave counts) and the LDS fallback."""
    inp, m = cases.f16_norm_case(rows, hidden, 1e-5, 7000 + rows + hidden)
    say(f"f16 norms rows={rows} hidden={hidden}")
    assert_bits("f16 norms", cases.f16_norm_gpu(rt, inp, m), cases.f16_norm_oracle(ora, inp, m))


@pytest.mark.parametrize("rows,hidden", [(2048 + 37, 2048), (512 + 5, 2048), (300, 4096), (77, 1536)])
def test_f16_norm_exact_fold_adversarial_rows(rt, ora, rows, hidden):
    """The FP16 register engine's in-order fold against the oracle's sequential
    sum on adversarial f16 rows, both the plain and the add+norm form."""
    inp, m = cases.f16_norm_case(rows, hidden, 1e-5, 7100 + rows + hidden)
    inp["x"] = cases.adversarial_f16_rows(rows, hidden, 7200 + hidden)
    say(f"f16 norms adversarial rows={rows} hidden={hidden}")
    got, exp = cases.f16_norm_gpu(rt, inp, m), cases.f16_norm_oracle(ora, inp, m)
    for name, g, e in zip(("residual_out", "add+norm", "norm"), got, exp):
        gf, ef = g.view(np.float16), e.view(np.float16)
        same = (g == e) | (np.isnan(gf) & np.isnan(ef))
        if not same.all():
            j = int(np.nonzero(~same)[0][0])
            raise AssertionError(f"f16 {name}: {int((~same).sum())} of {g.size} differ; first at {j}: "
                                 f"gpu={gf[j]!r} oracle={ef[j]!r}")


def test_f16_norm_aliasing(rt, ora):
    """residual_out == input (the pre-norm add writes the residual stream in place)."""
    rows, h = 64, 2048
    inp, m = cases.f16_norm_case(rows, h, 1e-5, 7777)
    rs_exp, y_exp = ora.add_rms_norm_f16(inp["x"], inp["res"], inp["w"], rows, h, 1e-5)
    say("f16 add+norm in place")
    x, res, w = rt.upload(inp["x"]), rt.upload(inp["res"]), rt.upload(inp["w"])
    y = rt.empty(rows * h, np.uint16)
    rt.add_rms_norm_f16(x, res, w, x, y, rows, h, 1e-5)
    rt.sync()
    assert_bits("f16 in place", [x.download(rows * h), y.download(rows * h)], [rs_exp, y_exp])


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("tokens,heads,head_dim", [(2048, 32, 64), (37, 3, 128), (5, 2, 96), (9, 4, 6), (3, 1, 256),
                                                   (11, 5, 24), (301, 40, 64), (513, 16, 128), (1025, 9, 256)])
def test_rope_half_shapes(rt, ora, f16, tokens, heads, head_dim):
    """Half-split RoPE: the token engine (>= 8192 rows; ragged last workgroup, 1-8 head
    steps per lane, or the per-pair fallback when a lane would need more), the 128-bit
    per-pair paths (half % 4 / % 8) and the scalar path."""
    inp, m = cases.rope_half_case(tokens, heads, head_dim, 130000.0, 8000 + tokens + head_dim, f16)
    say(f"rope_half f16={f16} tokens={tokens} heads={heads} head_dim={head_dim}")
    tables = rope_tables_llama(inp["pos"], head_dim, 130000.0)
    assert_bits("rope_half", cases.rope_half_gpu(rt, inp, m, tables), cases.rope_half_oracle(ora, inp, m))


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("tokens,q_heads,k_heads,head_dim", [(2048, 32, 32, 64), (128, 9, 3, 64), (37, 4, 1, 128),
                                                             (5, 3, 2, 96), (9, 2, 1, 6), (1023, 24, 8, 64),
                                                             (777, 13, 5, 128)])
def test_rope_half_qk_one_launch(rt, ora, f16, tokens, q_heads, k_heads, head_dim):
    """Q and K in one launch (the Llama decode's two rope chains, executor.rs:1120-1166) give
    exactly the two single-tensor results; an unaligned K takes the scalar path for both."""
    q_inp, qm = cases.rope_half_case(tokens, q_heads, head_dim, 130000.0, 9100 + tokens, f16)
    k_inp, km = cases.rope_half_case(tokens, k_heads, head_dim, 130000.0, 9200 + tokens, f16)
    say(f"rope_half_qk f16={f16} tokens={tokens} q_heads={q_heads} k_heads={k_heads} head_dim={head_dim}")
    exp = cases.rope_half_oracle(ora, q_inp, qm) + cases.rope_half_oracle(ora, k_inp, km)
    c, s = rope_tables_llama(q_inp["pos"], head_dim, 130000.0)
    dt = q_inp["x"].dtype
    item = np.dtype(dt).itemsize
    for k_offset in (0, 1):
        cb, sb = rt.upload(c), rt.upload(s)
        qb = rt.upload(q_inp["x"])
        kraw = np.zeros(k_inp["x"].size + 1, dt)
        kraw[k_offset:k_offset + k_inp["x"].size] = k_inp["x"]
        kb = rt.upload(kraw)
        qo, ko = rt.empty(q_inp["x"].size, dt), rt.empty(kraw.size, dt)
        rt.rope_half_qk(qb, kb.ptr + item * k_offset, cb, sb, qo, ko.ptr + item * k_offset, tokens, q_heads,
                        k_heads, head_dim, head_dim // 2, f16=f16)
        rt.sync()
        got_k = ko.download(kraw.size, dt)[k_offset:k_offset + k_inp["x"].size]
        assert_bits(f"rope_half_qk k_offset={k_offset}", [qo.download(q_inp["x"].size, dt), got_k], exp)


def test_swiglu_f16_zero_signs_and_specials(rt, ora):
    """FP16 SwiGLU multiplies the activated gate by `up` with the f16 operand
    widened inside the multiply: products of +-0 keep their signs, subnormal
    and extreme `up` values round once, inf and NaN propagate.  The first
    4096 values hold only gates below 87 in magnitude (the in-range path of
    every wavefront), the rest mix in infinite, NaN and saturating gates
    (the guarded path)."""
    h16 = lambda a: np.asarray(a, np.float16).view(np.uint16)
    r = wl.rng(4242)
    n = 8192
    g = r.standard_normal(n).astype(np.float32) * np.float32(3.0)
    u = r.standard_normal(n).astype(np.float32)
    specials_u = np.array([0.0, -0.0, 6e-8, -6e-8, 6.1e-5, 65504.0, -65504.0, 1e-3], np.float32)
    u[:4096:7] = np.resize(specials_u, u[:4096:7].size)
    g[:4096:5] = np.resize(np.array([0.0, -0.0, 86.9, -86.9, 6e-8, -1e-4], np.float32), g[:4096:5].size)
    g[4096::3] = np.resize(np.array([np.inf, -np.inf, np.nan, 100.0, -100.0, 65504.0], np.float32), g[4096::3].size)
    u[4096::4] = np.resize(np.array([np.inf, -np.inf, np.nan, 0.0, -0.0], np.float32), u[4096::4].size)
    gb, ub = h16(g), h16(u)
    say("swiglu f16 zero signs and specials")
    got = cases.swiglu_f16_gpu(rt, {"gate": gb, "up": ub}, {"n": n})
    exp = np.asarray(ora.swiglu_f16(gb, ub), np.uint16)
    g16, e16 = np.asarray(got[0], np.uint16), exp
    same = (g16 == e16) | (np.isnan(g16.view(np.float16)) & np.isnan(e16.view(np.float16)))
    assert same.all(), f"{int((~same).sum())} of {n} differ; first at {int(np.nonzero(~same)[0][0])}"
    # the zero products keep their signs
    zero = (e16 & 0x7fff) == 0
    assert zero.sum() > 100 and np.array_equal(g16[zero], e16[zero])


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_rope_half_token_engine_signed_zeros_and_specials(rt, ora, f16, head_dim):
    """The token engine takes both halves as own*c + par*s', s' = -s on the
    first half's lanes: bit-identical to the reference's x0*c - x1*s and
    x0*s + x1*c for every finite input, signed zeros included -- rows of +-0 in
    either half (all four sign pairs), at position 0 (cos 1, sin 0) and at
    other positions -- and NaN where the reference gives NaN (infinities,
    NaN; compared NaN-equal).  f16 at head_dim 64 / 128 and f32 at 64 take the
    two mirrored DPP layouts, f32 at 128 the shuffle exchange."""
    tokens, heads = 2048, 8
    half = head_dim // 2
    r = wl.rng(4242 + head_dim + f16)
    x = wl.normal(r, tokens * heads * head_dim).reshape(tokens, heads, 2, half)
    zero_pairs = [(0.0, 0.0), (-0.0, 0.0), (0.0, -0.0), (-0.0, -0.0)]
    for i, (a, b) in enumerate(zero_pairs):
        x[i::16, :, 0, :] = a           # rows of position 0 and later ones
        x[i::16, :, 1, :] = b
    x[4::16, :, 1, :] = -0.0            # one half zero, the other normal
    x[5::16, :, 0, :] = -0.0
    x[6::16, :, 0, ::3] = np.inf
    x[7::16, :, 1, 1::3] = -np.inf
    x[8::16, :, 0, 2::5] = np.nan
    x[9::16, :, 1, ::7] = np.nan
    x = x.reshape(-1).astype(np.float32)
    if f16:
        x = x.astype(np.float16).view(np.uint16)
    inp, m = {"x": x, "pos": np.arange(tokens, dtype=np.uint32)}, dict(
        tokens=tokens, heads=heads, head_dim=head_dim, theta=130000.0, f16=f16)
    say(f"rope_half specials f16={f16} head_dim={head_dim}")
    got = cases.rope_half_gpu(rt, inp, m, rope_tables_llama(inp["pos"], head_dim, 130000.0))[0]
    exp = cases.rope_half_oracle(ora, inp, m)[0]
    if f16:
        g, e = got.view(np.float16), exp.view(np.float16)
        same = (got == exp) | (np.isnan(g) & np.isnan(e))
        assert same.all(), f"{int((~same).sum())} differ; first at {int(np.nonzero(~same)[0][0])}"
        zero = (exp & 0x7fff) == 0
    else:
        assert_bits_nan_equal("rope_half specials", [got], [exp])
        zero = (exp.view(np.uint32) & 0x7fffffff) == 0
    assert zero.sum() > 1000 and np.signbit(exp[zero].view(np.float16 if f16 else np.float32)).any()
