"""Seeded parity cases shared by the golden-fixture generator, the CPU
golden check and the GPU parity tests.

Each case builds its inputs from a seed (numpy PCG64), evaluates the CPU
oracle, and (on a GPU box) runs the same inputs through the HIP library's C
ABI.  All ops in their default (sequential-reduction) mode are expected to be
bit-identical to the oracle, so outputs are compared as raw bytes and the
golden fixtures store SHA-256 digests of the oracle outputs.
"""
from __future__ import annotations

import hashlib

import numpy as np

from atlas_amd import workloads as wl

f32 = np.float32


def digest(arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# -------------------------------------------------------------- comparisons

def assert_bits(name, got, exp):
    assert len(got) == len(exp), name
    for i, (g, e) in enumerate(zip(got, exp)):
        g, e = np.asarray(g).reshape(-1), np.asarray(e).reshape(-1)
        assert g.shape == e.shape, (name, i, g.shape, e.shape)
        gb, eb = g.view(np.uint8), e.view(np.uint8)
        if not np.array_equal(gb, eb):
            gf, ef = g.astype(np.float64), e.astype(np.float64)
            mism = np.nonzero((g != e) & ~(np.isnan(gf) & np.isnan(ef)))[0]
            j = mism[0] if mism.size else 0
            raise AssertionError(f"{name}[{i}]: {mism.size} of {g.size} elements differ; first at {j}: "
                                 f"gpu={g[j]!r} oracle={e[j]!r} max_abs={np.nanmax(np.abs(gf - ef)):.3e}")


def assert_bits_nan_equal(name, got, exp):
    for i, (g, e) in enumerate(zip(got, exp)):
        g, e = np.asarray(g).reshape(-1), np.asarray(e).reshape(-1)
        same = (g.view(np.uint32) == e.view(np.uint32)) | (np.isnan(g) & np.isnan(e))
        if not same.all():
            j = int(np.nonzero(~same)[0][0])
            raise AssertionError(f"{name}[{i}]: {int((~same).sum())} of {g.size} differ; first at {j}: "
                                 f"gpu={g[j]!r} oracle={e[j]!r}")


# ---------------------------------------------------------------- builders

def rms_case(rows, hidden, eps, seed, mode="plain"):
    r = wl.rng(seed)
    inp = {"x": wl.normal(r, rows * hidden), "w": wl.normal(r, hidden, 1.0, 0.1),
           "res": wl.normal(r, rows * hidden), "scale": np.array([0.6180339], f32)}
    meta = dict(rows=rows, hidden=hidden, eps=eps, mode=mode)
    return inp, meta


def rms_oracle(ora, inp, m):
    rows, h, eps = m["rows"], m["hidden"], m["eps"]
    if m["mode"] == "plain":
        return [ora.rms_norm(inp["x"], inp["w"], rows, h, eps)]
    if m["mode"] == "residual":
        n, out = ora.rms_norm_residual(inp["x"], inp["w"], inp["res"], rows, h, eps)
        return [n, out]
    if m["mode"] == "addnorm":
        rs, y = ora.add_rms_norm(inp["x"], inp["res"], inp["w"], rows, h, eps)
        return [rs, y]
    return [ora.rms_norm_add_scale(inp["x"], inp["w"], inp["res"], inp["scale"][0], rows, h, eps)]


def rms_gpu(rt, inp, m):
    rows, h, eps = m["rows"], m["hidden"], m["eps"]
    x, w, res = rt.upload(inp["x"]), rt.upload(inp["w"]), rt.upload(inp["res"])
    n = rows * h
    if m["mode"] == "plain":
        y = rt.empty(n)
        rt.rms_norm(x, w, y, rows, h, eps)
        rt.sync()
        return [y.download(n)]
    if m["mode"] == "residual":
        nb, out = rt.empty(n), rt.empty(n)
        rt.rms_norm_residual(x, w, res, nb, out, rows, h, eps)
        rt.sync()
        return [nb.download(n), out.download(n)]
    if m["mode"] == "addnorm":
        rs, y = rt.empty(n), rt.empty(n)
        rt.add_rms_norm(x, res, w, rs, y, rows, h, eps)
        rt.sync()
        return [rs.download(n), y.download(n)]
    sc = rt.upload(inp["scale"])
    rt.rms_norm_add_scale(x, w, res, sc, rows, h, eps)
    rt.sync()
    return [res.download(n)]


def qk_case(tokens, q_heads, head_dim, rope_stride, theta, eps, seed, has_key=True, start=0):
    r = wl.rng(seed)
    q = wl.normal(r, tokens * q_heads * head_dim)
    k = wl.normal(r, tokens * head_dim)
    qw = wl.normal(r, head_dim, 1.0, 0.1)
    kw = wl.normal(r, head_dim, 1.0, 0.1)
    pos = np.arange(start, start + tokens, dtype=np.uint32)
    return {"q": q, "k": k, "qw": qw, "kw": kw, "pos": pos}, dict(
        tokens=tokens, q_heads=q_heads, head_dim=head_dim, rope_stride=rope_stride, theta=theta, eps=eps,
        has_key=has_key)


def qk_tables(ora, inp, m):
    return ora.rope_tables_gemma4(inp["pos"], m["rope_stride"], m["head_dim"], m["theta"])


def qk_oracle(ora, inp, m):
    c, s = qk_tables(ora, inp, m)
    qo, ko = ora.qk_norm_rope(inp["q"], inp["k"], inp["qw"], inp["kw"], c, s, m["tokens"], m["q_heads"],
                              m["has_key"], m["head_dim"], m["rope_stride"], m["eps"])
    return [qo] + ([ko] if m["has_key"] else [])


def qk_gpu(rt, inp, m, tables):
    c, s = tables
    q, k = rt.upload(inp["q"]), rt.upload(inp["k"])
    qw, kw = rt.upload(inp["qw"]), rt.upload(inp["kw"])
    cb, sb = rt.upload(c), rt.upload(s)
    qo, ko = rt.empty(inp["q"].size), rt.empty(inp["k"].size)
    rt.qk_norm_rope(q, k, qw, kw, cb, sb, qo, ko, m["tokens"], m["q_heads"], 1 if m["has_key"] else 0,
                    m["head_dim"], m["rope_stride"], m["eps"])
    rt.sync()
    return [qo.download(inp["q"].size)] + ([ko.download(inp["k"].size)] if m["has_key"] else [])


def glu_case(n, seed, kind):
    r = wl.rng(seed)
    return {"gate": wl.normal(r, n), "up": wl.normal(r, n)}, dict(n=n, kind=kind)


def glu_oracle(ora, inp, m):
    return [ora.geglu(inp["gate"], inp["up"]) if m["kind"] == "geglu" else ora.swiglu(inp["gate"], inp["up"])]


def glu_gpu(rt, inp, m):
    g, u, o = rt.upload(inp["gate"]), rt.upload(inp["up"]), rt.empty(m["n"])
    (rt.geglu if m["kind"] == "geglu" else rt.swiglu)(g, u, o, m["n"])
    rt.sync()
    return [o.download(m["n"])]


def embed_q_case(vocab, hidden, tokens, seed, q6, fmt=None):
    """Token gather from a packed table: fmt "q4_0", "q6_k" (q6=True) or "q8_0"."""
    fmt = fmt or ("q6_k" if q6 else "q4_0")
    r = wl.rng(seed)
    make = {"q4_0": wl.q4_0_table, "q6_k": wl.q6_k_table, "q8_0": wl.q8_0_table}[fmt]
    table = make(r, vocab, hidden)
    ids = wl.token_ids(r, tokens, vocab)
    return {"table": table, "ids": ids}, dict(vocab=vocab, hidden=hidden, tokens=tokens, q6=fmt == "q6_k",
                                              fmt=fmt, scale=float(wl.f32_sqrt(hidden)))


def embed_q_oracle(ora, inp, m):
    fn = {"q4_0": ora.embed_q4_0, "q6_k": ora.embed_q6_k, "q8_0": ora.embed_q8_0}[m.get("fmt", "q6_k" if m["q6"]
                                                                                    else "q4_0")]
    return [fn(inp["table"], inp["ids"], m["vocab"], m["hidden"], m["scale"])]


def embed_q_gpu(rt, inp, m):
    t, ids = rt.upload(inp["table"]), rt.upload(inp["ids"])
    n = m["tokens"] * m["hidden"]
    o = rt.empty(n)
    rt.memset(o, 0, n * 4)
    fn = {"q4_0": rt.embed_q4_0, "q6_k": rt.embed_q6_k, "q8_0": rt.embed_q8_0}[m.get("fmt", "q6_k" if m["q6"]
                                                                                   else "q4_0")]
    fn(t, ids, o, m["vocab"], m["hidden"], m["tokens"], m["scale"])
    rt.sync()
    return [o.download(n)]


def ple_case(vocab, layers, width, tokens, seed, q6):
    r = wl.rng(seed)
    row = layers * width
    table = wl.q6_k_table(r, vocab, row) if q6 else wl.q4_0_table(r, vocab, row)
    ids = wl.token_ids(r, tokens, vocab)
    proj = wl.normal(r, tokens * row)
    return {"table": table, "ids": ids, "proj": proj}, dict(vocab=vocab, layers=layers, width=width, tokens=tokens,
                                                            q6=q6, es=16.0, os=float(wl.SQRT_2_RECIP))


def ple_oracle(ora, inp, m):
    return [ora.ple(inp["table"], inp["ids"], inp["proj"], m["vocab"], m["layers"], m["width"], m["es"], m["os"],
                    q6=m["q6"])]


def ple_gpu(rt, inp, m):
    t, ids, p = rt.upload(inp["table"]), rt.upload(inp["ids"]), rt.upload(inp["proj"])
    n = inp["proj"].size
    o = rt.empty(n)
    (rt.ple_q6_k if m["q6"] else rt.ple_q4_0)(t, ids, p, o, m["vocab"], m["layers"], m["width"], m["tokens"],
                                             m["es"], m["os"])
    rt.sync()
    return [o.download(n)]


def embed_f32_case(vocab, hidden, tokens, seed):
    r = wl.rng(seed)
    table = wl.normal(r, vocab * hidden, 0.0, 0.02)
    ids = wl.token_ids(r, tokens, vocab)
    return {"table": table, "ids": ids}, dict(vocab=vocab, hidden=hidden, tokens=tokens)


def embed_f32_oracle(ora, inp, m):
    return [ora.embed_f32(inp["table"], inp["ids"], m["vocab"], m["hidden"])]


def embed_f32_gpu(rt, inp, m):
    t, ids = rt.upload(inp["table"]), rt.upload(inp["ids"])
    n = m["tokens"] * m["hidden"]
    o = rt.empty(n)
    rt.embed_f32(t, ids, o, m["vocab"], m["hidden"], m["tokens"])
    rt.sync()
    return [o.download(n)]


def rope_half_case(tokens, heads, head_dim, theta, seed, f16=False):
    r = wl.rng(seed)
    x = wl.normal(r, tokens * heads * head_dim)
    if f16:
        x = x.astype(np.float16).view(np.uint16)
    return {"x": x, "pos": np.arange(tokens, dtype=np.uint32)}, dict(
        tokens=tokens, heads=heads, head_dim=head_dim, theta=theta, f16=f16)


def rope_half_oracle(ora, inp, m):
    c, s = ora.rope_tables_llama(inp["pos"], m["head_dim"], m["theta"])
    fn = ora.rope_half_f16 if m["f16"] else ora.rope_half
    return [fn(inp["x"], c, s, m["tokens"], m["heads"], m["head_dim"], m["head_dim"] // 2)]


def rope_half_gpu(rt, inp, m, tables):
    c, s = tables
    x, cb, sb = rt.upload(inp["x"]), rt.upload(c), rt.upload(s)
    n = inp["x"].size
    o = rt.empty(n, inp["x"].dtype)
    (rt.rope_half_f16 if m["f16"] else rt.rope_half)(x, cb, sb, o, m["tokens"], m["heads"], m["head_dim"],
                                                     m["head_dim"] // 2)
    rt.sync()
    return [o.download(n, inp["x"].dtype)]


def f16_norm_case(rows, hidden, eps, seed):
    r = wl.rng(seed)
    h16 = lambda a: a.astype(np.float16).view(np.uint16)
    return {"x": h16(wl.normal(r, rows * hidden)), "res": h16(wl.normal(r, rows * hidden)),
            "w": h16(wl.normal(r, hidden, 1.0, 0.1))}, dict(rows=rows, hidden=hidden, eps=eps)


def f16_norm_oracle(ora, inp, m):
    rs, y = ora.add_rms_norm_f16(inp["x"], inp["res"], inp["w"], m["rows"], m["hidden"], m["eps"])
    return [rs, y, ora.rms_norm_f16(inp["x"], inp["w"], m["rows"], m["hidden"], m["eps"])]


def f16_norm_gpu(rt, inp, m):
    n = m["rows"] * m["hidden"]
    x, res, w = rt.upload(inp["x"]), rt.upload(inp["res"]), rt.upload(inp["w"])
    rs, y, y2 = rt.empty(n, np.uint16), rt.empty(n, np.uint16), rt.empty(n, np.uint16)
    rt.add_rms_norm_f16(x, res, w, rs, y, m["rows"], m["hidden"], m["eps"])
    rt.rms_norm_f16(x, w, y2, m["rows"], m["hidden"], m["eps"])
    rt.sync()
    return [rs.download(n), y.download(n), y2.download(n)]


def swiglu_f16_case(n, seed):
    r = wl.rng(seed)
    h16 = lambda a: a.astype(np.float16).view(np.uint16)
    return {"gate": h16(wl.normal(r, n)), "up": h16(wl.normal(r, n))}, dict(n=n)


def swiglu_f16_oracle(ora, inp, m):
    return [ora.swiglu_f16(inp["gate"], inp["up"])]


def swiglu_f16_gpu(rt, inp, m):
    g, u, o = rt.upload(inp["gate"]), rt.upload(inp["up"]), rt.empty(m["n"], np.uint16)
    rt.swiglu_f16(g, u, o, m["n"])
    rt.sync()
    return [o.download(m["n"])]


# ------------------------------------------------------- adversarial rows

def adversarial_rows(rows, hidden, seed):
    """Rows that stress the exact wave-parallel fold of the sum of squares:
    rounding ties, binade crossings, zeros, subnormal and overflowing squares,
    non-finite values, wide exponent ranges and a sum that grows through many
    binades."""
    r = np.random.default_rng(seed)
    x = r.standard_normal((rows, hidden)).astype(f32)
    for i in range(rows):
        kind = i % 16
        row = x[i]
        if kind == 1:
            row *= f32(1e-20)                                   # subnormal squares
        elif kind == 2:
            row *= f32(1e18)                                    # sum overflows to inf
        elif kind == 3:
            row[r.random(hidden) < 0.5] = 0.0                   # many zeros
        elif kind == 4:
            row[:] = np.trunc(row * 4) / 4                      # coarse values: many exact ties
        elif kind == 5:
            row[7] = np.inf
        elif kind == 6:
            row[hidden // 3] = np.nan
        elif kind == 7:
            row[:] = 1.0
        elif kind == 8:
            row[:] = (np.arange(hidden) % 7) * f32(0.5)
        elif kind == 9:
            row[:100] *= f32(1e-3)                              # slow start
        elif kind == 10:
            row[:] = np.ldexp(1.0 + r.random(hidden), r.integers(-20, 20, hidden)).astype(f32)
        elif kind == 11:
            row[:] = 0.0
        elif kind == 12:
            row[:] = np.sqrt(np.ldexp(1.0, r.integers(0, 8, hidden))).astype(f32)
        elif kind == 13:
            row *= f32(1e-6)
        elif kind == 14:
            row[:] = np.trunc(row * 64) / 64
        elif kind == 15:
            # squares growing geometrically 1 .. 2^16: the sum climbs past the
            # four binades the decode-batch fold scans ahead, mid-row
            row[:] = np.sqrt(np.exp2(np.arange(hidden) * (16.0 / hidden))).astype(f32)
    return x.reshape(-1)


def adversarial_f16_rows(rows, hidden, seed):
    """FP16 rows built to break a reordered or wave-parallel fold: squares of f16
    values have few significant bits, so exact rounding ties are frequent; plus
    binade crossings from tiny to large sums, subnormal and zero stretches,
    mixed magnitudes, and inf / NaN."""
    r = np.random.default_rng(seed)
    x = r.standard_normal((rows, hidden)).astype(np.float16)
    kind = np.arange(rows) % 7
    few = np.array([0.5, 1.0, 1.5, 2.0, 2.5, 3.0, 0.75, 1.25], np.float16)
    x[kind == 1] = r.choice(few, (int((kind == 1).sum()), hidden)) * r.choice([-1, 1], (int((kind == 1).sum()), hidden))
    x[kind == 2] = (r.standard_normal((int((kind == 2).sum()), hidden)) * 1e-6).astype(np.float16)   # subnormal f16
    big = kind == 3
    x[big] = (r.standard_normal((int(big.sum()), hidden)) * np.where(r.random((int(big.sum()), hidden)) < 0.1, 3e3, 1e-2)
              ).astype(np.float16)
    sparse = kind == 4
    x[sparse] = np.where(r.random((int(sparse.sum()), hidden)) < 0.05, x[sparse], np.float16(0))
    x[kind == 5, hidden // 3] = np.float16(np.inf)
    x[kind == 6, hidden // 2] = np.float16(np.nan)
    return x.reshape(-1).view(np.uint16)


# ------------------------------------------------------------ case registry
# Golden-fixture cases: BASELINE shapes where the oracle runs in well under a
# second (C1 exact, C2/C3 at their full sizes, C4 gathers with a reduced
# vocabulary for the fixture; the full-vocabulary gathers are GPU tests).

def golden_cases():
    S1, S2, S3 = wl.SmolShape(), wl.LlamaPrefillShape(), wl.GemmaLayerShape()
    return {
        "c1_rms_norm": (lambda: rms_case(S1.tokens, S1.hidden, S1.eps, 101), rms_oracle),
        "c1_swiglu": (lambda: glu_case(S1.tokens * S1.ffn, 102, "swiglu"), glu_oracle),
        "c1_rope_q": (lambda: rope_half_case(S1.tokens, S1.q_heads, S1.head_dim, S1.theta, 103), rope_half_oracle),
        "c1_rope_k": (lambda: rope_half_case(S1.tokens, S1.kv_heads, S1.head_dim, S1.theta, 104), rope_half_oracle),
        "c1_embed_f32": (lambda: embed_f32_case(S1.vocab, S1.hidden, S1.tokens, 0), embed_f32_oracle),
        "c2_add_rms_norm_f16": (lambda: f16_norm_case(S2.tokens, S2.hidden, S2.eps, 201), f16_norm_oracle),
        "c2_rope_f16": (lambda: rope_half_case(S2.tokens, S2.heads, S2.head_dim, S2.theta, 202, f16=True),
                        rope_half_oracle),
        "c2_swiglu_f16": (lambda: swiglu_f16_case(S2.tokens * S2.ffn, 203), swiglu_f16_oracle),
        "c3_rms_norm": (lambda: rms_case(S3.tokens, S3.hidden, S3.eps, 301), rms_oracle),
        "c3_rms_residual": (lambda: rms_case(S3.tokens, S3.hidden, S3.eps, 302, "residual"), rms_oracle),
        "c3_qk_norm_rope_local": (lambda: qk_case(S3.tokens, S3.q_heads, S3.head_dim, 128, S3.theta_local, S3.eps,
                                                  303), qk_oracle),
        "c3_qk_norm_rope_global": (lambda: qk_case(S3.tokens, S3.q_heads, S3.head_dim, 128, S3.theta_global,
                                                   S3.eps, 304), qk_oracle),
        "c3_geglu": (lambda: glu_case(S3.tokens * S3.ffn, 305, "geglu"), glu_oracle),
        "c4_embed_q4_0": (lambda: embed_q_case(8192, 1536, 4096, 401, False), embed_q_oracle),
        "c4_embed_q6_k": (lambda: embed_q_case(8192, 1536, 4096, 402, True), embed_q_oracle),
        "c4_ple_q4_0": (lambda: ple_case(2048, 35, 256, 512, 403, False), ple_oracle),
    }
