"""GPU test of the GGUF path end to end: a Gemma-4-E2B-shaped file is written,
opened with the product reader (memory-mapped), its packed tables are
uploaded unconverted and read by the device ops, and every result is checked
against the oracle computed from the same file bytes.

Tensor names and layouts follow the reference model (token_embd.weight Q6_K
and per_layer_token_embd.weight Q4_0 as [vocab, row] tables, GGUF dims in
contiguous-first order; crates/atlas-model/src/gemma4_executor.rs:174-194,
1720-1738; crates/atlas-core/tests/phase_11a_gguf.rs:169,211).  The vocabulary
is cut to 4096 rows to keep the file small; rows are independent.
"""
import sys

import numpy as np
import pytest

import gguf_oracle as go
import matvec_cases as mc
from atlas_amd import workloads as wl
from atlas_amd.gguf import F32, Q4_0, Q6_K, GgufModel

pytestmark = pytest.mark.gpu
f32 = np.float32
VOCAB, HIDDEN, LAYERS, PLE_W, QN = 4096, 1536, 35, 256, 2048


def say(msg):
    print(f"[gpu-gguf] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def gemma_file(tmp_path_factory):
    r = wl.rng(606)
    tables = {
        "token_embd.weight": ([HIDDEN, VOCAB], Q6_K, wl.q6_k_table(r, VOCAB, HIDDEN)),
        "per_layer_token_embd.weight": ([LAYERS * PLE_W, VOCAB], Q4_0, wl.q4_0_table(r, VOCAB, LAYERS * PLE_W)),
        "blk.0.attn_q.weight": ([HIDDEN, QN], Q4_0, mc.random_q4_0(r, QN, HIDDEN)),
        "blk.0.attn_norm.weight": ([HIDDEN], F32, wl.normal(r, HIDDEN, 1.0, 0.1)),
    }
    w = go.Writer()
    w.meta("general.architecture", "gemma4")
    w.meta("gemma4.embedding_length", str(HIDDEN))
    for name, (dims, ttype, data) in tables.items():
        w.push_tensor(name, dims, ttype, np.ascontiguousarray(data).tobytes())
    path = tmp_path_factory.mktemp("gguf") / "gemma4-e2b-like.gguf"
    path.write_bytes(w.finish())
    return path, tables


def test_gguf_tables_feed_the_device_ops(rt, ora, gemma_file):
    path, tables = gemma_file
    say(f"open {path.name}")
    m = GgufModel.open(path)
    assert m.metadata["general.architecture"] == "gemma4"
    for name, (dims, ttype, data) in tables.items():
        t = m.tensor(name)
        assert t.dims == tuple(dims) and t.tensor_type == ttype
        assert bytes(m.tensor_data(t)) == np.ascontiguousarray(data).tobytes()
    r = wl.rng(7)
    T = 64
    ids = wl.token_ids(r, T, VOCAB)
    d_ids = rt.upload(ids)
    scale = float(wl.f32_sqrt(HIDDEN))

    say("token embedding Q6_K straight from the file")
    emb = m.tensor("token_embd.weight")
    d_emb = m.upload(rt, emb)
    assert np.array_equal(d_emb.download(emb.bytes, np.uint8), m.tensor_data(emb))
    out = rt.empty(T * HIDDEN)
    rt.embed_q6_k(d_emb, d_ids, out, VOCAB, HIDDEN, T, scale)
    rt.sync()
    exp = ora.embed_q6_k(np.asarray(m.tensor_data(emb)), ids, VOCAB, HIDDEN, scale)
    assert np.array_equal(out.download(T * HIDDEN).view(np.uint32), exp.view(np.uint32))

    say("PLE Q4_0 straight from the file")
    ple = m.tensor("per_layer_token_embd.weight")
    d_ple = m.upload(rt, ple)
    proj = wl.normal(r, (T, LAYERS, PLE_W))
    pout = rt.empty(T * LAYERS * PLE_W)
    rt.ple_q4_0(d_ple, d_ids, rt.upload(proj), pout, VOCAB, LAYERS, PLE_W, T, 16.0, float(wl.SQRT_2_RECIP))
    rt.sync()
    pexp = ora.ple(np.asarray(m.tensor_data(ple)), ids, proj, VOCAB, LAYERS, PLE_W, f32(16.0), wl.SQRT_2_RECIP)
    assert np.array_equal(pout.download(T * LAYERS * PLE_W).view(np.uint32), pexp.view(np.uint32))

    say("RMS-folded Q4_0 projection with the file's norm weight")
    q = m.tensor("blk.0.attn_q.weight")
    nw = m.tensor("blk.0.attn_norm.weight")
    d_q, d_nw = m.upload(rt, q), m.upload(rt, nw)
    x = wl.normal(r, HIDDEN)
    qout = rt.empty(QN)
    rt.matvec_q4_0_rms(rt.upload(x), d_q, qout, HIDDEN, QN, d_nw, 1e-6)
    rt.sync()
    norm_w = np.asarray(m.tensor_data(nw)).view(f32)
    exact, mag = ora.matvec_q4_0_rms_f64(x, np.asarray(m.tensor_data(q)), norm_w, HIDDEN, QN, 1e-6)
    err = np.abs(qout.download(QN).astype(np.float64) - exact)
    assert np.all(err <= 1e-5 * mag)
    m.close()
