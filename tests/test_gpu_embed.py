"""GPU parity of the device-token embedding gather (``vxt_hip_embed_dev``).

Expected values: ``oracle.embed_rows`` (decode_row then the embed_scale rule
of llm_cpu.rs:224-229), compared bit for bit.  The matrices include the
closed-form cb4 matrix of the reference's embedding probe
(metal_llm_tests.rs:31-58, rows 515, cols 1/129/257/385) and random cb4,
g64 and Q8 matrices.  Ids past the last row read the last row, as the
device runner's gather does (vxt_cb4_fast_ops.metal:107).
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine, synth
from parity_util import assert_bits_equal, closed_form, f16b, make

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


def run_embed(eng, t, tokens, stride=None, scale=1.0, fill=np.nan):
    tokens = np.asarray(tokens, np.uint32)
    stride = t.cols if stride is None else stride
    td = eng.to_device(tokens) if tokens.size else None
    out = eng.to_device(np.full((max(tokens.size, 1), stride), fill, np.float32))
    try:
        eng.embed_dev(t, td.ptr if td else 0, tokens.size, out.ptr, stride, scale, eng.stream)
        eng.synchronize()
        return out.download(np.float32, (tokens.size, stride))
    finally:
        out.free()
        if td:
            td.free()


@pytest.mark.parametrize("cols", [1, 129, 257, 385])
def test_reference_probe_matrix(eng, cols):
    m = closed_form(515, cols, lambda c: [(f16b(v) << 16) | (c - 1)
                                          for v in (0.33325195, -0.125, 0.0009765625)])
    t = eng.upload_packed(m)
    toks = [0, 1, 514]
    assert_bits_equal(run_embed(eng, t, toks), oracle.embed_rows(m, toks))
    t.free()


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("cols", [64, 300, 2048])
def test_kinds_batches_and_padding(eng, kind, cols):
    m = make(kind, 257, cols, seed=cols + 3)
    t = eng.upload_packed(m)
    toks = np.random.default_rng(cols).integers(0, m.rows, 37).astype(np.uint32)
    toks[:3] = [0, m.rows - 1, 5]
    got = run_embed(eng, t, toks, stride=cols + 70)
    assert_bits_equal(got[:, :cols], oracle.embed_rows(m, toks))
    assert np.array_equal(got[:, cols:], np.zeros((toks.size, 70), np.float32))
    t.free()


@pytest.mark.parametrize("scale", [1.0, 2.0, float(np.float32(np.sqrt(2048.0))),
                                   float(np.float32(1.0) - np.float32(2.0 ** -24)),
                                   float(np.float32(1.0) + np.float32(2.0 ** -23)), -0.5])
def test_embed_scale_rule(eng, scale):
    m = synth.make_cb4(99, 2048, seed=8, outlier_frac=0.03)
    t = eng.upload_packed(m)
    toks = [3, 98, 0, 50]
    assert_bits_equal(run_embed(eng, t, toks, scale=scale), oracle.embed_rows(m, toks, scale))
    t.free()


def test_concatenated_parts(eng):
    parts = [synth.make_cb4(r, 384, seed=20 + i, outlier_frac=0.02) for i, r in enumerate((5, 9, 3))]
    t = eng.upload_concat(parts)
    toks = [0, 4, 5, 13, 14, 16]
    want = np.concatenate([oracle.decode_rows(p) for p in parts])[toks]
    assert_bits_equal(run_embed(eng, t, toks), want)
    t.free()


def test_out_of_range_ids_read_the_last_row(eng):
    m = make("cb4", 50, 200, seed=1)
    t = eng.upload_packed(m)
    got = run_embed(eng, t, [50, 0xFFFFFFFF, 49])
    last = oracle.embed_rows(m, [49])[0]
    for r in got:
        assert_bits_equal(r, last)
    t.free()


def test_greedy_feeds_embedding_on_device(eng):
    """The device-resident token step: logits -> greedy id -> embedding row,
    with the id never leaving the GPU; also inside a captured graph."""
    m = make("cb4", 151_936, 64, seed=2)
    t = eng.upload_packed(m)
    n = m.rows
    logits, ids, row = eng.alloc(n * 4), eng.alloc(8), eng.alloc(64 * 4)

    def step(s):
        eng.greedy_dev(logits.ptr, n, ids.ptr, s)
        eng.embed_dev(t, ids.ptr, 1, row.ptr, 64, 1.0, s)

    try:
        g = eng.capture(step)
        try:
            for seed in range(3):
                a = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
                logits.upload(a)
                want_id, _ = oracle.greedy(a)
                if seed == 1:
                    step(eng.stream)
                    eng.synchronize()
                else:
                    g.launch(1)
                assert int(ids.download(np.uint32, (2,))[0]) == want_id
                assert_bits_equal(row.download(np.float32, (64,)), oracle.embed_rows(m, [want_id])[0])
        finally:
            g.free()
    finally:
        for b in (logits, ids, row):
            b.free()
        t.free()


def test_argument_errors(eng):
    m = make("q8", 8, 64, seed=0)
    t = eng.upload_packed(m)
    buf = eng.alloc(4096)
    try:
        run_embed(eng, t, [])                                   # batch 0 is a no-op
        for kw, code in [(dict(out_stride=63), engine.VXT_E_SHAPE),
                         (dict(embed_scale=float("inf")), engine.VXT_E_ARG),
                         (dict(embed_scale=float("nan")), engine.VXT_E_ARG)]:
            with pytest.raises(engine.BackendError) as e:
                eng.embed_dev(t, buf.ptr, 1, buf.ptr + 256, stream=eng.stream, **kw)
            assert e.value.code == code
        with pytest.raises(engine.BackendError) as e:
            eng.embed_dev(t, 0, 1, buf.ptr, stream=eng.stream)
        assert e.value.code == engine.VXT_E_ARG
    finally:
        buf.free()
        t.free()
