"""GPU parity of row-concatenated tensors and of the decode-step linear stack.

Concatenation follows the reference's device packer: up to three codebook
parts, each with its own centroid table, share one arena with rebased CSR
row pointers (metal_cb4_fast_ffi.rs:89-104, metal_cb4_fast.mm:140-171).  The
expected values are the oracle's on each part separately.
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine, stack, synth
from vxg_amd.formats import bf16_bits_to_f32
from parity_util import (THREADS, assert_bf16_close, assert_bits_equal, floor_scale, gemv_ref,
                         make, max_rel, run_dev)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


def cb4_parts(rows, cols, seed):
    """Parts with distinct centroid tables and outlier streams."""
    return [synth.make_cb4(r, cols, seed=seed + i, outlier_frac=0.02) for i, r in enumerate(rows)]


def stacked_ref(parts, fn):
    return np.concatenate([fn(p) for p in parts], axis=-1)


@pytest.mark.parametrize("rows", [(5,), (3, 9), (2, 17, 7), (64, 64, 64)])
@pytest.mark.parametrize("cols", [129, 544])
def test_cb4_concat_dequant_bit_exact(eng, rows, cols):
    parts = cb4_parts(rows, cols, seed=sum(rows) + cols)
    t = eng.upload_concat(parts)
    assert t.rows == sum(rows)
    got = eng.dequant_rows(t)
    assert_bits_equal(got, np.concatenate([oracle.decode_rows(p) for p in parts]))
    # a window straddling the first part boundary
    if len(rows) > 1:
        r0 = rows[0] - 1
        assert_bits_equal(eng.dequant_rows(t, r0, 2), got[r0:r0 + 2])


@pytest.mark.parametrize("M", [1, 3, 8])
def test_cb4_concat_gemv(eng, M):
    parts = cb4_parts((6, 33, 70), 544, seed=M)
    t = eng.upload_concat(parts)
    xb = synth.make_x_bf16(M, 544, seed=M)
    X = bf16_bits_to_f32(xb)
    y = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    yref = stacked_ref(parts, lambda p: gemv_ref(p, X))
    W = np.concatenate([oracle.decode_rows(p) for p in parts])
    assert max_rel(y, yref, floor_scale(W, X)) <= 1e-3


def test_cb4_concat_gemm(eng):
    parts = cb4_parts((40, 100), 300, seed=5)
    t = eng.upload_concat(parts)
    xb = synth.make_x_bf16(37, 300, seed=5)
    X = bf16_bits_to_f32(xb)
    yb = run_dev(eng, t, xb, engine.DTYPE_BF16, 37, engine.DTYPE_BF16)
    yref = stacked_ref(parts, lambda p: oracle.gemm(p, X, threads=THREADS))
    W = np.concatenate([oracle.decode_rows(p) for p in parts])
    assert_bf16_close(yb, yref, floor_scale(W, X))


@pytest.mark.parametrize("kind", ["g64", "q8"])
def test_stacked_g64_q8(eng, kind):
    parts = [make(kind, r, 320, seed=r) for r in (11, 64, 5)]
    t = eng.upload_concat(parts)
    x = synth.make_x_f32(2, 320, seed=1)
    y = run_dev(eng, t, x, engine.DTYPE_F32, 2, engine.DTYPE_F32)
    W = np.concatenate([oracle.decode_rows(p) for p in parts])
    assert max_rel(y, stacked_ref(parts, lambda p: gemv_ref(p, x)), floor_scale(W, x)) <= 1e-3
    assert_bits_equal(eng.dequant_rows(t), W)


def test_concat_errors(eng):
    p = synth.make_cb4(4, 256, seed=1)
    with pytest.raises(engine.BackendError) as ei:
        eng.upload_concat([p, p, p, p])
    assert ei.value.code == engine.VXT_E_ARG
    with pytest.raises(engine.BackendError) as ei:
        eng.upload_concat([p, synth.make_cb4(4, 128, seed=2)])
    assert ei.value.code == engine.VXT_E_SHAPE
    with pytest.raises(engine.BackendError):
        eng.upload_concat([p, synth.make_q8(4, 256)])


# ---------------------------------------------------------------- decode stack

def small_stack(eng, kind, n_layers, hidden=256, ffn=384, vocab=1000, seed=0):
    """Layers of [q;k;v], o, [gate;up], down (cb4 parts concatenated on upload)."""
    gen = {"cb4": lambda r, c, s: synth.make_cb4(r, c, seed=s, outlier_frac=0.01),
           "g64": lambda r, c, s: synth.make_g64(r, c, seed=s)}[kind]
    host, layers = [], []
    for li in range(n_layers):
        s = seed + 10 * li
        qkv = [gen(hidden, hidden, s), gen(hidden, hidden, s + 1), gen(hidden, hidden, s + 2)]
        o = gen(hidden, hidden, s + 3)
        gu = [gen(ffn, hidden, s + 4), gen(ffn, hidden, s + 5)]
        dn = gen(hidden, ffn, s + 6)
        host.append((qkv, o, gu, dn))
        layers.append(stack.LayerWeights(eng.upload_concat(qkv), eng.upload_packed(o),
                                         eng.upload_concat(gu), eng.upload_packed(dn)))
    head = synth.make_q8(vocab, hidden, seed=seed + 999)
    st = stack.DecodeStack(eng, layers, eng.upload_packed(head))
    return st, host, head


def test_stack_one_layer_stages(eng):
    """Each projection of a layer against the oracle on the GPU's own inputs."""
    st, host, head = small_stack(eng, "cb4", 1)
    (qkv, o, gu, dn), = host
    xb = synth.make_x_bf16(1, st.hidden, seed=3)[0]
    st.set_input(xb)
    st.enqueue()
    eng.synchronize()

    def check(parts, x_bits, y_bits):
        x = bf16_bits_to_f32(x_bits)
        yref = np.concatenate([oracle.gemv(p, x, threads=THREADS) for p in parts])
        W = np.concatenate([oracle.decode_rows(p) for p in parts])
        assert_bf16_close(y_bits, yref, floor_scale(W, x[None])[0])

    qkv_y = st.qkv_out.download(np.uint16, 3 * st.hidden)
    check(qkv, xb, qkv_y)
    o_y = st.o_out.download(np.uint16, st.hidden)
    check([o], qkv_y[: o.cols], o_y)
    gu_y = st.gu_out.download(np.uint16, 2 * 384)
    check(gu, o_y, gu_y)
    dn_y = st.dn_out.download(np.uint16, st.hidden)
    check([dn], gu_y[: dn.cols], dn_y)
    logits = st.logits.download(np.float32, head.rows)
    x = bf16_bits_to_f32(dn_y)
    assert max_rel(logits, oracle.gemv(head, x, threads=THREADS),
                   floor_scale(oracle.decode_rows(head), x[None])[0]) <= 1e-3
    assert st.launches == 5


@pytest.mark.parametrize("kind", ["cb4", "g64"])
def test_stack_graph_replays_match_eager(eng, kind):
    """One token captured as a graph, replayed several times with eager work between."""
    st, _, head = small_stack(eng, kind, 3, seed=7)
    st.set_input(synth.make_x_bf16(1, st.hidden, seed=4)[0])
    st.enqueue()
    eng.synchronize()
    ref = st.logits.download(np.float32, head.rows)
    assert np.all(np.isfinite(ref))
    g = st.capture()
    for i in range(3):
        st.logits.upload(np.full(head.rows, np.nan, np.float32))
        g.launch(1 + i)
        assert np.array_equal(st.logits.download(np.float32, head.rows), ref), i
        st.enqueue()              # eager work between replays
        eng.synchronize()
    g.free()
    st.free()


def test_stack_shape_checks(eng):
    a = eng.upload_packed(synth.make_g64(64, 64, seed=1))
    b = eng.upload_packed(synth.make_g64(64, 128, seed=1))
    with pytest.raises(ValueError):
        stack.DecodeStack(eng, [stack.LayerWeights(a, a, a, b)], a)
    with pytest.raises(ValueError):
        stack.DecodeStack(eng, [], a)
