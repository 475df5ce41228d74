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


# ---------------------------------------------------------------- whole decode step

def small_step(eng, kind, n_layers, seed=0, activation=engine.ACT_SILU, hidden=256, ffn=384, fuse_norm=False):
    st, host, head = small_stack(eng, kind, n_layers, hidden=hidden, ffn=ffn, seed=seed)
    rng = np.random.default_rng(seed + 5)
    norm_w = [(1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32) for _ in range(2 * n_layers + 1)]
    bufs = [eng.to_device(w) for w in norm_w]
    norms = [stack.LayerNorms(bufs[2 * i], bufs[2 * i + 1]) for i in range(n_layers)]
    step = stack.DecodeStep(eng, st.layers, norms, bufs[-1], st.lm_head, st.lm_head, eps=1e-6,
                            activation=activation, fuse_norm=fuse_norm)
    return step, st, host, head, norm_w, bufs


def emulate_step(host, head, norm_w, token, gelu, eps=1e-6):
    """The same step on the CPU from oracle pieces, bf16 where the GPU keeps bf16."""
    from vxg_amd.formats import f32_to_bf16_bits
    r16 = lambda v: bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(v, np.float32)))
    cur = oracle.embed_rows(head, [token])[0]
    delta = None
    for i, (qkv, o, gu, dn) in enumerate(host):
        if delta is not None:
            cur = cur + delta
        x = r16(oracle.rms_norm(cur, norm_w[2 * i], eps))
        q = r16(np.concatenate([oracle.gemv(p, x, threads=THREADS) for p in qkv]))
        a = oracle.gemv(o, q[: o.cols], threads=THREADS)
        cur = cur + a
        x = r16(oracle.rms_norm(cur, norm_w[2 * i + 1], eps))
        act = r16(oracle.glu(oracle.gemv(gu[0], x, threads=THREADS), oracle.gemv(gu[1], x, threads=THREADS),
                             gelu))
        delta = oracle.gemv(dn, act, threads=THREADS)
    cur = cur + delta
    x = r16(oracle.rms_norm(cur, norm_w[-1], eps))
    return oracle.gemv(head, x, threads=THREADS)


@pytest.mark.parametrize("activation", [engine.ACT_SILU, engine.ACT_GELU_TANH])
def test_decode_step_matches_cpu_emulation(eng, activation):
    step, st, host, head, norm_w, bufs = small_step(eng, "cb4", 2, seed=3, activation=activation)
    step.set_token(123)
    step.enqueue()
    eng.synchronize()
    logits = step.logits.download(np.float32, head.rows)
    tok, nonfinite = step.read_token()
    assert (tok, nonfinite) == oracle.greedy(logits)
    want = emulate_step(host, head, norm_w, 123, activation == engine.ACT_GELU_TANH)
    # bf16 roundings at the projection inputs may land on different sides of
    # a tie between the two computations; the drift stays small.
    assert np.abs(logits - want).max() <= 2e-2 * np.abs(want).max()
    cos = float(np.dot(logits, want) / np.linalg.norm(logits) / np.linalg.norm(want))
    assert cos > 0.9999
    assert step.launches == 16
    step.free()
    st.free()
    for b in bufs:
        b.free()


def test_decode_step_graph_advances_tokens_like_eager(eng):
    step, st, host, head, norm_w, bufs = small_step(eng, "g64", 3, seed=11)
    step.set_token(7)
    eager = []
    for _ in range(4):
        step.enqueue()
        eng.synchronize()
        eager.append((step.read_token(), step.logits.download(np.float32, head.rows)))
    step.set_token(7)
    g = step.capture()
    try:
        for i in range(4):
            g.launch(1)
            assert step.read_token() == eager[i][0], i
            assert np.array_equal(step.logits.download(np.float32, head.rows), eager[i][1]), i
    finally:
        g.free()
    step.free()
    st.free()
    for b in bufs:
        b.free()


@pytest.mark.parametrize("kind", ["cb4", "g64"])
def test_decode_step_fused_norms_bit_identical(eng, kind):
    """Norms built inside the projections: same tokens, logits and residual
    stream as the separate RMSNorm launches, eager and captured."""
    runs = []
    for fuse in (False, True):
        step, st, host, head, norm_w, bufs = small_step(eng, kind, 3, seed=21,
                                                        activation=engine.ACT_GELU_TANH, fuse_norm=fuse)
        assert step.launches == (16 if fuse else 22)
        step.set_token(99)
        seq = []
        for _ in range(3):
            step.enqueue()
            eng.synchronize()
            seq.append((step.read_token(), step.logits.download(np.float32, head.rows),
                        step.residual.download(np.float32, (step.hidden,))))
        step.set_token(99)
        g = step.capture()
        for i in range(3):
            g.launch(1)
            assert step.read_token() == seq[i][0]
            assert np.array_equal(step.logits.download(np.float32, head.rows), seq[i][1])
        g.free()
        runs.append(seq)
        step.free()
        st.free()
        for b in bufs:
            b.free()
    for (ta, la, ca), (tb, lb, cb) in zip(*runs):
        assert ta == tb
        assert np.array_equal(la, lb)
        assert np.array_equal(ca, cb)


def test_decode_step_shape_checks(eng):
    st, host, head = small_stack(eng, "g64", 1)
    w = eng.to_device(np.ones(256, np.float32))
    with pytest.raises(ValueError):
        stack.DecodeStep(eng, st.layers, [], w, st.lm_head, st.lm_head)
    other = eng.upload_packed(synth.make_q8(10, 128, seed=1))
    with pytest.raises(ValueError):
        stack.DecodeStep(eng, st.layers, [stack.LayerNorms(w, w)], w, st.lm_head, other)
    other.free()
    w.free()
    st.free()
