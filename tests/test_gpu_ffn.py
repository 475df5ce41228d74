"""GPU parity of the gated FFN projection and the residual-add + RMSNorm.

Gated FFN (``vxt_hip_ffn_glu_dev``): the tensor is ``[gate; up]``; the
expected activation is the oracle's ``glu`` (llm_cpu.rs:457-464) of the
oracle's GEMVs.  The bar propagates the GEMV bar (relative error 1e-3 of
max(|y|, 2^-10 sum|w x|)) through act(g) * u:
    |act - act_ref| <= 1e-3 (|act'(g) u| F_g + |act(g)| F_u).
A second check isolates the epilogue: the GPU's own plain GEMV of the same
tensor gives g and u with the same summation, and act must equal the
oracle's glu of those up to expf's last bits: 8 ulp for silu; for gelu_tanh
also 0.5 |g u| 2^-21, since 1 + tanh cancels for negative g and turns an
ulp of exp into many ulps of the result.

RMSNorm (``vxt_hip_rms_norm_dev``): the residual add is exact (bit-equal to
numpy's f32 add); the normalised output is within 2e-6 relative of the
oracle's rms_norm (llm_ops.rs:48-57) of the updated row -- the sum of
squares runs in a different order -- and bf16 outputs within 1 bf16 ulp.
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine, synth
from vxg_amd.formats import bf16_bits_to_f32, f32_to_bf16_bits
from parity_util import THREADS, floor_scale, make

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


def upload_gate_up(eng, kind, n_ff, cols, seed):
    gate, up = make(kind, n_ff, cols, seed), make(kind, n_ff, cols, seed + 1000)
    return gate, up, eng.upload_concat([gate, up])


def act_prime(g, gelu):
    g = g.astype(np.float64)
    if gelu:
        z = 0.7978846 * (g + 0.044715 * g ** 3)
        t = np.tanh(z)
        return 0.5 * (1 + t) + 0.5 * g * (1 - t * t) * 0.7978846 * (1 + 3 * 0.044715 * g * g)
    s = 1 / (1 + np.exp(-g))
    return s * (1 + g * (1 - s))


def ulp_dist(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, np.int64(-2**31) - a, a)
    b = np.where(b < 0, np.int64(-2**31) - b, b)
    return np.abs(a - b)


def run_glu(eng, t, X, x_dtype, act_dtype, act_stride, activation):
    M = X.shape[0]
    xh = f32_to_bf16_bits(X) if x_dtype == engine.DTYPE_BF16 else X
    esz = 2 if act_dtype == engine.DTYPE_BF16 else 4
    xd, ad = eng.to_device(xh), eng.alloc(M * act_stride * esz)
    try:
        ad.upload(np.full(M * act_stride * esz, 0x7F, np.uint8))      # garbage in the padding
        eng.ffn_glu_dev(t, xd.ptr, x_dtype, M, ad.ptr, act_dtype, act_stride, activation, eng.stream)
        eng.synchronize()
        if act_dtype == engine.DTYPE_BF16:
            return bf16_bits_to_f32(ad.download(np.uint16, (M, act_stride)))
        return ad.download(np.float32, (M, act_stride))
    finally:
        xd.free()
        ad.free()


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("M", [1, 2, 3, 8, 16])
@pytest.mark.parametrize("shape", [(77, 300), (6144, 2048)])
def test_gated_ffn_parity(eng, kind, M, shape):
    n_ff, cols = shape
    print(f"glu kind={kind} M={M} n_ff={n_ff} cols={cols}", flush=True)
    gate, up, t = upload_gate_up(eng, kind, n_ff, cols, seed=n_ff + M)
    rng = np.random.default_rng(M + cols)
    X = rng.standard_normal((M, cols)).astype(np.float32)
    Xq = bf16_bits_to_f32(f32_to_bf16_bits(X))
    for activation in (engine.ACT_SILU, engine.ACT_GELU_TANH):
        gelu = activation == engine.ACT_GELU_TANH
        got = run_glu(eng, t, X, engine.DTYPE_BF16, engine.DTYPE_F32, n_ff + 13, activation)
        assert np.all(got[:, n_ff:] == 0)
        g = np.stack([oracle.gemv(gate, Xq[m], threads=THREADS) for m in range(M)])
        u = np.stack([oracle.gemv(up, Xq[m], threads=THREADS) for m in range(M)])
        want = np.stack([oracle.glu(g[m], u[m], gelu) for m in range(M)])
        Wg, Wu = oracle.decode_rows(gate), oracle.decode_rows(up)
        Fg = np.maximum(np.abs(g), floor_scale(Wg, Xq))
        Fu = np.maximum(np.abs(u), floor_scale(Wu, Xq))
        sg = np.abs(want.astype(np.float64)) / np.maximum(np.abs(u.astype(np.float64)), 1e-30)
        bound = 1e-3 * (np.abs(act_prime(g, gelu) * u) * Fg + sg * Fu) + 1e-30
        err = np.abs(got[:, :n_ff].astype(np.float64) - want)
        assert np.all(err <= bound), (activation, float((err / bound).max()))
    t.free()


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("M", [1, 2, 5])
def test_gated_epilogue_matches_plain_gemv(eng, kind, M):
    """Same sums as the plain GEMV of [gate; up]; only the activation's expf
    differs.  (Q8 with bf16 x at M = 2 takes the packed-dot kernel for the
    plain GEMV, whose sums run in another order, so that case feeds f32 x.)"""
    n_ff, cols = 1536, 2048
    _, _, t = upload_gate_up(eng, kind, n_ff, cols, seed=7 + M)
    X = np.random.default_rng(M).standard_normal((M, cols)).astype(np.float32)
    xdt = engine.DTYPE_F32 if (kind == "q8" and M == 2) else engine.DTYPE_BF16
    xd = eng.to_device(X if xdt == engine.DTYPE_F32 else f32_to_bf16_bits(X))
    yd = eng.alloc(M * 2 * n_ff * 4)
    try:
        eng.matmul_dev(t, xd.ptr, xdt, M, yd.ptr, engine.DTYPE_F32, eng.stream)
        eng.synchronize()
        gu = yd.download(np.float32, (M, 2 * n_ff))
    finally:
        xd.free()
        yd.free()
    for activation in (engine.ACT_SILU, engine.ACT_GELU_TANH):
        got = run_glu(eng, t, X, xdt, engine.DTYPE_F32, n_ff, activation)
        want = np.stack([oracle.glu(gu[m, :n_ff], gu[m, n_ff:], activation == engine.ACT_GELU_TANH)
                         for m in range(M)])
        if activation == engine.ACT_SILU:
            assert ulp_dist(got, want).max() <= 8
        else:
            slack = 0.5 * np.abs(gu[:, :n_ff].astype(np.float64) * gu[:, n_ff:]) * 2.0 ** -21
            ok = (ulp_dist(got, want) <= 8) | (np.abs(got.astype(np.float64) - want) <= slack)
            assert ok.all()
    t.free()


def test_gated_ffn_f32_x_and_bf16_act(eng):
    n_ff, cols = 300, 544
    gate, up, t = upload_gate_up(eng, "cb4", n_ff, cols, seed=3)
    X = np.random.default_rng(9).standard_normal((2, cols)).astype(np.float32)
    f32 = run_glu(eng, t, X, engine.DTYPE_F32, engine.DTYPE_F32, n_ff, engine.ACT_SILU)
    b16 = run_glu(eng, t, X, engine.DTYPE_F32, engine.DTYPE_BF16, n_ff + 5, engine.ACT_SILU)
    assert np.array_equal(b16[:, :n_ff], bf16_bits_to_f32(f32_to_bf16_bits(f32)))
    assert np.all(b16[:, n_ff:] == 0)
    g = np.stack([oracle.gemv(gate, X[m], threads=THREADS) for m in range(2)])
    u = np.stack([oracle.gemv(up, X[m], threads=THREADS) for m in range(2)])
    want = np.stack([oracle.glu(g[m], u[m]) for m in range(2)])
    assert np.allclose(f32, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())
    t.free()


def test_gated_ffn_errors(eng):
    odd = eng.upload_packed(make("q8", 5, 64, seed=0))
    even = eng.upload_packed(make("q8", 6, 64, seed=0))
    buf = eng.alloc(4096)
    try:
        cases = [(odd, dict(), engine.VXT_E_SHAPE),
                 (even, dict(act_stride=2), engine.VXT_E_SHAPE),
                 (even, dict(activation=7), engine.VXT_E_ARG)]
        for t, kw, code in cases:
            with pytest.raises(engine.BackendError) as e:
                eng.ffn_glu_dev(t, buf.ptr, engine.DTYPE_F32, 1, buf.ptr + 1024, engine.DTYPE_F32,
                                stream=eng.stream, **kw)
            assert e.value.code == code
    finally:
        buf.free()
        odd.free()
        even.free()


# ---------------------------------------------------------------- RMSNorm

def run_norm(eng, cur, delta, w, eps, stride, out_dtype, inplace=False):
    M = cur.shape[0]
    dim = w.size
    cd = eng.to_device(cur)
    dd = eng.to_device(delta) if delta is not None else None
    wd = eng.to_device(w)
    esz = 2 if out_dtype == engine.DTYPE_BF16 else 4
    od = None if inplace else eng.to_device(np.full(M * stride * esz, 0x7F, np.uint8))
    try:
        eng.rms_norm_dev(cd.ptr, dd.ptr if dd else 0, wd.ptr, cd.ptr if inplace else od.ptr, out_dtype,
                         dim, stride, M, eps, eng.stream)
        eng.synchronize()
        new_cur = cd.download(np.float32, (M, stride))
        if inplace:
            out = new_cur
        elif out_dtype == engine.DTYPE_BF16:
            out = bf16_bits_to_f32(od.download(np.uint16, (M, stride)))
        else:
            out = od.download(np.float32, (M, stride))
        return new_cur, out
    finally:
        for b in (cd, dd, wd, od):
            if b is not None:
                b.free()


@pytest.mark.parametrize("dim,stride", [(1, 1), (77, 80), (2048, 2048), (4099, 4352), (6144, 6144)])
@pytest.mark.parametrize("with_delta", [False, True])
def test_rms_norm_parity(eng, dim, stride, with_delta):
    rng = np.random.default_rng(dim)
    M = 3
    cur = np.zeros((M, stride), np.float32)
    cur[:, :dim] = rng.standard_normal((M, dim)).astype(np.float32) * 2
    delta = None
    if with_delta:
        delta = np.zeros((M, stride), np.float32)
        delta[:, :dim] = rng.standard_normal((M, dim)).astype(np.float32)
    w = (rng.standard_normal(dim) * 0.5 + 1).astype(np.float32)
    eps = 1e-6
    new_cur, out = run_norm(eng, cur, delta, w, eps, stride, engine.DTYPE_F32)
    ref_cur = cur + delta if with_delta else cur
    assert np.array_equal(new_cur[:, :dim], ref_cur[:, :dim])
    for m in range(M):
        ref = oracle.rms_norm(ref_cur[m, :dim], w, eps)
        assert np.all(np.abs(out[m, :dim] - ref) <= 2e-6 * np.abs(ref) + 1e-30)
    assert np.all(out[:, dim:] == 0)
    _, outb = run_norm(eng, cur, delta, w, eps, stride, engine.DTYPE_BF16)
    for m in range(M):
        ref = oracle.rms_norm(ref_cur[m, :dim], w, eps)
        lo = np.minimum(ref * (1 - 2e-6), ref * (1 + 2e-6))
        hi = np.maximum(ref * (1 - 2e-6), ref * (1 + 2e-6))
        cand = {tuple(bf16_bits_to_f32(f32_to_bf16_bits(v))) for v in (lo, hi)}
        ok = np.zeros(dim, bool)
        for c in cand:
            ok |= np.asarray(c, np.float32) == outb[m, :dim]
        assert ok.all()
    assert np.all(outb[:, dim:] == 0)


def test_rms_norm_in_place_and_eps(eng):
    rng = np.random.default_rng(2)
    cur = rng.standard_normal((2, 512)).astype(np.float32) * 1e-3
    w = np.ones(512, np.float32)
    for eps in (1e-6, 1e-5, 0.5):
        _, out = run_norm(eng, cur.copy(), None, w, eps, 512, engine.DTYPE_F32, inplace=True)
        for m in range(2):
            ref = oracle.rms_norm(cur[m], w, eps)
            assert np.all(np.abs(out[m] - ref) <= 2e-6 * np.abs(ref) + 1e-30)


def test_rms_norm_errors(eng):
    buf = eng.alloc(8192)
    try:
        p = buf.ptr
        cases = [(dict(cur_ptr=p, delta_ptr=0, weight_ptr=p + 4096, out_ptr=p + 2048, out_dtype=0, dim=0),
                  engine.VXT_E_SHAPE),
                 (dict(cur_ptr=p, delta_ptr=0, weight_ptr=p + 4096, out_ptr=p + 2048, out_dtype=0, dim=8,
                       stride=4), engine.VXT_E_SHAPE),
                 (dict(cur_ptr=p, delta_ptr=0, weight_ptr=p + 4096, out_ptr=p, out_dtype=1, dim=8),
                  engine.VXT_E_ARG),
                 (dict(cur_ptr=p, delta_ptr=p + 1024, weight_ptr=p + 4096, out_ptr=p + 1024, out_dtype=0,
                       dim=8), engine.VXT_E_ARG),
                 (dict(cur_ptr=0, delta_ptr=0, weight_ptr=p + 4096, out_ptr=p, out_dtype=0, dim=8),
                  engine.VXT_E_ARG)]
        for kw, code in cases:
            with pytest.raises(engine.BackendError) as e:
                eng.rms_norm_dev(stream=eng.stream, **kw)
            assert e.value.code == code
    finally:
        buf.free()


# ---------------------------------------------------------------- norm prologue

def norm_pair_reference(eng, t, cur, delta, w, eps, mode, y_dtype, y_stride):
    """The two-launch form on the GPU: vxt_hip_rms_norm_dev (bf16 out) then the
    projection reading it."""
    H = cur.size
    cd, wd = eng.to_device(cur), eng.to_device(w)
    dd = eng.to_device(delta) if delta is not None else None
    xd = eng.alloc(H * 2)
    esz = 2 if y_dtype == engine.DTYPE_BF16 else 4
    outs = t.rows if mode == engine.NORM_PLAIN else y_stride
    yd = eng.alloc(outs * esz)
    try:
        eng.rms_norm_dev(cd.ptr, dd.ptr if dd else 0, wd.ptr, xd.ptr, engine.DTYPE_BF16, H, H, 1, eps, eng.stream)
        if mode == engine.NORM_PLAIN:
            eng.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 1, yd.ptr, y_dtype, eng.stream)
        else:
            act = engine.ACT_GELU_TANH if mode == engine.NORM_GLU_GELU_TANH else engine.ACT_SILU
            eng.ffn_glu_dev(t, xd.ptr, engine.DTYPE_BF16, 1, yd.ptr, y_dtype, y_stride, act, eng.stream)
        eng.synchronize()
        return cd.download(np.float32, (H,)), yd.download(np.uint16 if esz == 2 else np.uint32, (outs,))
    finally:
        for b in (cd, wd, dd, xd, yd):
            if b is not None:
                b.free()


def run_norm_matmul(eng, t, cur, delta, w, eps, mode, y_dtype, y_stride):
    H = cur.size
    cd, wd = eng.to_device(cur), eng.to_device(w)
    dd = eng.to_device(delta) if delta is not None else None
    od = eng.to_device(np.full(H, np.nan, np.float32))
    esz = 2 if y_dtype == engine.DTYPE_BF16 else 4
    outs = t.rows if mode == engine.NORM_PLAIN else y_stride
    yd = eng.to_device(np.full(outs * esz, 0x7F, np.uint8))
    try:
        eng.norm_matmul_dev(t, cd.ptr, dd.ptr if dd else 0, wd.ptr, eps, od.ptr if dd else 0, mode, yd.ptr,
                            y_dtype, y_stride, eng.stream)
        eng.synchronize()
        return od.download(np.float32, (H,)), yd.download(np.uint16 if esz == 2 else np.uint32, (outs,))
    finally:
        for b in (cd, wd, dd, od, yd):
            if b is not None:
                b.free()


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("mode", [engine.NORM_PLAIN, engine.NORM_GLU_SILU, engine.NORM_GLU_GELU_TANH])
@pytest.mark.parametrize("cols", [64, 300, 2048, 4096])
def test_norm_matmul_bit_identical_to_the_pair(eng, kind, mode, cols):
    rows = 3000 if mode == engine.NORM_PLAIN else 2 * 1500
    print(f"norm_matmul kind={kind} mode={mode} cols={cols}", flush=True)
    t = eng.upload_packed(make(kind, rows, cols, seed=cols + mode))
    rng = np.random.default_rng(cols)
    cur = rng.standard_normal(cols).astype(np.float32) * 3
    delta = rng.standard_normal(cols).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    stride = rows // 2 + 7 if mode != engine.NORM_PLAIN else None
    for d in (None, delta):
        for ydt in (engine.DTYPE_F32, engine.DTYPE_BF16):
            ref_cur, ref_y = norm_pair_reference(eng, t, cur, d, w, 1e-6, mode, ydt, stride)
            got_cur, got_y = run_norm_matmul(eng, t, cur, d, w, 1e-6, mode, ydt, stride)
            assert np.array_equal(got_y, ref_y), (d is None, ydt)
            if d is not None:
                assert np.array_equal(got_cur.view(np.uint32), (cur + d).view(np.uint32))
                assert np.array_equal(got_cur, ref_cur)
            else:
                assert np.all(np.isnan(got_cur))          # nothing stored without delta
    t.free()


def test_norm_matmul_lm_head_rows(eng):
    """The four-rows-per-wave launch (rows >= 65536), Q8 like the LM head."""
    t = eng.upload_packed(make("q8", 70001, 256, seed=1))
    rng = np.random.default_rng(0)
    cur, delta = rng.standard_normal(256).astype(np.float32), rng.standard_normal(256).astype(np.float32)
    w = np.ones(256, np.float32)
    ref = norm_pair_reference(eng, t, cur, delta, w, 1e-5, engine.NORM_PLAIN, engine.DTYPE_F32, None)[1]
    got = run_norm_matmul(eng, t, cur, delta, w, 1e-5, engine.NORM_PLAIN, engine.DTYPE_F32, None)[1]
    assert np.array_equal(got, ref)
    t.free()


def test_norm_matmul_errors(eng):
    wide = eng.upload_packed(make("q8", 8, 4128, seed=0))
    odd = eng.upload_packed(make("q8", 7, 64, seed=0))
    ok = eng.upload_packed(make("q8", 8, 64, seed=0))
    buf = eng.alloc(1 << 16)
    p = buf.ptr
    try:
        cases = [(wide, dict(delta_ptr=0, cur_out_ptr=0, mode=0), engine.VXT_E_UNSUPPORTED),
                 (odd, dict(delta_ptr=0, cur_out_ptr=0, mode=1), engine.VXT_E_SHAPE),
                 (ok, dict(delta_ptr=p + 4096, cur_out_ptr=0, mode=0), engine.VXT_E_ARG),
                 (ok, dict(delta_ptr=p + 4096, cur_out_ptr=p, mode=0), engine.VXT_E_ARG),
                 (ok, dict(delta_ptr=p + 4096, cur_out_ptr=p + 4096, mode=0), engine.VXT_E_ARG),
                 (ok, dict(delta_ptr=0, cur_out_ptr=0, mode=9), engine.VXT_E_ARG)]
        for t, kw, code in cases:
            with pytest.raises(engine.BackendError) as e:
                eng.norm_matmul_dev(t, p, weight_ptr=p + 8192, eps=1e-6, y_ptr=p + 16384,
                                    y_dtype=engine.DTYPE_F32, stream=eng.stream, **kw)
            assert e.value.code == code
    finally:
        for x in (buf, wide, odd, ok):
            x.free()
