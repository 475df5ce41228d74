"""Prefill GEMM with activations of any magnitude.

The reference's gemm_cpu takes f32 X of any magnitude
(crates/vxg-tensor/src/llm_prefill.rs:156-255); the device multiplies f16
operands, so every activation row carries a power-of-two scale that puts its
largest magnitude in [2^14, 2^15) and the epilogue undoes it.  These tests
drive rows from 2^-30 to 2^100 (bf16, about 1e30) and 2^-30 to 2^90 (f32)
through every GEMM path (fused, two-phase with the own dense kernel, two-phase
with the library dense phase), each pinned, at the GEMM bars.
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine, synth
from vxg_amd.formats import bf16_bits_to_f32, f32_to_bf16_bits

from parity_util import THREADS, assert_bf16_close, floor_scale, make, max_rel, run_dev

pytestmark = pytest.mark.gpu

PATHS = {"fused": engine.GEMM_FUSED, "panel": engine.GEMM_PANEL, "library": engine.GEMM_LIBRARY}


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine(0)
    yield e
    e.close()


def ranged_rows(M, cols, lo, hi, seed):
    """N(0,1) rows, row i scaled by 2^p_i with p_i spread over [lo, hi]; one
    row mixes magnitudes within 2^20 (elements scaled by 2^0..2^19)."""
    g = np.random.default_rng(seed)
    X = g.standard_normal((M, cols)).astype(np.float64)
    p = np.round(np.linspace(lo, hi, M)).astype(np.int64)
    X *= np.exp2(p)[:, None]
    X[M // 2] *= np.exp2(g.integers(0, 20, size=cols))
    return X


def check(y, yref, W, X, bf16):
    fl = floor_scale(W, X)
    assert np.all(np.isfinite(yref))
    if bf16:
        assert_bf16_close(y, yref, fl)
    else:
        err = max_rel(y, yref, fl)
        assert err <= 1e-3, err


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("kind", ["g64", "q8", "cb4"])
@pytest.mark.parametrize("M", [24, 130])
def test_gemm_bf16_activations_any_magnitude(eng, path, kind, M):
    print(f"gemm range bf16 path={path} kind={kind} M={M}", flush=True)
    m = make(kind, 70, 320, seed=M + 17)
    t = eng.upload_packed(m)
    xb = f32_to_bf16_bits(ranged_rows(M, 320, -30, 100, seed=M).astype(np.float32))
    X = bf16_bits_to_f32(xb).reshape(M, 320)
    yref = oracle.gemm(m, X, threads=THREADS)
    W = oracle.decode_rows(m)
    eng.set_gemm_path(PATHS[path])
    try:
        check(run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32), yref, W, X, False)
        check(run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16), yref, W, X, True)
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    t.free()


@pytest.mark.parametrize("path", ["panel", "library"])
@pytest.mark.parametrize("kind", ["g64", "q8", "cb4"])
def test_gemm_f32_activations_any_magnitude(eng, path, kind):
    print(f"gemm range f32 path={path} kind={kind}", flush=True)
    M = 40
    m = make(kind, 70, 320, seed=41)
    t = eng.upload_packed(m)
    X = ranged_rows(M, 320, -30, 90, seed=5).astype(np.float32)
    yref = oracle.gemm(m, X, threads=THREADS)
    W = oracle.decode_rows(m)
    eng.set_gemm_path(PATHS[path])
    try:
        check(run_dev(eng, t, X, engine.DTYPE_F32, M, engine.DTYPE_F32), yref, W, X, False)
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    t.free()


def test_gemm_host_api_large_activations(eng):
    """vxt_hip_gemm (f32 in and out, the reference's gemm_cpu signature) with
    activations above the f16 range."""
    m = make("cb4", 50, 300, seed=3)
    t = eng.upload_packed(m)
    X = (synth.make_x_f32(12, 300, seed=3) * np.float32(1e6)).astype(np.float32)
    Y = eng.gemm(t, X)
    check(Y, oracle.gemm(m, X, threads=THREADS), oracle.decode_rows(m), X, False)
    t.free()


def test_gemm_nonfinite_activation_row_propagates(eng):
    """An Inf in one activation row gives non-finite outputs in that row only,
    as the reference's f32 arithmetic does; other rows keep the bar."""
    m = make("g64", 40, 256, seed=8)
    t = eng.upload_packed(m)
    X = synth.make_x_f32(16, 256, seed=8)
    X[3, 17] = np.inf
    xb = f32_to_bf16_bits(X)
    Xq = bf16_bits_to_f32(xb).reshape(16, 256)
    y = run_dev(eng, t, xb, engine.DTYPE_BF16, 16, engine.DTYPE_F32)
    assert not np.all(np.isfinite(y[3]))
    keep = np.r_[0:3, 4:16]
    yref = oracle.gemm(m, Xq[keep], threads=THREADS)
    check(y[keep], yref, oracle.decode_rows(m), Xq[keep], False)
    t.free()


def _inf_rows(M, cols, seed):
    """Activations whose rows 3 and 7 each hold one Inf next to finite entries
    far above the f16 range (1e10): the row's scale must come from its finite
    entries so they stay finite, and the Inf must reach every product."""
    X = synth.make_x_f32(M, cols, seed=seed)
    X[3] *= np.float32(1e10)
    X[3, 17] = np.inf
    X[7] *= np.float32(-3e9)
    X[7, cols - 5] = -np.inf
    return X


@pytest.mark.parametrize("kind,rows,M,path", [
    ("g64", 192, 128, engine.GEMM_AUTO), ("g64", 192, 300, engine.GEMM_AUTO), ("g64", 192, 300, engine.GEMM_PANEL),
    ("g64", 192, 128, engine.GEMM_FUSED), ("g64", 6144, 2048, engine.GEMM_PANEL),
    ("q8", 192, 128, engine.GEMM_AUTO), ("q8", 192, 300, engine.GEMM_PANEL), ("q8", 2048, 2048, engine.GEMM_AUTO),
    ("cb4", 192, 300, engine.GEMM_PANEL), ("cb4", 192, 2048, engine.GEMM_AUTO), ("cb4", 4096, 2048, engine.GEMM_AUTO),
    ("cb4", 4096, 1024, engine.GEMM_AUTO), ("cb4", 2048, 2048, engine.GEMM_AUTO), ("q8", 6144, 512, engine.GEMM_AUTO)])
def test_gemm_inf_with_large_finite_entries(eng, kind, rows, M, path):
    """Rows holding an Inf and finite entries above 65504 give exactly the
    oracle's pattern of +-Inf and NaN outputs (gemm_cpu: w * Inf is +-Inf, or
    NaN where w = 0), and finite rows keep the bar.  The g64 tile path (M =
    128..767), the fused/tile pin, the dense kernels of the two-phase path
    (plain, Q8 block and hi/lo, on both the 128 x 128 and the large-tile
    kernel) are covered."""
    cols = 544
    m = make(kind, rows, cols, seed=21)
    t = eng.upload_packed(m)
    X = _inf_rows(M, cols, seed=22)
    xb = f32_to_bf16_bits(X)
    Xq = bf16_bits_to_f32(xb).reshape(M, cols)
    sel = np.r_[0:9, M - 3:M]
    with np.errstate(invalid="ignore", over="ignore"):
        yref = oracle.gemm(m, Xq[sel], threads=THREADS)
    eng.set_gemm_path(path)
    try:
        y = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)[sel]
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    assert np.array_equal(np.isnan(y), np.isnan(yref))
    assert np.array_equal(np.isinf(y), np.isinf(yref))
    both = np.isinf(y) & np.isinf(yref)
    assert np.array_equal(np.sign(y[both]), np.sign(yref[both]))
    fin = np.all(np.isfinite(yref), axis=1)
    assert fin.sum() == len(sel) - 2
    check(y[fin], yref[fin], oracle.decode_rows(m), Xq[sel][fin], False)
    t.free()


def test_gemm_inf_rows_cb4_tile_path(eng):
    """The cb4 decode-in-loop tile kernel multiplies a residual operand that
    is zero off the residual columns, so an Inf activation gives NaN (not
    +-Inf) across its row; that row is non-finite as in gemm_cpu, the others
    keep the bar."""
    rows, cols = 192, 544
    m = make("cb4", rows, cols, seed=23)
    t = eng.upload_packed(m)
    M = 256
    X = _inf_rows(M, cols, seed=24)
    xb = f32_to_bf16_bits(X)
    Xq = bf16_bits_to_f32(xb).reshape(M, cols)
    eng.set_gemm_path(engine.GEMM_FUSED)
    try:
        y = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    assert not np.isfinite(y[3]).any() and not np.isfinite(y[7]).any()
    keep = np.r_[0:3, 4:7, 8:12]
    check(y[keep], oracle.gemm(m, Xq[keep], threads=THREADS), oracle.decode_rows(m), Xq[keep], False)
    t.free()


# g64 tile-kernel grids (GEMM_FUSED pins the tile kernel above batch 64)
# with one K-way: 100 x 300 x 1576 splits K in 5 slices with a partial
# activation tile, a partial weight tile and columns past K inside the last K
# tile; 128 x 2048 x 2048 splits K in 8 slices; 2048 x 3072 x 512 has one
# slice per tile over 384 tiles (bf16 rows written through LDS).
TILE_SLICES = [(100, 300, 1576), (128, 2048, 2048), (2048, 3072, 512)]


@pytest.mark.parametrize("M,rows,cols", TILE_SLICES)
def test_gemm_tile_slices_any_magnitude(eng, M, rows, cols):
    print(f"gemm tile slices range M={M} rows={rows} cols={cols}", flush=True)
    m = make("g64", rows, cols, seed=M + cols)
    t = eng.upload_packed(m)
    xb = f32_to_bf16_bits(ranged_rows(M, cols, -30, 100, seed=M).astype(np.float32))
    X = bf16_bits_to_f32(xb).reshape(M, cols)
    sel = np.unique(np.r_[0:4, M // 2, M - 4:M, np.random.default_rng(M).choice(M, 8, replace=False)])
    yref = oracle.gemm(m, X[sel], threads=THREADS)
    W = oracle.decode_rows(m)
    eng.set_gemm_path(engine.GEMM_FUSED)
    try:
        check(run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)[sel], yref, W, X[sel], False)
        check(run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16)[sel], yref, W, X[sel], True)
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    t.free()


@pytest.mark.parametrize("M,rows,cols", TILE_SLICES)
def test_gemm_tile_slices_inf_with_large_finite_entries(eng, M, rows, cols):
    """The Inf / NaN pattern of test_gemm_inf_with_large_finite_entries on the
    tile grids above, split K included: the row scale comes from the finite
    entries, and an Inf reaches the partial sums of its slice."""
    print(f"gemm tile slices inf M={M} rows={rows} cols={cols}", flush=True)
    m = make("g64", rows, cols, seed=31)
    t = eng.upload_packed(m)
    X = _inf_rows(M, cols, seed=32)
    xb = f32_to_bf16_bits(X)
    Xq = bf16_bits_to_f32(xb).reshape(M, cols)
    sel = np.r_[0:9, M - 3:M]
    with np.errstate(invalid="ignore", over="ignore"):
        yref = oracle.gemm(m, Xq[sel], threads=THREADS)
    for ydt in (engine.DTYPE_F32, engine.DTYPE_BF16):
        eng.set_gemm_path(engine.GEMM_FUSED)
        try:
            yraw = run_dev(eng, t, xb, engine.DTYPE_BF16, M, ydt)[sel]
        finally:
            eng.set_gemm_path(engine.GEMM_AUTO)
        y = yraw if ydt == engine.DTYPE_F32 else bf16_bits_to_f32(yraw).reshape(yraw.shape)
        assert np.array_equal(np.isnan(y), np.isnan(yref))
        assert np.array_equal(np.isinf(y), np.isinf(yref))
        both = np.isinf(y) & np.isinf(yref)
        assert np.array_equal(np.sign(y[both]), np.sign(yref[both]))
        fin = np.all(np.isfinite(yref), axis=1)
        assert fin.sum() == len(sel) - 2
        check(yraw[fin], yref[fin], oracle.decode_rows(m), Xq[sel][fin], ydt == engine.DTYPE_BF16)
    t.free()
