"""GPU parity of the large-batch GEMM kernels: the g64 tile kernel
(gemm_tile.hip) and the interleaved dense kernel of the two-phase path
(gemm_dense.hip), at ragged shapes and through every K-way / split / epilogue
branch, against the oracle's gemm_cpu (llm_prefill.rs:156-255).

Bars as in test_gpu_parity: f32 out within 1e-3 of the oracle relative to
max(|y|, 2^-10 sum|wx|); bf16 out within 1 ulp of f32_to_bf16(y_ref); bf16
output equal to the rounding of the f32 output of the same call path.
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine, synth
from vxg_amd.formats import Cb4G64Matrix, bf16_bits_to_f32, f32_to_bf16_bits, f32_to_f16_bits
from parity_util import THREADS, assert_bf16_close, floor_scale, make, max_rel, run_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


def check(eng, m, M, path, sel=None, seed=0):
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(M, m.cols, seed=seed)
    X = bf16_bits_to_f32(xb).reshape(M, m.cols)
    sel = np.unique(np.r_[0:3, M // 2, M - 3:M]) if sel is None else sel
    W = oracle.decode_rows(m)
    yref = oracle.gemm(m, X[sel], threads=THREADS)
    eng.set_gemm_path(path)
    try:
        yf = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        yb = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16)
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    fl = floor_scale(W, X[sel])
    assert max_rel(yf[sel], yref, fl) <= 1e-3
    assert_bf16_close(yb[sel], yref, fl)
    assert np.array_equal(yb, f32_to_bf16_bits(yf))
    t.free()
    return yf


# The tile kernel (pinned: GEMM_FUSED takes it for g64 above batch 64): one
# K-way from 384 tiles of 128 x 128, two below; split K below ~256
# workgroups; ragged M, N and K; N not a multiple of 8 (per-lane epilogue)
# and of 128 (partial last tile).
@pytest.mark.parametrize("M,N,K", [(65, 97, 64), (130, 640, 100), (300, 1500, 1000), (129, 2048, 3000),
                                   (1000, 384, 2048), (2048, 6144, 192), (640, 8200, 448)])
def test_tile_kernel_shapes(eng, M, N, K):
    check(eng, synth.make_g64(N, K, seed=M + N), M, engine.GEMM_FUSED, seed=K)


def test_tile_kernel_repeatable(eng):
    """Split-K partial sums are added in slice order: bit-identical reruns."""
    m = synth.make_g64(256, 6144, seed=5)
    a = check(eng, m, 200, engine.GEMM_FUSED)
    b = check(eng, m, 200, engine.GEMM_FUSED)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_g64_nonfinite_padding_table(eng):
    """Padding columns (>= K) index table entries; decode_row stops at cols, so
    an Inf entry reached only from padding must not reach the output.  Such
    tensors take the panel path; the same matrix with a finite entry takes
    the tile kernel.  Both match the oracle."""
    m = synth.make_g64(200, 100, seed=11)        # padded to 128: columns 100..127 are padding
    idx = m.idx.reshape(200, 64).copy()
    lut = m.lut_f16.reshape(200, 2, 16).copy()
    # last group: real columns use entries 0..14, padding columns entry 15
    for r in range(200):
        nib = np.zeros(64, np.uint8)
        nib[:36] = np.random.default_rng(r).integers(0, 15, 36)   # columns 64..99
        nib[36:] = 15                                                # columns 100..127
        idx[r, 32:] = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    for entry in (0x7C00, 0x3C00):   # +Inf (panel path), then 1.0 (tile kernel)
        lut[:, 1, 15] = entry
        mm = Cb4G64Matrix(200, 100, 128, idx.reshape(-1).copy(), lut.reshape(-1).copy())
        y = check(eng, mm, 300, engine.GEMM_AUTO)
        assert np.isfinite(y).all()


# The interleaved dense kernel (two-phase path, 128 x 128 tiles for M >= 256)
# in each weight mode: g64 plain, Q8 block scales, cb4 hi/lo; ragged shapes;
# split K on small grids.
@pytest.mark.parametrize("kind", ["g64", "q8", "cb4"])
@pytest.mark.parametrize("M,N,K", [(256, 97, 64), (300, 1500, 1000), (1000, 130, 4096), (513, 2048, 2048)])
def test_dense_kernel_modes(eng, kind, M, N, K):
    check(eng, make(kind, N, K, seed=M + K), M, engine.GEMM_PANEL, seed=N)


# The large-tile dense kernel (gemm_dense3.hip) streams both operands from
# planes of 1 KB pieces (16 rows x 32 columns, rows padded to 16): batch and
# weight row counts that are not multiples of 16, K short of a whole piece,
# every wave tile and weight mode the planner gives it (plain on 256 x 192,
# 256 x 128 and 128 x 128 of 4 waves; Q8 block and hi/lo on 128 x 128 of 4
# waves and 256 x 128 of 8 waves), 128 x 128 in one K range and in two.
@pytest.mark.parametrize("kind,M,N,K", [("g64", 1800, 5376, 512), ("g64", 1030, 6600, 256),
                                        ("g64", 1100, 3100, 1000), ("g64", 1000, 1500, 1000),
                                        ("q8", 1000, 3000, 1000), ("q8", 1000, 1500, 1000),
                                        ("q8", 1000, 6100, 256), ("cb4", 1000, 3000, 1000),
                                        ("cb4", 1000, 1500, 1000), ("cb4", 1000, 6100, 256)])
def test_large_tile_kernel_ragged(eng, kind, M, N, K):
    check(eng, make(kind, N, K, seed=M + N), M, engine.GEMM_PANEL, seed=K)


@pytest.mark.parametrize("rows,K,M", [(300, 2048, 512), (3000, 1024, 1000), (6144, 256, 1024)])
def test_dense_kernel_q8_block_scales_extreme(eng, rows, K, M):
    """Block scales spanning subnormal to 2^15 in one row (each block's
    fragment is scaled on its own), on the interleaved kernel and on the
    large-tile kernel's 4-wave and 8-wave tiles."""
    q = synth.make_q8(rows, K, seed=7)
    b = q.blocks.copy().reshape(-1, 34)
    b[0::5, 0:2] = np.array([0x7800], np.uint16).view(np.uint8)   # d = 32768
    b[1::7, 0:2] = np.array([0x0001], np.uint16).view(np.uint8)   # subnormal d
    q.blocks = b.reshape(-1)
    check(eng, q, M, engine.GEMM_PANEL)


# ---- the cb4 decode-in-loop tile kernel (GEMM_FUSED pins it for eligible
# tensors: finite planes, each row's residual columns increasing, at most
# 16384 residuals per 128-row block) ------------------------------------------

def check_parts(eng, parts, M, path, seed=0):
    """check() for a row-concatenated tensor of cb4 parts."""
    t = eng.upload_concat(parts)
    K = parts[0].cols
    xb = synth.make_x_bf16(M, K, seed=seed)
    X = bf16_bits_to_f32(xb).reshape(M, K)
    sel = np.unique(np.r_[0:3, M // 2, M - 3:M])
    W = np.concatenate([oracle.decode_rows(p) for p in parts])
    yref = np.concatenate([oracle.gemm(p, X[sel], threads=THREADS) for p in parts], axis=1)
    eng.set_gemm_path(path)
    try:
        yf = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        yb = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16)
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    fl = floor_scale(W, X[sel])
    assert max_rel(yf[sel], yref, fl) <= 1e-3
    assert_bf16_close(yb[sel], yref, fl)
    assert np.array_equal(yb, f32_to_bf16_bits(yf))
    t.free()
    return yf


# ragged M, N and K; split K on small grids (M <= 128, short N); a residual
# density that puts several residuals in one lane's 8-column window
@pytest.mark.parametrize("M,N,K,frac", [(9, 130, 100, 0.0074), (130, 640, 300, 0.0074), (300, 1500, 1000, 0.0074),
                                        (129, 2048, 3000, 0.0074), (1000, 384, 2048, 0.0074),
                                        (2048, 640, 192, 0.0074), (64, 900, 448, 0.05)])
def test_cb4_tile_kernel_shapes(eng, M, N, K, frac):
    m = synth.make_cb4(N, K, seed=M + N, outlier_frac=frac)
    check(eng, m, M, engine.GEMM_FUSED, seed=K)


def test_cb4_tile_kernel_repeatable(eng):
    """Split-K partial sums are added in slice order: bit-identical reruns."""
    m = synth.make_cb4(256, 6144, seed=5)
    a = check(eng, m, 200, engine.GEMM_FUSED)
    b = check(eng, m, 200, engine.GEMM_FUSED)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_cb4_tile_kernel_concatenated_parts(eng):
    """Three parts with their own centroid tables, split at rows that are not
    multiples of 32, so lanes of one wave read different tables."""
    parts = [synth.make_cb4(r, 700, seed=20 + i) for i, r in enumerate((45, 70, 51))]
    for i, p in enumerate(parts):
        p.centroids = (p.centroids * (1.0 + 3 * i)).astype(np.float32)
    check_parts(eng, parts, 150, engine.GEMM_FUSED, seed=3)


def test_cb4_tile_kernel_scales_zero_and_extreme(eng):
    """Zero-scale groups, scales near the f16 maximum and centroids far below
    one in the same tensor: the per-row exponents keep every hi / lo split in
    the f16 range."""
    m = synth.make_cb4(300, 1024, seed=9)
    sc = m.scales_f16.reshape(300, -1).copy()
    sc[0::7, 1] = 0
    sc[3::11, :] = np.array([0x7BFF], np.uint16)        # 65504
    sc[5::13, 2] = np.array([0x0001], np.uint16)        # smallest subnormal
    m.scales_f16 = sc.reshape(-1)
    m.centroids = (m.centroids * 1e-3).astype(np.float32)
    check(eng, m, 260, engine.GEMM_FUSED, seed=4)


def test_cb4_tile_kernel_ineligible_tensor(eng):
    """A residual column repeated within a row (decode_row adds both) makes
    the tensor take the two-phase path, which meets the same bar."""
    m = synth.make_cb4(200, 512, seed=12)
    rp = m.outlier_row_ptr
    r = int(np.argmax(np.diff(rp.astype(np.int64)) >= 2))
    m.outliers_packed = m.outliers_packed.copy()
    a = int(rp[r])
    m.outliers_packed[a + 1] = (m.outliers_packed[a + 1] & 0xFFFF0000) | (m.outliers_packed[a] & 0xFFFF)
    check(eng, m, 150, engine.GEMM_FUSED, seed=6)


@pytest.mark.parametrize("M", [128, 300])
def test_cb4_tile_kernel_on_auto_path(eng, M):
    """From batch 128 to 511 (K >= N here; to 255 when K < N) the automatic
    choice takes the cb4 tile kernel for an eligible tensor: the same bits
    as the pinned kernel, and the
    oracle bar; an ineligible tensor keeps the two-phase path there."""
    m = synth.make_cb4(640, 2048, seed=M)
    a = check(eng, m, M, engine.GEMM_AUTO, seed=1)
    b = check(eng, m, M, engine.GEMM_FUSED, seed=1)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    rp = m.outlier_row_ptr
    r = int(np.argmax(np.diff(rp.astype(np.int64)) >= 2))
    m.outliers_packed = m.outliers_packed.copy()
    i = int(rp[r])
    m.outliers_packed[i + 1] = (m.outliers_packed[i + 1] & 0xFFFF0000) | (m.outliers_packed[i] & 0xFFFF)
    c = check(eng, m, M, engine.GEMM_AUTO, seed=2)
    d = check(eng, m, M, engine.GEMM_PANEL, seed=2)
    assert np.array_equal(c.view(np.uint32), d.view(np.uint32))


def _block_of_residuals(total, seed):
    """128 x 6144 cb4 whose one 128-row block holds `total` residuals:
    128 per row at increasing columns, the remainder on row 0."""
    m = synth.make_cb4(128, 6144, seed=seed, outlier_frac=0.0)
    g = np.random.default_rng(seed)
    per = np.full(128, total // 128, np.int64)
    per[0] += total - per.sum()
    ents = []
    for r in range(128):
        cols = np.sort(g.choice(6144, size=int(per[r]), replace=False)).astype(np.uint32)
        vals = f32_to_f16_bits(g.normal(0, 0.02, size=cols.size).astype(np.float32)).astype(np.uint32)
        ents.append(cols | (vals << np.uint32(16)))
    m.outliers_packed = np.concatenate(ents).astype(np.uint32)
    m.outlier_row_ptr = np.r_[0, np.cumsum(per)].astype(np.uint32)
    return m


def test_cb4_tile_kernel_residual_cap(eng):
    """Eligibility at the LDS cap: a block of exactly 16384 residuals takes
    the tile kernel (on the automatic route at batch 200 its results are the
    pinned kernel's bits, which differ from the two-phase path's summation),
    one more residual makes the tensor take the two-phase path (automatic =
    pinned panel bits).  Both at the bar."""
    at_cap = _block_of_residuals(16384, seed=41)
    over = _block_of_residuals(16385, seed=41)
    a = check(eng, at_cap, 200, engine.GEMM_AUTO, seed=5)
    b = check(eng, at_cap, 200, engine.GEMM_FUSED, seed=5)
    p = check(eng, at_cap, 200, engine.GEMM_PANEL, seed=5)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert not np.array_equal(b.view(np.uint32), p.view(np.uint32))
    c = check(eng, over, 200, engine.GEMM_AUTO, seed=5)
    d = check(eng, over, 200, engine.GEMM_PANEL, seed=5)
    e = check(eng, over, 200, engine.GEMM_FUSED, seed=5)   # pinned: falls back to the two-phase path too
    assert np.array_equal(c.view(np.uint32), d.view(np.uint32))
    assert np.array_equal(e.view(np.uint32), d.view(np.uint32))
