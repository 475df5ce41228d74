"""GPU: prefill GEMM with the weights decoded inside the MFMA loop.

For g64 and Q8_0 tensors with bf16 activations, ``vxt_hip_set_gemm_path(FUSED)``
pins the kernels that decode inside the MFMA loop (the fused kernel; for g64
above batch 64 the tile kernel), and ``PANEL`` pins the two-phase path (f16
panel, then the dense kernel).  Both must meet the GEMM
bar against the oracle (max relative error <= 1e-3 of
max(|y_ref|, 2^-10 * sum |w x|); bf16 outputs within 1 bf16 ulp), on shapes
that cross every tile edge of the fused kernel: M around 32 / 64 / 128 (the
three fragment counts and several M tiles), rows around 128 (a workgroup's
rows), columns around 64 (a K tile), 256 (a chunk) and odd multiples of 32
(a Q8 row whose last K tile holds one block), plus K split across
workgroups.
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine, synth
from vxg_amd.formats import bf16_bits_to_f32, f32_to_bf16_bits
from parity_util import THREADS, assert_bf16_close, floor_scale, make, max_rel, run_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


def both_paths(eng, t, xb, M):
    """(f32 out, bf16 out) of the decode-in-loop path, then f32 out of the
    panel path."""
    eng.set_gemm_path(engine.GEMM_FUSED)
    try:
        yf = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        yb = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16)
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    eng.set_gemm_path(engine.GEMM_PANEL)
    try:
        yp = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    return yf, yb, yp


def check(m, xb, M, yf, yb, yp, sample=None):
    X = bf16_bits_to_f32(xb).reshape(M, m.cols)
    sel = np.arange(M) if sample is None else sample
    W = oracle.decode_rows(m)
    yref = oracle.gemm(m, X[sel], threads=THREADS)
    fl = floor_scale(W, X[sel])
    assert max_rel(yf[sel], yref, fl) <= 1e-3
    assert max_rel(yp[sel], yref, fl) <= 1e-3
    assert_bf16_close(yb[sel], yref, fl)
    assert np.array_equal(yb, f32_to_bf16_bits(yf))


@pytest.mark.parametrize("kind", ["g64", "q8"])
@pytest.mark.parametrize("rows,cols", [(1, 32), (31, 96), (127, 200), (129, 544), (260, 1056)])
@pytest.mark.parametrize("M", [9, 32, 33, 64, 65, 128, 161])
def test_fused_tail_shapes(eng, kind, rows, cols, M):
    m = make(kind, rows, cols, seed=rows * 7 + cols + M)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(M, cols, seed=M + cols)
    yf, yb, yp = both_paths(eng, t, xb, M)
    check(m, xb, M, yf, yb, yp)
    t.free()


@pytest.mark.parametrize("kind", ["g64", "q8"])
@pytest.mark.parametrize("M,N,K", [(16, 64, 4096), (40, 300, 3000), (128, 2048, 6144), (96, 6144, 2048),
                                   (300, 1500, 3000), (384, 2048, 6144)])
def test_fused_split_k_deterministic(eng, kind, M, N, K):
    """K split across workgroups: fixed-order partial sums, identical across runs."""
    m = make(kind, N, K, seed=M + N)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(M, K, seed=K)
    yf, yb, yp = both_paths(eng, t, xb, M)
    sel = np.unique(np.r_[0, M - 1, np.random.default_rng(M).choice(M, min(M, 12), replace=False)])
    check(m, xb, M, yf, yb, yp, sample=sel)
    eng.set_gemm_path(engine.GEMM_FUSED)   # the same path again
    try:
        y2 = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    assert np.array_equal(yf.view(np.uint32), y2.view(np.uint32))
    t.free()


@pytest.mark.parametrize("kind", ["g64", "q8"])
@pytest.mark.parametrize("M,N,K", [(16, 6144, 6144), (200, 4096, 4096), (24, 1000, 5000)])
def test_fused_multi_chunk_workgroups(eng, kind, M, N, K):
    """Workgroups that walk 3-5 chunks (both activation buffers in turn, an
    odd count ending on the first), several M tiles, ragged row counts."""
    m = make(kind, N, K, seed=M + K)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(M, K, seed=N)
    yf, yb, yp = both_paths(eng, t, xb, M)
    sel = np.unique(np.r_[0, M - 1, np.random.default_rng(N).choice(M, min(M, 10), replace=False)])
    check(m, xb, M, yf, yb, yp, sample=sel)
    t.free()


@pytest.mark.parametrize("kind", ["g64", "q8"])
def test_fused_path_forced_at_large_batch(eng, kind):
    """GEMM_FUSED decodes inside the MFMA loop past the automatic batch limit
    (Q8: the fused kernel; g64: the tile kernel)."""
    M, N, K = 512, 640, 1024
    m = make(kind, N, K, seed=77)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(M, K, seed=78)
    eng.set_gemm_path(engine.GEMM_FUSED)
    try:
        yf = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    finally:
        eng.set_gemm_path(engine.GEMM_AUTO)
    yp = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)   # auto: the two-phase path at M = 512
    X = bf16_bits_to_f32(xb).reshape(M, K)
    sel = np.r_[0:8, 250:260, 504:512]
    fl = floor_scale(oracle.decode_rows(m), X[sel])
    yref = oracle.gemm(m, X[sel], threads=THREADS)
    assert max_rel(yf[sel], yref, fl) <= 1e-3
    assert max_rel(yp[sel], yref, fl) <= 1e-3
    t.free()


def test_fused_ragged_row_ignores_padding_table_entries(eng):
    """Padding columns of a g64 row point at an Inf table entry that no real
    column uses: the fused decode zeroes them, so outputs stay finite."""
    rows, cols = 70, 100                       # kp 128: columns 100..127 are padding
    m = synth.make_g64(rows, cols, seed=3)
    idx = m.idx.reshape(rows, m.padded_cols // 2).copy()
    for c in range(cols):                      # real columns: indices 0..14
        sh = 4 * (c % 2)
        q = (idx[:, c // 2] >> sh) & 0xF
        q = np.where(q == 15, 14, q).astype(np.uint8)
        idx[:, c // 2] = (idx[:, c // 2] & np.uint8(0xF0 >> sh)) | (q << sh).astype(np.uint8)
    for c in range(cols, m.padded_cols):       # padding columns: index 15
        sh = 4 * (c % 2)
        idx[:, c // 2] = (idx[:, c // 2] & np.uint8(0xF0 >> sh)) | np.uint8(15 << sh)
    m.idx = idx.reshape(-1)
    lut = m.lut_f16.reshape(-1, 16).copy()
    lut[1::2, 15] = 0x7C00                     # Inf in the last group of every row
    m.lut_f16 = lut.reshape(-1)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(40, cols, seed=4)
    eng.set_gemm_path(engine.GEMM_AUTO)
    yf = run_dev(eng, t, xb, engine.DTYPE_BF16, 40, engine.DTYPE_F32)
    X = bf16_bits_to_f32(xb).reshape(40, cols)
    assert np.isfinite(yf).all()
    assert max_rel(yf, oracle.gemm(m, X, threads=THREADS), floor_scale(oracle.decode_rows(m), X)) <= 1e-3
    t.free()


def test_fused_unaligned_activations(eng):
    """Activations at an address that is not 16-byte aligned take the guarded
    copy into LDS; the result is bit-identical to the aligned one."""
    m = make("q8", 200, 512, seed=6)
    t = eng.upload_packed(m)
    M = 48
    xb = synth.make_x_bf16(M, 512, seed=7)
    buf = eng.alloc(xb.nbytes + 64)
    yd = eng.alloc(M * 200 * 4)
    outs = []
    for off in (0, 2):
        staged = np.zeros(xb.nbytes // 2 + 32, np.uint16)
        staged[off // 2: off // 2 + xb.size] = xb.reshape(-1)
        buf.upload(staged)
        eng.matmul_dev(t, buf.ptr + off, engine.DTYPE_BF16, M, yd.ptr, engine.DTYPE_F32, eng.stream)
        eng.synchronize()
        outs.append(yd.download(np.float32, (M, 200)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    X = bf16_bits_to_f32(xb).reshape(M, 512)
    assert max_rel(outs[0], oracle.gemm(m, X, threads=THREADS), floor_scale(oracle.decode_rows(m), X)) <= 1e-3
    buf.free()
    yd.free()
    t.free()


def test_gemm_path_rejects_unknown(eng):
    with pytest.raises(engine.BackendError):
        eng.set_gemm_path(4)
