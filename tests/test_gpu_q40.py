"""GPU parity of Q4_0 weights (q4_0.rs) through the C ABI.

The device keeps a Q4_0 matrix in its own planes (16 nibble bytes and one f16
scale per block of 32: 4.5 bits per weight) and streams the nibbles in the
GEMV (vxt_gemv.metal:461-520); prefill decodes them into the GEMM's weight
panel.  Bars as in test_gpu_parity:
dequant bit-exact against decode_row (q4_0.rs:77-97); GEMV and GEMM within
1e-3 of the oracle (gemv_cpu, q4_0.rs:109-145, and gemm_cpu over decode_row)
relative to max(|y|, 2^-10 sum|wx|); bf16 outputs within 1 ulp.
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine, loaders, synth
from vxg_amd.formats import Q4_0Matrix, bf16_bits_to_f32, f32_to_bf16_bits
from archive_util import q4_0_section, write_vxt
from parity_util import THREADS, assert_bf16_close, assert_bits_equal, floor_scale, max_rel, run_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


def make_q40(rows, cols, seed, std=0.02):
    g = np.random.default_rng(seed)
    return oracle.q40_encode(rows, cols, g.normal(0, std, (rows, cols)).astype(np.float32))


@pytest.mark.parametrize("rows,cols", [(1, 32), (9, 70), (33, 544), (64, 4096)])
def test_q40_dequant_bit_exact(eng, rows, cols):
    m = make_q40(rows, cols, seed=rows + cols)
    sc = m.scales_f16.copy()
    sc[::5] = 0x0001            # subnormal scales
    sc[1::7] = 0x0000           # zero scale
    sc[2::11] = 0xBC00          # negative scale (-1)
    m = Q4_0Matrix(m.rows, m.cols, m.padded_cols, sc, m.qs_words)
    t = eng.upload_packed(m)
    got = eng.dequant_rows(t)
    assert_bits_equal(got, oracle.decode_rows(m))
    assert (t.kind, t.rows, t.cols) == (engine.KIND_Q4_0, rows, cols)
    kb = (cols + 31) // 32   # 18 bytes per block resident, each plane 256-byte aligned
    assert t.device_bytes <= rows * kb * 18 + 512
    t.free()


def test_q40_dequant_nonfinite_scales(eng):
    m = make_q40(4, 64, seed=3)
    sc = m.scales_f16.copy()
    sc[0], sc[3], sc[5] = 0x7C00, 0xFC00, 0x7E00     # +inf, -inf, NaN
    m = Q4_0Matrix(m.rows, m.cols, m.padded_cols, sc, m.qs_words)
    t = eng.upload_packed(m)
    assert_bits_equal(eng.dequant_rows(t), oracle.decode_rows(m))
    t.free()


@pytest.mark.parametrize("rows,cols", [(197, 544), (2048, 2048), (1000, 70)])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_q40_gemv(eng, rows, cols, M, xdt):
    m = make_q40(rows, cols, seed=rows * 7 + M)
    t = eng.upload_packed(m)
    if xdt == "bf16":
        xh = synth.make_x_bf16(M, cols, seed=M)
        X = bf16_bits_to_f32(xh).reshape(M, cols)
        xd = engine.DTYPE_BF16
    else:
        X = synth.make_x_f32(M, cols, seed=M)
        xh, xd = X, engine.DTYPE_F32
    yref = np.stack([oracle.gemv(m, X[i], threads=THREADS) for i in range(M)])
    fl = floor_scale(oracle.decode_rows(m), X)
    y = run_dev(eng, t, xh, xd, M, engine.DTYPE_F32)
    assert max_rel(y, yref, fl) <= 1e-3
    yb = run_dev(eng, t, xh, xd, M, engine.DTYPE_BF16)
    assert_bf16_close(yb, yref, fl)
    t.free()


def test_q40_gemv_reference_bar_197x544(eng):
    """tensor_roundtrip_gemv.rs:273-279's GPU bar (max |err| < 2e-4) on Q4_0."""
    m = make_q40(197, 544, seed=77, std=0.05)
    t = eng.upload_packed(m)
    x = synth.make_x_f32(1, 544, seed=78)[0]
    y = np.empty(197, np.float32)
    t.run_gemv(eng, x, y)
    assert np.max(np.abs(y - oracle.gemv(m, x))) < 2e-4
    t.free()


@pytest.mark.parametrize("M", [9, 64, 300])
@pytest.mark.parametrize("path", [engine.GEMM_AUTO, engine.GEMM_PANEL, engine.GEMM_FUSED])
def test_q40_gemm(eng, M, path):
    rows, cols = 520, 1000
    m = make_q40(rows, cols, seed=M)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(M, cols, seed=M + 1)
    X = bf16_bits_to_f32(xb).reshape(M, cols)
    sel = np.r_[0:3, M // 2, M - 3:M]
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


def test_q40_archive_upload_matches_planes(eng):
    m = make_q40(40, 300, seed=5)
    with loaders.VxtArchive(write_vxt([("w", q4_0_section(0, 0, m))])) as ar:
        ta = ar.upload(eng, "w")
    tp = eng.upload_packed(m)
    assert_bits_equal(eng.dequant_rows(ta), eng.dequant_rows(tp))
    assert_bits_equal(eng.dequant_rows(ta), oracle.decode_rows(m))
    ta.free()
    tp.free()
