"""GPU parity: the HIP path against the CPU oracle, through the C ABI.

Bars (written into each check):
  * dequant: bit-exact (NaN patterns compared as NaN);
  * GEMV / GEMM, f32 out: max relative error <= 1e-3, where the error of an
    output is measured against max(|y_ref|, 2^-10 * sum_c |w_c x_c|) so that
    outputs that cancel to near zero are judged on the scale of their terms;
  * bf16 out: within 1 bf16 ulp of f32_to_bf16(y_ref) (or inside the same
    near-zero floor);
  * the reference's own GPU-vs-CPU bar, max |err| < 2e-4 at rows=197,
    cols=544 (tensor_roundtrip_gemv.rs:273-279), is checked as written;
  * run-to-run and launch-grouping bit identity (llm_gpu_cpu_parity.rs:697).
"""
import os

import numpy as np
import pytest

import oracle
from vxg_amd import engine, synth
from vxg_amd.formats import (CodebookMatrix, bf16_bits_to_f32, f32_to_bf16_bits,
                             f32_to_f16_bits)
from parity_util import (GOLD, THREADS, assert_bf16_close, assert_bits_equal, closed_form, f16b,
                         floor_scale, gemv_ref, make, max_rel, q8_floor, run_dev)

pytestmark = pytest.mark.gpu

@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


# ---------------------------------------------------------------- dequant

@pytest.mark.parametrize("cols", [1, 129, 257, 385])
def test_dequant_closed_form_fixture(eng, cols):
    """metal_llm_tests.rs:31-58 (+ :135-139): exact GPU cb4 row dequant."""
    m = closed_form(515, cols, lambda c: [(f16b(v) << 16) | (c - 1)
                                          for v in (0.33325195, -0.125, 0.0009765625)])
    t = eng.upload_packed(m)
    got = eng.dequant_rows(t)
    gold = np.load(os.path.join(GOLD, "cb4_closed_form.npz"))
    for i, r in enumerate(gold[f"c{cols}_rows"]):
        assert_bits_equal(got[r], gold[f"c{cols}_expected"][i])
    assert_bits_equal(got, oracle.decode_rows(m))
    # a row window (the embedding-row probe): rows 513..514
    assert_bits_equal(eng.dequant_rows(t, 513, 2), got[513:515])


@pytest.mark.parametrize("rows", [1, 3, 4, 5, 7, 9, 17])
@pytest.mark.parametrize("cols", [1, 129, 257, 513])
def test_dequant_duplicate_column_outliers(eng, rows, cols):
    m = closed_form(rows, cols, lambda c: [f16b(0.25) << 16, f16b(-0.125) << 16,
                                           (f16b(0.5) << 16) | (c - 1)])
    gold = np.load(os.path.join(GOLD, "cb4_dup_outlier.npz"))
    got = eng.dequant_rows(eng.upload_packed(m))
    assert_bits_equal(got, gold[f"r{rows}_c{cols}"])


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 33), (197, 544), (512, 2048), (64, 6144)])
def test_dequant_random_bit_exact(eng, kind, rows, cols):
    m = make(kind, rows, cols, seed=rows + cols)
    got = eng.dequant_rows(eng.upload_packed(m))
    assert_bits_equal(got, oracle.decode_rows(m))


def test_dequant_special_values(eng):
    """Subnormal, zero, inf and NaN scales / table entries dequantise exactly."""
    m = synth.make_g64(4, 128, seed=1)
    lut = m.lut_f16.copy()
    lut[:8] = [0x0000, 0x8000, 0x0001, 0x83FF, 0x7C00, 0xFC00, 0x7E01, 0x7C01]
    m.lut_f16 = lut
    m.idx = np.arange(m.idx.size, dtype=np.uint32).astype(np.uint8)
    got = eng.dequant_rows(eng.upload_packed(m))
    assert_bits_equal(got, oracle.decode_rows(m))
    q = synth.make_q8(2, 64, seed=2)
    b = q.blocks.copy().reshape(-1, 34)
    b[0, 0:2] = np.array([0x0001], np.uint16).view(np.uint8)   # subnormal d
    b[1, 0:2] = np.array([0x7C00], np.uint16).view(np.uint8)   # inf d
    q.blocks = b.reshape(-1)
    got = eng.dequant_rows(eng.upload_packed(q))
    assert_bits_equal(got, oracle.decode_rows(q))


# ---------------------------------------------------------------- GEMV

@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("cols", [1, 129, 257, 513, 544])
def test_gemv_tail_shapes_host_api(eng, kind, cols):
    for rows in (1, 3, 5, 7, 9, 17):
        m = make(kind, rows, cols, seed=rows * 7 + cols)
        t = eng.upload_packed(m)
        x = synth.make_x_f32(1, cols, seed=cols)[0]
        y = np.full(rows, np.nan, np.float32)
        t.run_gemv(eng, x, y)
        W = oracle.decode_rows(m)
        yref = oracle.gemv(m, x)
        assert max_rel(y, yref, floor_scale(W, x[None])[0]) <= 1e-3, (rows, cols)


def test_gemv_reference_bar_197x544(eng):
    """tensor_roundtrip_gemv.rs:188-279: GPU vs CPU max_abs_err < 2e-4."""
    for kind in ("cb4", "g64", "q8"):
        m = make(kind, 197, 544, seed=11)
        x = synth.make_x_f32(1, 544, seed=999)[0] * np.float32(0.1)
        y = np.empty(197, np.float32)
        eng.upload_packed(m).run_gemv(eng, x, y)
        assert np.max(np.abs(y - oracle.gemv(m, x, threads=4))) < 2e-4, kind


BENCH_SHAPES = [(2048, 2048), (2048, 6144), (6144, 2048), (4096, 4096)]


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("K,N", BENCH_SHAPES)
@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_gemv_baseline_shapes_bf16(eng, kind, K, N, M):
    m = make(kind, N, K, seed=K + N + M)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(M, K, seed=M)
    X = bf16_bits_to_f32(xb).reshape(M, K)
    yf = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    yb = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16)
    yref = gemv_ref(m, X)
    W = oracle.decode_rows(m)
    fl = floor_scale(W, X)
    assert max_rel(yf, yref, fl) <= 1e-3
    assert_bf16_close(yb, yref, fl)


@pytest.mark.parametrize("rows,cols", [(6144, 2048), (12288, 2048), (2048, 6144), (300, 2052), (77, 4100),
                                       (5, 130)])
def test_gemv_g64_one_token_f32_x(eng, rows, cols):
    """g64 at M = 1 with f32 activations (an attention output): the one-token
    LDS-staged kernel stages them as they are (cols % 4 == 0; one, two and
    three K steps, one and two rows per wave), the generic kernel otherwise
    (130 columns).  Against the oracle, and bit-equal to the bf16-activation
    call on the same (bf16-representable) values: both stage f32 in LDS and
    sum in one order."""
    m = make("g64", rows, cols, seed=rows + cols)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(1, cols, seed=cols)
    X = bf16_bits_to_f32(xb).reshape(1, cols)
    yf = run_dev(eng, t, np.ascontiguousarray(X, dtype=np.float32), engine.DTYPE_F32, 1, engine.DTYPE_F32)
    yb = run_dev(eng, t, np.ascontiguousarray(X, dtype=np.float32), engine.DTYPE_F32, 1, engine.DTYPE_BF16)
    ref = gemv_ref(m, X)
    fl = floor_scale(oracle.decode_rows(m), X)
    assert max_rel(yf, ref, fl) <= 1e-3
    assert_bf16_close(yb, ref, fl)
    if cols % 8 == 0:
        assert_bits_equal(run_dev(eng, t, xb, engine.DTYPE_BF16, 1, engine.DTYPE_F32), yf)


def test_gemv_q8_config0_f32(eng):
    """Config 0: Q8, M=1, K=N=4096, x f32 N(0,1), y f32, seed 0."""
    m = synth.make_q8(4096, 4096, seed=0)
    x = synth.make_x_f32(1, 4096, seed=0)
    t = eng.upload_packed(m)
    y = run_dev(eng, t, x, engine.DTYPE_F32, 1, engine.DTYPE_F32)
    yref = oracle.gemv(m, x[0], threads=THREADS)
    assert max_rel(y[0], yref, floor_scale(oracle.decode_rows(m), x)[0]) <= 1e-3


def test_gemv_lm_head_q8(eng):
    """Q8 LM head 151936 x 2048 at M = 1, 2, 4 and 8 against the oracle."""
    m = synth.make_q8(151936, 2048, seed=5)
    t = eng.upload_packed(m)
    for M in (1, 2, 4, 8):
        xb = synth.make_x_bf16(M, 2048, seed=M)
        X = bf16_bits_to_f32(xb).reshape(M, 2048)
        y = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        for i in range(M):
            yref = oracle.gemv(m, X[i], threads=THREADS)
            assert max_rel(y[i], yref, q8_floor(m, X[i])) <= 1e-3


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("M", [2, 3, 5, 8])
def test_gemv_small_batch_tails_bf16(eng, kind, M):
    """M = 2..8 with bf16 x at ragged shapes (cols % 8 != 0 takes the element-wise x path)."""
    for rows, cols in [(1, 1), (7, 129), (33, 257), (5, 544), (9, 2050)]:
        m = make(kind, rows, cols, seed=rows + cols + M)
        t = eng.upload_packed(m)
        xb = synth.make_x_bf16(M, cols, seed=cols + M)
        X = bf16_bits_to_f32(xb).reshape(M, cols)
        yf = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        yb = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16)
        yref = gemv_ref(m, X)
        fl = floor_scale(oracle.decode_rows(m), X)
        assert max_rel(yf, yref, fl) <= 1e-3, (rows, cols)
        assert_bf16_close(yb, yref, fl)
        yf2 = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        assert np.array_equal(yf.view(np.uint32), yf2.view(np.uint32)), "run-to-run bits"


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("M", [4, 8])
def test_gemv_small_batch_f32_x(eng, kind, M):
    for rows, cols in [(3, 100), (64, 2048), (16, 6144)]:
        m = make(kind, rows, cols, seed=rows * cols + M)
        t = eng.upload_packed(m)
        X = synth.make_x_f32(M, cols, seed=M)
        y = run_dev(eng, t, X, engine.DTYPE_F32, M, engine.DTYPE_F32)
        assert max_rel(y, gemv_ref(m, X), floor_scale(oracle.decode_rows(m), X)) <= 1e-3, (rows, cols)


@pytest.mark.parametrize("cols", [100, 2048, 2050, 4096])
def test_gemv_q8_many_rows_small_batch(eng, cols):
    """Row counts >= 65536 with M = 2..8: the persistent MFMA kernel where
    kp is a multiple of 512 (2048; 4096 on two staged K steps), the
    LDS-staged persistent dot2 kernel otherwise (100 -> kp 128, 2050 -> kp
    2080).  The last row tile is partial (65541 rows)."""
    m = synth.make_q8(65541, cols, seed=cols)
    t = eng.upload_packed(m)
    for M in (2, 3, 4, 5, 6, 7, 8):
        xb = synth.make_x_bf16(M, cols, seed=M)
        X = bf16_bits_to_f32(xb).reshape(M, cols)
        y = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        yb = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16)
        for i in range(M):
            yref = oracle.gemv(m, X[i], threads=THREADS)
            fl = q8_floor(m, X[i])
            assert max_rel(y[i], yref, fl) <= 1e-3, (M, i)
            assert_bf16_close(yb[i], yref, fl)
        y2 = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        assert np.array_equal(y.view(np.uint32), y2.view(np.uint32)), "run-to-run bits"


@pytest.mark.parametrize("M", [5, 6, 7, 8])
def test_gemv_q8_mfma_batch_edges(eng, M):
    """Q8 x bf16 at M = 5..8, cols % 8 == 0 and K <= 2048 (the MFMA kernel):
    row counts off the 16-row tile, cols off the 32-column block (pieces past
    cols read as zero), odd block counts (a pair without its second block),
    and more waves than block pairs (cols <= 96)."""
    for rows, cols in [(1, 8), (5, 40), (37, 136), (16, 96), (300, 2048), (77, 1032), (4099, 2048)]:
        m = synth.make_q8(rows, cols, seed=rows + cols + M)
        t = eng.upload_packed(m)
        xb = synth.make_x_bf16(M, cols, seed=cols + 7 * M)
        X = bf16_bits_to_f32(xb).reshape(M, cols)
        yf = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        yb = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16)
        yref = gemv_ref(m, X)
        fl = floor_scale(oracle.decode_rows(m), X)
        assert max_rel(yf, yref, fl) <= 1e-3, (rows, cols)
        assert_bf16_close(yb, yref, fl)
        yf2 = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        assert np.array_equal(yf.view(np.uint32), yf2.view(np.uint32)), "run-to-run bits"


@pytest.mark.parametrize("M", [5, 6, 7, 8])
def test_gemv_q8_mfma8_batch_edges(eng, M):
    """Q8 x bf16 at M = 5..8 with K > 4096 and <= 4096 rows (the 8-row MFMA
    kernel): row counts off the 8-row tile, cols off the 32-column block
    (pieces past cols read as zero), odd block counts (a pair without its
    second block) and the longest rows it takes (K = 8192, 256 blocks)."""
    for rows, cols in [(1, 4104), (13, 6144), (37, 5000), (2049, 6152), (4096, 8192)]:
        print(f"q8 mfma8 edges M={M} rows={rows} cols={cols}", flush=True)
        m = synth.make_q8(rows, cols, seed=rows + cols + M)
        t = eng.upload_packed(m)
        xb = synth.make_x_bf16(M, cols, seed=cols + 7 * M)
        X = bf16_bits_to_f32(xb).reshape(M, cols)
        yf = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        yb = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16)
        yref = gemv_ref(m, X)
        fl = floor_scale(oracle.decode_rows(m), X)
        assert max_rel(yf, yref, fl) <= 1e-3, (rows, cols)
        assert_bf16_close(yb, yref, fl)
        yf2 = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        assert np.array_equal(yf.view(np.uint32), yf2.view(np.uint32)), "run-to-run bits"
        t.free()


def test_gemv_deterministic_and_grouping_invariant(eng):
    for kind in ("cb4", "g64", "q8"):
        m = make(kind, 17, 513, seed=3)
        x = synth.make_x_f32(1, 513, seed=4)[0]
        t = eng.upload_packed(m)
        y1 = np.empty(17, np.float32)
        y2 = np.empty(17, np.float32)
        t.run_gemv(eng, x, y1)
        t.run_gemv(eng, x, y2)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
        # the first 5 rows as their own matrix give the same bits
        if kind == "q8":
            sub = synth.make_q8(17, 513, seed=3)
            sub.rows, sub.blocks = 5, sub.blocks[: 5 * sub.blocks_per_row * 34]
        elif kind == "g64":
            sub = synth.make_g64(17, 513, seed=3)
            sub.rows = 5
            sub.idx = sub.idx[: 5 * sub.padded_cols // 2]
            sub.lut_f16 = sub.lut_f16[: 5 * sub.padded_cols // 64 * 16]
        else:
            sub = synth.make_cb4(17, 513, seed=3)
            sub.rows = 5
            sub.scales_f16 = sub.scales_f16[: 5 * sub.padded_cols // 128]
            sub.packed_words = sub.packed_words[: 5 * sub.padded_cols // 8]
            sub.outlier_row_ptr = sub.outlier_row_ptr[:6]
            sub.outliers_packed = sub.outliers_packed[: int(sub.outlier_row_ptr[5])]
        y5 = np.empty(5, np.float32)
        eng.upload_packed(sub).run_gemv(eng, x, y5)
        assert np.array_equal(y5.view(np.uint32), y1[:5].view(np.uint32)), kind


def test_run_multi_same_x(eng):
    """metal.rs:466 / tensor_roundtrip_gemv.rs:284-300: one x, several tensors."""
    ms = [make(k, 97, 640, seed=i) for i, k in enumerate(["cb4", "g64", "q8", "cb4"])]
    ts = [eng.upload_packed(m) for m in ms]
    x = synth.make_x_f32(1, 640, seed=9)[0]
    ys = [np.empty(97, np.float32) for _ in ts]
    eng.run_multi_same_x(x, list(zip(ts, ys)))
    for m, t, y in zip(ms, ts, ys):
        y1 = np.empty(97, np.float32)
        t.run_gemv(eng, x, y1)
        assert np.array_equal(y.view(np.uint32), y1.view(np.uint32))


def test_clone_and_free(eng):
    m = make("g64", 64, 256, seed=1)
    t = eng.upload_packed(m)
    c = t.clone()
    x = synth.make_x_f32(1, 256, seed=1)[0]
    y1, y2 = np.empty(64, np.float32), np.empty(64, np.float32)
    t.run_gemv(eng, x, y1)
    t.free()
    c.run_gemv(eng, x, y2)
    assert np.array_equal(y1, y2)


def test_error_paths(eng):
    m = make("q8", 8, 64, seed=1)
    t = eng.upload_packed(m)
    with pytest.raises(engine.BackendError) as ei:
        eng.run_multi_same_x(np.zeros(32, np.float32), [(t, np.empty(8, np.float32))])
    assert ei.value.code == engine.VXT_E_SHAPE
    bad = synth.make_cb4(4, 256, seed=1)
    bad.packed_words = bad.packed_words[:-1]
    with pytest.raises(engine.BackendError) as ei:
        eng.upload_packed(bad)
    assert ei.value.code == engine.VXT_E_FORMAT
    with pytest.raises(engine.BackendError):
        eng.dequant_rows(t, 7, 2)
    with pytest.raises(engine.BackendError) as ei:
        eng.matmul_dev(t, 0, engine.DTYPE_F32, 1, 0, engine.DTYPE_F32)
    assert ei.value.code == engine.VXT_E_ARG


def test_graph_replays_match_eager(eng):
    """Captured GEMVs replayed several times, with eager work in between."""
    m = make("g64", 2048, 2048, seed=2)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(1, 2048, seed=2)
    xd = eng.to_device(xb)
    yd = eng.alloc(2048 * 4)
    eng.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 1, yd.ptr, engine.DTYPE_F32, eng.stream)
    eng.synchronize()
    ref = yd.download(np.float32, 2048)
    g = eng.capture(lambda s: [eng.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 1, yd.ptr,
                                              engine.DTYPE_F32, s) for _ in range(3)])
    other = eng.alloc(2048 * 4)
    for rep in range(4):
        yd.upload(np.full(2048, np.nan, np.float32))
        eng.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 1, other.ptr, engine.DTYPE_F32, eng.stream)
        g.launch(1 + rep)
        assert np.array_equal(yd.download(np.float32, 2048).view(np.uint32), ref.view(np.uint32)), rep
    g.free()


# ---------------------------------------------------------------- GEMM

def gemm_check(y, yref, W, X, bf16):
    fl = floor_scale(W, X)
    if bf16:
        assert_bf16_close(y, yref, fl)
    else:
        assert max_rel(y, yref, fl) <= 1e-3


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 33), (97, 130), (130, 257), (257, 544)])
@pytest.mark.parametrize("M", [9, 11, 64, 129])
def test_gemm_tail_shapes_host_api(eng, kind, rows, cols, M):
    m = make(kind, rows, cols, seed=rows + cols + M)
    t = eng.upload_packed(m)
    X = synth.make_x_f32(M, cols, seed=M)
    Y = eng.gemm(t, X)
    gemm_check(Y, oracle.gemm(m, X, threads=THREADS), oracle.decode_rows(m), X, False)


def test_gemm_matches_per_token_gemv_96x256x11(eng):
    """vxt_roadmap_steps.rs:210-230 on the device: gemm vs per-token gemv."""
    for kind in ("cb4", "g64", "q8"):
        m = make(kind, 96, 256, seed=901)
        t = eng.upload_packed(m)
        X = synth.make_x_f32(11, 256, seed=902)
        Yg = eng.gemm(t, X)
        Yv = np.stack([np.empty(96, np.float32) for _ in range(11)])
        for i in range(11):
            t.run_gemv(eng, X[i], Yv[i])
        a, b = Yg.astype(np.float64).ravel(), Yv.astype(np.float64).ravel()
        assert a @ b / (np.linalg.norm(a) * np.linalg.norm(b)) > 0.999999, kind


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("K,N", [(2048, 6144), (6144, 2048)])
@pytest.mark.parametrize("M", [128, 512, 1024, 2048])
def test_gemm_prefill_shapes_bf16(eng, kind, K, N, M):
    """Config 3: bf16 activations, fp32 accumulate, bf16 output (and f32);
    M = 1024 is between the config's batches (the planner's thresholds)."""
    m = make(kind, N, K, seed=K + M)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(M, K, seed=M)
    X = bf16_bits_to_f32(xb).reshape(M, K)
    yb = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_BF16)
    yf = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    # oracle on a token sample (tokens are independent rows of the product)
    sel = np.unique(np.r_[0, M - 1, np.random.default_rng(M).choice(M, 14, replace=False)])
    W = oracle.decode_rows(m)
    yref = oracle.gemm(m, X[sel], threads=THREADS)
    gemm_check(yb[sel], yref, W, X[sel], True)
    gemm_check(yf[sel], yref, W, X[sel], False)
    # every token: bf16 output is the rounding of the f32 output
    assert np.array_equal(yb, f32_to_bf16_bits(yf))


def test_gemm_extreme_weight_magnitudes(eng):
    """Weights far outside the f16 range (and subnormal scales) keep the GEMM bar:
    each panel row carries its own power-of-two scale."""
    q = synth.make_q8(70, 320, seed=3)
    b = q.blocks.copy().reshape(-1, 34)
    b[0::3, 0:2] = np.array([0x7800], np.uint16).view(np.uint8)   # d = 32768: |w| up to 4.2e6
    b[1::7, 0:2] = np.array([0x0001], np.uint16).view(np.uint8)   # subnormal d
    q.blocks = b.reshape(-1)
    c = synth.make_cb4(70, 320, seed=4, outlier_frac=0.02)
    c.scales_f16 = np.where(np.arange(c.scales_f16.size) % 2 == 0, np.uint16(0x7800), c.scales_f16)
    c.centroids = c.centroids * np.float32(500.0)
    for m in (q, c):
        t = eng.upload_packed(m)
        xb = synth.make_x_bf16(24, 320, seed=5)
        X = bf16_bits_to_f32(xb).reshape(24, 320)
        yref = oracle.gemm(m, X, threads=THREADS)
        W = oracle.decode_rows(m)
        gemm_check(run_dev(eng, t, xb, engine.DTYPE_BF16, 24, engine.DTYPE_F32), yref, W, X, False)
        gemm_check(run_dev(eng, t, xb, engine.DTYPE_BF16, 24, engine.DTYPE_BF16), yref, W, X, True)


@pytest.mark.parametrize("M", [16, 300])
def test_gemm_cb4_unsorted_and_duplicate_outliers(eng, M):
    """CSR rows in any order, with repeated columns (decode_row adds them in
    CSR order, codebook.rs:316-333): the panel decode takes its general path
    for such rows and the sorted fast path for the others."""
    m = synth.make_cb4(130, 2500, seed=9, outlier_frac=0.03)
    g = np.random.default_rng(9)
    rp, pk = m.outlier_row_ptr, m.outliers_packed
    rows = []
    for r in range(m.rows):
        e = pk[rp[r]:rp[r + 1]].copy()
        if r % 3 == 0 and e.size:        # shuffled, plus a second residual on two columns
            g.shuffle(e)
            extra = (e[:2] & np.uint32(0xFFFF)) | (np.uint32(f16b(0.0625)) << np.uint32(16))
            e = np.concatenate([e, extra])
        rows.append(e)
    m.outliers_packed = np.concatenate(rows).astype(np.uint32)
    m.outlier_row_ptr = np.r_[0, np.cumsum([len(e) for e in rows])].astype(np.uint32)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(M, m.cols, seed=M)
    X = bf16_bits_to_f32(xb).reshape(M, m.cols)
    W = oracle.decode_rows(m)
    sel = np.r_[0:4, M - 4:M]
    yref = oracle.gemm(m, X[sel], threads=THREADS)
    for path in (engine.GEMM_AUTO, engine.GEMM_PANEL):
        eng.set_gemm_path(path)
        try:
            y = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
        finally:
            eng.set_gemm_path(engine.GEMM_AUTO)
        gemm_check(y[sel], yref, W, X[sel], False)
    t.free()


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("M,N,K", [(16, 64, 4096), (40, 300, 3000), (9, 2048, 6144)])
def test_gemm_split_k(eng, kind, M, N, K):
    """Small M x N grids split K across workgroups; partial sums are added in a fixed order."""
    m = make(kind, N, K, seed=M + N)
    t = eng.upload_packed(m)
    xb = synth.make_x_bf16(M, K, seed=K)
    X = bf16_bits_to_f32(xb).reshape(M, K)
    yref = oracle.gemm(m, X, threads=THREADS)
    y1 = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    gemm_check(y1, yref, oracle.decode_rows(m), X, False)
    y2 = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("M,N,K,xdt", [(300, 130, 700, "bf16"), (257, 2048, 2048, "f32"), (1024, 96, 4096, "bf16")])
def test_gemm_library_dense_phase(eng, kind, M, N, K, xdt):
    """Two-phase GEMM with the dense phase on hipBLASLt (automatic above
    batch 256): hi/lo terms for cb4 and Q8, split f32 activations, the 1/s
    epilogue and bf16 rounding, against the oracle and the own dense kernel."""
    m = make(kind, N, K, seed=M + N + K)
    t = eng.upload_packed(m)
    if xdt == "bf16":
        xh = synth.make_x_bf16(M, K, seed=M)
        X = bf16_bits_to_f32(xh).reshape(M, K)
        xd = engine.DTYPE_BF16
    else:
        X = synth.make_x_f32(M, K, seed=M)
        xh, xd = X, engine.DTYPE_F32
    sel = np.r_[0:3, M // 2, M - 3:M]
    W = oracle.decode_rows(m)
    yref = oracle.gemm(m, X[sel], threads=THREADS)
    out = {}
    for path in (engine.GEMM_LIBRARY, engine.GEMM_PANEL):
        eng.set_gemm_path(path)
        try:
            out[path, 0] = run_dev(eng, t, xh, xd, M, engine.DTYPE_F32)
            out[path, 1] = run_dev(eng, t, xh, xd, M, engine.DTYPE_BF16)
        finally:
            eng.set_gemm_path(engine.GEMM_AUTO)
        gemm_check(out[path, 0][sel], yref, W, X[sel], False)
        gemm_check(out[path, 1][sel], yref, W, X[sel], True)
    assert np.array_equal(out[engine.GEMM_LIBRARY, 1], f32_to_bf16_bits(out[engine.GEMM_LIBRARY, 0]))
    t.free()


def test_gemm_library_in_captured_graph():
    """The library dense phase (pinned) records into a graph, also as a strided
    batch over K slices (K = 4096 at 300 x 640: four slices); every replay
    (with eager work and synchronisation between replays) matches the eager
    result."""
    e = engine.HipEngine()
    e.set_gemm_path(engine.GEMM_LIBRARY)
    try:
        for kind, cols, M in (("g64", 1024, 512), ("cb4", 1024, 512), ("g64", 4096, 300), ("q8", 4096, 300)):
            m = make(kind, 640, cols, seed=12)
            t = e.upload_packed(m)
            xd = e.to_device(synth.make_x_bf16(M, cols, seed=13))
            yd = e.alloc(M * 640 * 2)
            e.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, M, yd.ptr, engine.DTYPE_BF16, e.stream)
            e.synchronize()
            ref = yd.download(np.uint16, (M, 640))
            X = bf16_bits_to_f32(synth.make_x_bf16(M, cols, seed=13)).reshape(M, cols)
            assert_bf16_close(ref, gemv_ref(m, X), floor_scale(oracle.decode_rows(m), X))
            g = e.capture(lambda s: e.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, M, yd.ptr, engine.DTYPE_BF16, s))
            for rep in range(3):
                yd.upload(np.full((M, 640), 0x7FC0, np.uint16))
                g.launch(1)
                assert np.array_equal(yd.download(np.uint16, (M, 640)), ref), (kind, cols, rep)
                e.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, M, yd.ptr, engine.DTYPE_BF16, e.stream)
                e.synchronize()
            g.free()
            t.free()
            xd.free()
            yd.free()
    finally:
        e.close()


def test_gemm_in_captured_graph():
    """A GEMM records into a graph once its workspace is sized by an eager call."""
    e = engine.HipEngine()
    try:
        m = synth.make_q8(512, 1024, seed=8)
        t = e.upload_packed(m)
        xd = e.to_device(synth.make_x_bf16(64, 1024, seed=8))
        yd = e.alloc(64 * 512 * 4)
        with pytest.raises(engine.BackendError) as ei:
            e.capture(lambda s: e.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 64, yd.ptr, engine.DTYPE_F32, s))
        assert ei.value.code == engine.VXT_E_ARG
        e.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 64, yd.ptr, engine.DTYPE_F32, e.stream)
        e.synchronize()
        ref = yd.download(np.float32, (64, 512))
        g = e.capture(lambda s: e.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 64, yd.ptr, engine.DTYPE_F32, s))
        for rep in range(3):
            yd.upload(np.full((64, 512), np.nan, np.float32))
            g.launch(1)
            assert np.array_equal(yd.download(np.float32, (64, 512)).view(np.uint32), ref.view(np.uint32)), rep
            e.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 64, yd.ptr, engine.DTYPE_F32, e.stream)
            e.synchronize()
        g.free()
    finally:
        e.close()

@pytest.mark.parametrize("M", [1, 3, 24])
def test_cb4_zero_scale_group_with_nonfinite_x(eng, M):
    """codebook.rs:384-386: the CPU GEMV skips a 128-group whose scale is
    zero, so Inf / NaN activations inside such a group leave the row finite;
    batch_m <= 8 follows that per token.  The GEMM (batch_m > 8) follows
    gemm_cpu (llm_prefill.rs:156-255), which decodes the group to zeros and
    multiplies them: 0 * Inf is NaN there too."""
    m = synth.make_cb4(40, 512, seed=21, outlier_frac=0.0)
    sc = m.scales_f16.reshape(40, 4).copy()
    sc[::2, 1] = 0          # even rows: group 1 (columns 128..255) has scale 0
    sc[5, 1] = 0x8000       # row 5: -0, which is zero too
    m.scales_f16 = sc.reshape(-1)
    t = eng.upload_packed(m)
    X = synth.make_x_f32(M, 512, seed=M)
    X[:, 130] = np.inf      # both inside group 1
    X[:, 200] = np.nan
    xb = f32_to_bf16_bits(X)
    Xq = bf16_bits_to_f32(xb).reshape(M, 512)
    y = run_dev(eng, t, xb, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    if M <= 8:
        ref = np.stack([oracle.gemv(m, Xq[i], threads=THREADS) for i in range(M)])
    else:
        ref = oracle.gemm(m, Xq, threads=THREADS)
    fin = np.isfinite(ref)
    skipped = np.zeros(40, bool)
    skipped[::2] = True
    skipped[5] = True
    if M <= 8:
        assert np.array_equal(fin, np.broadcast_to(skipped, fin.shape))
    else:
        assert not fin.any()
    assert np.array_equal(np.isfinite(y), fin)
    W = oracle.decode_rows(m)
    Xf = np.where(np.isfinite(Xq), Xq, 0)
    fl = floor_scale(W, Xf)
    err = np.abs(y[fin].astype(np.float64) - ref[fin]) / np.maximum(np.abs(ref[fin]), fl[fin])
    assert err.size == 0 or err.max() <= 1e-3


@pytest.mark.parametrize("kind", ["cb4", "g64", "q8"])
@pytest.mark.parametrize("rows,cols", [(7, 4100), (300, 6144), (65, 9000)])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_gemv_split_k_shapes(eng, kind, rows, cols, xdt):
    """M = 1 with K of two or more 2048-column steps: 4100 and 9000 columns
    (x rows not 16-byte multiples, and more than three steps) take the
    split-K kernel where the kind allows it (the K steps of a row on separate
    waves, summed in wave order); 6144 columns with aligned rows take the
    one-token LDS-staged kernels (three K steps).  Ragged K, a few rows, cb4
    residuals anywhere in the row."""
    m = make(kind, rows, cols, seed=rows + cols)
    t = eng.upload_packed(m)
    if xdt == "bf16":
        xh = synth.make_x_bf16(1, cols, seed=3)
        X = bf16_bits_to_f32(xh).reshape(1, cols)
        y = run_dev(eng, t, xh, engine.DTYPE_BF16, 1, engine.DTYPE_F32)
    else:
        X = synth.make_x_f32(1, cols, seed=3)
        y = run_dev(eng, t, X, engine.DTYPE_F32, 1, engine.DTYPE_F32)
    ref = gemv_ref(m, X)
    assert max_rel(y, ref, floor_scale(oracle.decode_rows(m), X)) <= 1e-3
    y2 = run_dev(eng, t, xh if xdt == "bf16" else X, engine.DTYPE_BF16 if xdt == "bf16" else engine.DTYPE_F32, 1,
                 engine.DTYPE_F32)
    assert_bits_equal(y2, y)   # deterministic: the waves' sums are added in a fixed order


def _shuffled_duplicate_outliers(m, seed, every=3, extra=2):
    """Rows r % every == 0 get their CSR entries shuffled plus `extra` more
    residuals on columns they already hold (decode_row adds each in CSR
    order, codebook.rs:316-333; the GEMV adds each f16(res) * x[col])."""
    g = np.random.default_rng(seed)
    rp, pk = m.outlier_row_ptr, m.outliers_packed
    rows = []
    for r in range(m.rows):
        e = pk[rp[r]:rp[r + 1]].copy()
        if r % every == 0 and e.size:
            g.shuffle(e)
            add = (e[:extra] & np.uint32(0xFFFF)) | (np.uint32(f16b(0.0625)) << np.uint32(16))
            e = np.concatenate([e, add])
        rows.append(e)
    m.outliers_packed = np.concatenate(rows).astype(np.uint32)
    m.outlier_row_ptr = np.r_[0, np.cumsum([len(e) for e in rows])].astype(np.uint32)
    return m


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_gemv_cb4_unsorted_and_duplicate_outliers(eng, M, xdt):
    """The decode GEMV at every batch size on CSR rows in any order with
    repeated columns (llm_gpu_cpu_parity.rs:678-690's case at scale): the
    one-token LDS-staged kernel (aligned rows, 2304 columns) and the generic
    kernels add every entry, in any order, at the GEMV bar."""
    m = _shuffled_duplicate_outliers(synth.make_cb4(130, 2304, seed=31, outlier_frac=0.03), seed=31)
    t = eng.upload_packed(m)
    if xdt == "bf16":
        xh = synth.make_x_bf16(M, m.cols, seed=M)
        X = bf16_bits_to_f32(xh).reshape(M, m.cols)
        xd = engine.DTYPE_BF16
    else:
        X = synth.make_x_f32(M, m.cols, seed=M)
        xh, xd = X, engine.DTYPE_F32
    W = oracle.decode_rows(m)
    y = run_dev(eng, t, xh, xd, M, engine.DTYPE_F32)
    assert max_rel(y, gemv_ref(m, X), floor_scale(W, X)) <= 1e-3
    t.free()


@pytest.mark.parametrize("rows", [1, 5, 17])
@pytest.mark.parametrize("cols", [129, 513])
@pytest.mark.parametrize("M", [1, 2, 8])
def test_gemv_duplicate_column_fixture(eng, rows, cols, M):
    """The duplicate-column fixture of llm_gpu_cpu_parity.rs:680-688 (two
    residuals on column 0, one on the last column, every row) through the
    GEMV, against the oracle's gemv_cpu."""
    m = closed_form(rows, cols, lambda c: [f16b(0.25) << 16, f16b(-0.125) << 16,
                                           (f16b(0.5) << 16) | (c - 1)])
    t = eng.upload_packed(m)
    X = synth.make_x_f32(M, cols, seed=cols)
    y = run_dev(eng, t, X, engine.DTYPE_F32, M, engine.DTYPE_F32)
    assert max_rel(y, gemv_ref(m, X), floor_scale(oracle.decode_rows(m), X)) <= 1e-3
    t.free()


@pytest.mark.parametrize("M", [1, 2, 8])
def test_gemv_cb4_sink_row(eng, M):
    """A "sink" row holding thousands of residuals (the reference's encoder
    puts most of a tensor's outliers on a few rows, reports/cb4-v2-2026-11-08.md)
    next to ordinary rows: every lane walks many entries of that row."""
    m = synth.make_cb4(300, 6144, seed=33)
    g = np.random.default_rng(33)
    sink = np.sort(g.choice(6144, size=5000, replace=False)).astype(np.uint32)
    vals = f32_to_f16_bits(g.normal(0, 0.02, size=5000).astype(np.float32)).astype(np.uint32)
    rp, pk = m.outlier_row_ptr, m.outliers_packed
    r = 123
    m.outliers_packed = np.concatenate([pk[:rp[r]], sink | (vals << np.uint32(16)), pk[rp[r + 1]:]]).astype(np.uint32)
    cnt = np.diff(rp.astype(np.int64))
    cnt[r] = 5000
    m.outlier_row_ptr = np.r_[0, np.cumsum(cnt)].astype(np.uint32)
    t = eng.upload_packed(m)
    xh = synth.make_x_bf16(M, 6144, seed=M + 3)
    X = bf16_bits_to_f32(xh).reshape(M, 6144)
    y = run_dev(eng, t, xh, engine.DTYPE_BF16, M, engine.DTYPE_F32)
    assert max_rel(y, gemv_ref(m, X), floor_scale(oracle.decode_rows(m), X)) <= 1e-3
    t.free()
