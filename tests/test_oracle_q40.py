"""Pin the oracle's Q4_0 restatement (q4_0.rs:17-145) before trusting it.

==============================  ================================================
oracle function                 pinned by
==============================  ================================================
encode (q4_0.rs:17-64)          a hand-packed block (bytes and words written out
                                by hand); the floor(v / d + 8.5) rounding at
                                exact halves; zero blocks; NaN and inf weights
                                (Rust's saturating, NaN -> 0 `as i32`); ragged
                                cols; |decode(encode(w)) - w| <= d / 2
decode_row (q4_0.rs:77-97)      GGUF Q4_0 dequant (gguf.rs:211-221: 16 low
                                nibbles, then 16 high nibbles) written with
                                numpy over the same bytes, bit for bit
gemv (q4_0.rs:109-145)          unit vectors e_c give decode_row's column c
                                exactly; fp64 bound K * 2^-23 * sum|wx|; a
                                cancellation case whose answer is fixed by the
                                (j, j + 16) chain order; 1- vs 4-thread identity
gemm via decode_row             equals per-token gemv within the fp64 bound
==============================  ================================================
"""
import numpy as np
import pytest

import oracle
from vxg_amd.formats import FormatError, Q4_0Matrix


def _block_matrix(rows, cols, scales, words):
    m = Q4_0Matrix(rows, cols, (cols + 31) // 32 * 32, np.asarray(scales, np.uint16),
                   np.asarray(words, np.uint32))
    m.validate()
    return m


def test_encode_hand_packed_block():
    # q[j] = j % 15 + 1 over one 32-column block, d = 1/16: w = (q - 8) / 16,
    # amax = 7/16 so d = amax / 7 = 1/16 exactly (f16 0x2c00).
    q = np.array([j % 15 + 1 for j in range(32)])
    w = ((q - 8) / 16.0).astype(np.float32).reshape(1, 32)
    m = oracle.q40_encode(1, 32, w)
    assert m.scales_f16.tolist() == [0x2C00]
    # byte j = q[j] | q[j + 16] << 4: q[0..3] = 1, 2, 3, 4 and q[16..19] = 2, 3, 4, 5
    assert int(m.qs_words[0]) == 0x54433221
    # q[12..15] = 13, 14, 15, 1 and q[28..31] = 14, 15, 1, 2: bytes ED FE 1F 21
    assert int(m.qs_words[3]) == 0x211FFEED
    np.testing.assert_array_equal(oracle.decode_rows(m), w)


def test_encode_rounds_half_up():
    # amax = 7 -> d = 1: v + 8.5 floored, so halves round toward +inf
    v = np.zeros(32, np.float32)
    v[0] = 7.0
    v[1:9] = [0.5, -0.5, 2.5, -2.5, 0.49, -0.51, 6.5, -6.5]
    m = oracle.q40_encode(1, 32, v.reshape(1, 32))
    d = oracle.decode_rows(m)[0]
    np.testing.assert_array_equal(d[:9], [7.0, 1.0, 0.0, 3.0, -2.0, 0.0, -1.0, 7.0, -6.0])


def test_encode_zero_block_and_ragged_cols():
    w = np.zeros((2, 40), np.float32)
    w[1, 33] = -3.5
    m = oracle.q40_encode(2, 40, w)
    assert m.padded_cols == 64 and m.scales_f16.size == 4
    # zero blocks: d = 0, id = 0, every q = floor(8.5) = 8 -> bytes 0x88
    assert m.scales_f16[0] == 0 and (m.qs_words[0:4] == 0x88888888).all()
    # block 1 of row 1: amax = 3.5 -> d = 0.5; padding columns (>= 40) encode 0 -> q = 8
    assert m.scales_f16[3] == 0x3800
    d = oracle.decode_rows(m)
    np.testing.assert_array_equal(d, w)


def test_encode_nan_and_inf_follow_rust_casts():
    v = np.zeros(32, np.float32)
    v[0], v[1] = np.nan, 7.0
    d = oracle.decode_rows(oracle.q40_encode(1, 32, v.reshape(1, 32)))[0]
    # NaN is skipped by the amax compare; NaN * id + 8.5 -> `as i32` = 0 -> q = 0 -> -8 d
    assert d[0] == -8.0 and d[1] == 7.0 and (d[2:] == 0).all()
    v = np.zeros(32, np.float32)
    v[3] = np.inf
    m = oracle.q40_encode(1, 32, v.reshape(1, 32))
    # amax = inf -> d = f16 inf, id = 1 / inf = 0; inf * 0 = NaN -> q = 0; others q = 8
    assert m.scales_f16[0] == 0x7C00
    b = m.qs_words.view(np.uint8)
    assert (b[3] & 0xF) == 0 and (b[np.arange(16) != 3] == 0x88).all()
    d = oracle.decode_rows(m)[0]
    assert d[3] == -np.inf and np.isnan(np.delete(d, 3)).all()   # (q-8)*inf: 0*inf = NaN


def test_encode_error_within_half_step():
    g = np.random.default_rng(5)
    w = g.normal(0, 1, (16, 96)).astype(np.float32)
    m = oracle.q40_encode(16, 96, w)
    d = oracle.decode_rows(m)
    step = oracle.f16_to_f32(m.scales_f16).reshape(16, 3)
    err = np.abs(d - w).reshape(16, 3, 32)
    assert (err <= step[:, :, None] * (0.5 + 1e-6)).all()


def _gguf_dequant(m):
    """gguf.rs:211-221 over the same bytes: 16 low nibbles, then 16 high nibbles."""
    b = m.gguf_blocks().reshape(-1, 18)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    qs = b[:, 2:18].astype(np.int32)
    vals = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=1).astype(np.float32) * d
    return vals.reshape(m.rows, -1)[:, :m.cols]


def test_decode_row_matches_gguf_dequant():
    g = np.random.default_rng(7)
    rows, cols = 9, 96
    sc = oracle.f32_to_f16(g.uniform(1e-3, 2.0, rows * 3).astype(np.float32))
    sc[4] = 0x0001          # subnormal scale
    sc[5] = 0x8400          # negative scale
    words = g.integers(0, 2**32, rows * 3 * 4, dtype=np.uint64).astype(np.uint32)
    m = _block_matrix(rows, cols, sc, words)
    np.testing.assert_array_equal(oracle.decode_rows(m), _gguf_dequant(m))
    m2 = Q4_0Matrix.from_gguf_blocks(rows, cols, m.gguf_blocks())
    assert (m2.scales_f16 == m.scales_f16).all() and (m2.qs_words == m.qs_words).all()


def test_gemv_unit_vectors_give_columns():
    g = np.random.default_rng(11)
    rows, cols = 5, 70
    m = oracle.q40_encode(rows, cols, g.normal(0, 1, (rows, cols)).astype(np.float32))
    dec = oracle.decode_rows(m)
    for c in (0, 1, 15, 16, 17, 31, 32, 47, 48, 69):
        e = np.zeros(cols, np.float32)
        e[c] = 1.0
        np.testing.assert_array_equal(oracle.gemv(m, e), dec[:, c])


def test_gemv_fp64_bound_and_threads():
    g = np.random.default_rng(13)
    rows, cols = 64, 1000
    m = oracle.q40_encode(rows, cols, g.normal(0, 0.02, (rows, cols)).astype(np.float32))
    x = g.normal(0, 1, cols).astype(np.float32)
    y1 = oracle.gemv(m, x, threads=1)
    y4 = oracle.gemv(m, x, threads=4)
    np.testing.assert_array_equal(y1, y4)
    dec = oracle.decode_rows(m).astype(np.float64)
    ref = dec @ x.astype(np.float64)
    bound = cols * 2.0**-23 * (np.abs(dec) @ np.abs(x.astype(np.float64)))
    assert (np.abs(y1 - ref) <= bound).all()


def test_gemv_chain_order_j_then_j_plus_16():
    # every q = 9 (weight 1 * d, d = 1): the chain visits x[0], x[16], x[1], ...
    # x[0] = 2^24, x[16] = 1, x[1] = -2^24: 2^24 + 1 rounds back to 2^24 before
    # x[1] cancels it, so the chain gives 0 (column order 0, 1, ..., 16 gives 1)
    m = _block_matrix(1, 32, [0x3C00], [0x99999999] * 4)
    x = np.zeros(32, np.float32)
    x[0], x[16], x[1] = 2.0**24, 1.0, -(2.0**24)
    assert oracle.gemv(m, x)[0] == 0.0
    x2 = x.copy()
    x2[16], x2[2] = 0.0, 1.0      # the 1 now comes after the cancellation
    assert oracle.gemv(m, x2)[0] == 1.0


def test_gemm_matches_gemv():
    g = np.random.default_rng(17)
    rows, cols, M = 40, 200, 5
    m = oracle.q40_encode(rows, cols, g.normal(0, 0.02, (rows, cols)).astype(np.float32))
    X = g.normal(0, 1, (M, cols)).astype(np.float32)
    Y = oracle.gemm(m, X, threads=4)
    Yv = oracle.gemv_batch(m, X)
    dec = oracle.decode_rows(m).astype(np.float64)
    bound = cols * 2.0**-23 * (np.abs(X.astype(np.float64)) @ np.abs(dec).T)
    assert (np.abs(Y - Yv) <= 2 * bound).all()
    assert (np.abs(Y - X.astype(np.float64) @ dec.T) <= bound).all()


def test_validate_rules():
    with pytest.raises(FormatError, match="padded_cols"):
        Q4_0Matrix(1, 40, 40, np.zeros(2, np.uint16), np.zeros(8, np.uint32)).validate()
    with pytest.raises(FormatError, match="plane lengths"):
        Q4_0Matrix(1, 40, 64, np.zeros(1, np.uint16), np.zeros(8, np.uint32)).validate()
