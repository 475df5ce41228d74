"""Shared helpers of the GPU parity tests: device round trips and the error bars.

Relative error of an output is measured against max(|y_ref|, 2^-10 * sum_c
|w_c x_c|), so outputs that cancel to near zero are judged on the scale of
their terms; bf16 outputs must sit within 1 bf16 ulp of f32_to_bf16(y_ref).
"""
import os

import numpy as np

import oracle
from vxg_amd import engine, synth
from vxg_amd.formats import CodebookMatrix, bf16_bits_to_f32, f32_to_bf16_bits, f32_to_f16_bits

THREADS = min(os.cpu_count() or 1, 16)
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def run_dev(eng, t, x_host, x_dtype, M, y_dtype):
    """matmul_dev with engine-owned device buffers; returns the host result."""
    xd = eng.to_device(x_host)
    ybytes = M * t.rows * (4 if y_dtype == engine.DTYPE_F32 else 2)
    yd = eng.alloc(ybytes)
    eng.matmul_dev(t, xd.ptr, x_dtype, M, yd.ptr, y_dtype, eng.stream)
    eng.synchronize()
    out = yd.download(np.float32 if y_dtype == engine.DTYPE_F32 else np.uint16, (M, t.rows))
    xd.free()
    yd.free()
    return out


def make(kind, rows, cols, seed):
    if kind == "q8":
        return synth.make_q8(rows, cols, seed=seed)
    if kind == "g64":
        return synth.make_g64(rows, cols, seed=seed)
    return synth.make_cb4(rows, cols, seed=seed, outlier_frac=0.0074)


def floor_scale(W, X):
    """2^-10 * sum_c |w_rc x_mc| as [M, rows]."""
    return 2.0 ** -10 * (np.abs(X.astype(np.float64)) @ np.abs(W.astype(np.float64)).T)


def q8_floor(m, x):
    """2^-10 * sum_c |w_rc x_c| for a Q8 matrix, computed in row chunks."""
    kb = m.blocks_per_row
    xa = np.zeros(kb * 32, np.float32)
    xa[: m.cols] = np.abs(x)
    xa = xa.reshape(kb, 32)
    d = np.abs(m.scales_f16().view(np.float16).astype(np.float32)).reshape(m.rows, kb)
    qs = m.qs().reshape(m.rows, kb, 32)
    out = np.empty(m.rows, np.float64)
    for r0 in range(0, m.rows, 8192):
        q = np.abs(qs[r0:r0 + 8192].astype(np.float32))
        out[r0:r0 + 8192] = ((q * xa[None]).sum(-1) * d[r0:r0 + 8192]).sum(-1)
    return 2.0 ** -10 * out


def max_rel(y, yref, floor):
    y = np.asarray(y, np.float64)
    yref = np.asarray(yref, np.float64)
    return float(np.max(np.abs(y - yref) / np.maximum(np.abs(yref), floor)))


def assert_bf16_close(y_bits, yref, floor):
    a = y_bits.astype(np.int32)
    b = f32_to_bf16_bits(yref.astype(np.float32)).astype(np.int32)
    # map sign-magnitude bf16 to a monotone integer line
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    ulps = np.abs(a - b)
    near_zero = np.abs(bf16_bits_to_f32(y_bits) - yref) <= 1e-3 * floor
    assert np.all((ulps <= 1) | near_zero), int(ulps.max())


def assert_bits_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    assert np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan])


def gemv_ref(m, X):
    return np.stack([oracle.gemv(m, X[i], threads=THREADS) for i in range(X.shape[0])])


# metal_llm_tests.rs:95-117: 515 logits of -3 with the edits below; the
# answers follow from llm_ops.rs:318-327 (strict > from -inf, first index).
GREEDY_REFERENCE_CASES = [
    # (edits, fill, expected id, expected nonfinite)
    ({257: 9.0, 513: 9.0}, -3.0, 257, False),
    ({514: 0.0}, -0.0, 0, False),                 # -0 == +0: index 0 stays
    ({}, -np.inf, 0, True),                       # nothing above -inf
    ({7: np.nan, 514: 4.0}, -3.0, 514, True),     # NaN never wins
    ({300: np.inf, 2: np.inf}, -3.0, 2, True),    # equal +inf: lower index
    ({}, np.nan, 0, True),
]


def greedy_reference_logits(case):
    edits, fill, _, _ = case
    a = np.full(515, fill, dtype=np.float32)
    for i, v in edits.items():
        a[i] = v
    return a


# metal_llm_tests.rs:31-58: the closed-form cb4 matrix of the reference's
# embedding probe; packed_fn(cols) gives each row's packed outliers.
def closed_form(rows, cols, packed_fn):
    padded = (cols + 127) // 128 * 128
    groups = padded // 128
    cent = ((np.arange(16, dtype=np.float32) - np.float32(7.5)) * np.float32(0.1234567)).astype(np.float32)
    scales = f32_to_f16_bits(np.float32(0.125) + (np.arange(rows * groups) % 11).astype(np.float32) * np.float32(0.25))
    rot = np.array([((0x76543210 << s) | (0x76543210 >> (32 - s))) & 0xFFFFFFFF if s else 0x76543210
                    for s in range(0, 32, 4)], dtype=np.uint64).astype(np.uint32)
    words = rot[np.arange(rows * groups * 16) % 8]
    packed = np.array([x for _ in range(rows) for x in packed_fn(cols)], np.uint32)
    row_ptr = np.arange(0, packed.size + 1, packed.size // rows if rows else 1, dtype=np.uint32)
    return CodebookMatrix(rows, cols, padded, cent, scales, words, row_ptr, packed)


def f16b(v):
    return int(f32_to_f16_bits(np.array([v], np.float32))[0])
