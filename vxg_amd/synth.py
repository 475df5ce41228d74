"""Seeded synthetic weights and activations for the benchmark configurations.

The reference generates its bench/test inputs from seeded generators
(SplitMix64 + Irwin-Hall normals, ``crates/vxg-tensor/src/bench.rs:17-71,
464-490``).  Packed layouts here are drawn directly in their compressed form,
as the benchmark configurations specify, with numpy's PCG64 generator:

* Q8 (configs 0, 2, 3, 4 LM head): int8 uniform in [-127, 127] in blocks of
  32 along K, one fp16 scale per block uniform in [0.002, 0.02].
* cb4-g64 (configs 1, 3, 4): 4-bit indices uniform in 0..15, and per
  64-group a 16-entry fp16 codebook drawn from N(0, 0.02) and sorted.
* cb4 reference layout: 16 sorted f32 centroids from N(0, 1), per-128-group
  fp16 scales uniform in [0.002, 0.02], and ~0.74 % CSR outliers at ascending
  columns with f16(N(0, 0.02)) residuals (the reference encoder's outlier
  fraction, ``cb4_opt.rs:132``'s 0.0074 target).
* Q4_0 (the secondary line at config 1's shape): nibbles uniform in 0..15
  (values q - 8), one fp16 scale per block of 32 uniform in [0.002, 0.02].
* Activations: f32 or bf16 N(0, 1).
"""
from __future__ import annotations

import numpy as np

from .formats import (Cb4G64Matrix, CodebookMatrix, Q4_0Matrix, Q8Matrix, f32_to_bf16_bits,
                      f32_to_f16_bits, q8_from_planes)


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def make_q8(rows: int, cols: int, seed: int = 0) -> Q8Matrix:
    g = rng(seed)
    kb = (cols + 31) // 32
    qs = g.integers(-127, 128, size=(rows, kb * 32), dtype=np.int8)
    if kb * 32 != cols:
        qs[:, cols:] = 0
    d = f32_to_f16_bits(g.uniform(0.002, 0.02, size=rows * kb).astype(np.float32))
    return q8_from_planes(rows, cols, qs, d)


def make_q40(rows: int, cols: int, seed: int = 3) -> Q4_0Matrix:
    g = rng(seed)
    kb = (cols + 31) // 32
    words = g.integers(0, 2**32, size=rows * kb * 4, dtype=np.uint64).astype(np.uint32)
    if kb * 32 != cols:
        # padding columns carry q = 8 (value 0); x is zero there in every consumer
        b = words.view(np.uint8).reshape(rows, kb * 16)
        for c in range(cols, kb * 32):
            j = (kb - 1) * 16 + (c % 32) % 16
            b[:, j] = (b[:, j] & np.uint8(0xF0)) | np.uint8(8) if c % 32 < 16 else (b[:, j] & np.uint8(0x0F)) | np.uint8(0x80)
    d = f32_to_f16_bits(g.uniform(0.002, 0.02, size=rows * kb).astype(np.float32))
    return Q4_0Matrix(rows, cols, kb * 32, d, words)


def make_g64(rows: int, cols: int, seed: int = 1) -> Cb4G64Matrix:
    g = rng(seed)
    kp = (cols + 63) // 64 * 64
    groups = rows * (kp // 64)
    idx = g.integers(0, 256, size=rows * kp // 2, dtype=np.uint8)
    if kp != cols:
        # Padding columns carry index 0; x is zero there in every consumer.
        idx2 = idx.reshape(rows, kp // 2)
        for c in range(cols, kp):
            idx2[:, c // 2] &= np.uint8(0xF0 if c % 2 == 0 else 0x0F)
    lut = np.sort(g.standard_normal(size=(groups, 16), dtype=np.float32) * np.float32(0.02), axis=1)
    lut_f16 = f32_to_f16_bits(lut).reshape(-1)
    return Cb4G64Matrix(rows, cols, kp, idx, lut_f16)


def make_cb4(rows: int, cols: int, seed: int = 2, outlier_frac: float = 0.0074,
             pad_to: int = 256, centred: bool = False) -> CodebookMatrix:
    """Reference cb4 layout.  ``centred``: subtract the table's mean from the
    16 centroids.  A shared table with a non-zero mean gives every row the same
    bias, so a long chain of projections with no norms between them (the
    matmul-only decode stack) grows the activations' common part by about
    0.01 * mean * K per projection until it overflows; a centred table keeps
    such a chain in range."""
    g = rng(seed)
    kp = (cols + pad_to - 1) // pad_to * pad_to
    cent = np.sort(g.normal(0.0, 1.0, size=16).astype(np.float32))
    if centred:
        cent = np.sort((cent - cent.mean()).astype(np.float32))
    scales = f32_to_f16_bits(g.uniform(0.002, 0.02, size=rows * (kp // 128)).astype(np.float32))
    words = g.integers(0, 2**32, size=rows * kp // 8, dtype=np.uint64).astype(np.uint32)
    counts = g.binomial(cols, outlier_frac, size=rows).astype(np.int64)
    row_ptr = np.zeros(rows + 1, dtype=np.uint32)
    row_ptr[1:] = np.cumsum(counts).astype(np.uint32)
    nnz = int(row_ptr[-1])
    packed = np.empty(nnz, dtype=np.uint32)
    res = f32_to_f16_bits(g.normal(0.0, 0.02, size=nnz).astype(np.float32)).astype(np.uint32)
    pos = 0
    for r in range(rows):
        n = int(counts[r])
        if n:
            colsel = np.sort(g.choice(cols, size=n, replace=False)).astype(np.uint32)
            packed[pos:pos + n] = colsel | (res[pos:pos + n] << 16)
            pos += n
    return CodebookMatrix(rows, cols, kp, cent, scales, words, row_ptr, packed)


def make_x_f32(m: int, k: int, seed: int = 0) -> np.ndarray:
    return rng(seed + 1000).standard_normal(size=(m, k), dtype=np.float32)


def make_x_bf16(m: int, k: int, seed: int = 0) -> np.ndarray:
    """bf16 bits (uint16) of N(0, 1) activations."""
    return f32_to_bf16_bits(make_x_f32(m, k, seed)).reshape(m, k)
