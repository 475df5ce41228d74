"""Write the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

The reference cannot be compiled or imported here (no Rust toolchain), so the
fixtures restate the known-answer inputs that the reference's own tests use and
compute the expected outputs with an implementation independent of the C
oracle: vectorised numpy over the documented bit layout (numpy's IEEE float16
widening, float32 multiplies, sequential float32 adds).  The C oracle is then
checked against these files bit for bit.

Fixtures:

* ``f16_boundaries.json`` -- the f32 -> f16 subnormal rounding table of
  ``crates/vxg-tensor/src/fp16.rs:89-108`` (both signs).
* ``cb4_closed_form.npz`` -- ``metal_llm_tests.rs:31-58``: rows = 515,
  cols in {1, 129, 257, 385}, padded_cols = roundup(cols, 128),
  ``centroids[i] = (i - 7.5) * 0.1234567``,
  ``scales[i] = f16(0.125 + (i % 11) * 0.25)``,
  ``words[i] = 0x76543210.rotate_left((i % 8) * 4)``, and three outliers per
  row on column cols-1 (0.33325195, -0.125, 0.0009765625).  Expected:
  ``decode_row`` of rows 0, 1 and 514 (the tokens the reference checks).
* ``cb4_dup_outlier.npz`` -- the CSR of ``llm_gpu_cpu_parity.rs:680-688``
  (per row: col 0 += 0.25, col 0 += -0.125, col cols-1 += 0.5) on closed-form
  base planes (the reference draws its base planes from its encoder, which
  is off the device path), rows in {1,3,4,5,7,9,17}, cols in {1,129,257,513}.
  Expected: every decoded row.
"""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f32_bits(v: float) -> int:
    return int(np.array([v], dtype=np.float32).view(np.uint32)[0])


def f16_np(v: float) -> int:
    return int(np.array([v], dtype=np.float32).astype(np.float16).view(np.uint16)[0])


def f16_boundaries():
    """fp16.rs:89-108.  Expected f16 bits are the reference test's literals."""
    midpoint = 2.0 ** -25
    mid_bits = f32_bits(midpoint)
    sub_max = float(np.array([0x03FF], dtype=np.uint16).view(np.float16).astype(np.float32)[0])
    cases = [
        (f32_bits(0.0), 0),
        (1, 0),                                           # f32::from_bits(1)
        (mid_bits - 1, 0),
        (mid_bits, 0),
        (mid_bits + 1, 1),
        (f32_bits(0.75 * 2.0 ** -24), 1),
        (f32_bits(2.0 ** -24), 1),
        (f32_bits(3.0 * midpoint), 2),
        (f32_bits(5.0 * midpoint), 2),
        (f32_bits(np.float32(sub_max) + np.float32(midpoint)), 0x0400),
    ]
    out = []
    for bits, exp in cases:
        out.append({"f32_bits": bits, "f16_bits": exp})
        out.append({"f32_bits": bits | 0x80000000, "f16_bits": 0x8000 | exp})
    return out


def rotl32(x: int, s: int) -> int:
    s %= 32
    return ((x << s) | (x >> (32 - s))) & 0xFFFFFFFF if s else x


def closed_form_planes(rows: int, cols: int):
    padded = (cols + 127) // 128 * 128
    groups = padded // 128
    cent = ((np.arange(16, dtype=np.float32) - np.float32(7.5)) * np.float32(0.1234567)).astype(np.float32)
    sc_f32 = (np.float32(0.125) + (np.arange(rows * groups) % 11).astype(np.float32) * np.float32(0.25))
    scales = sc_f32.astype(np.float32).astype(np.float16).view(np.uint16)
    n_words = rows * groups * 16
    rot = np.array([rotl32(0x76543210, (i % 8) * 4) for i in range(8)], dtype=np.uint32)
    words = rot[np.arange(n_words) % 8]
    return padded, cent, scales, words


def decode_numpy(rows, cols, padded, cent, scales, words, row_ptr, packed):
    """Independent dense decode: nibble c%8 of word c/8, scale c/128, then CSR adds."""
    wpr = padded // 8
    gpr = padded // 128
    w = words.reshape(rows, wpr)
    c = np.arange(cols)
    q = (w[:, c // 8] >> ((c % 8) * 4).astype(np.uint32)) & 0xF
    sc = scales.view(np.float16).astype(np.float32).reshape(rows, gpr)[:, c // 128]
    dense = (sc * cent[q]).astype(np.float32)          # one f32 rounding per element
    for r in range(rows):
        for i in range(int(row_ptr[r]), int(row_ptr[r + 1])):
            col = int(packed[i]) & 0xFFFF
            res = np.array([int(packed[i]) >> 16], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
            if col < cols:
                dense[r, col] = np.float32(dense[r, col] + res)
    return dense


def cb4_closed_form():
    out = {}
    for cols in (1, 129, 257, 385):
        rows = 515
        padded, cent, scales, words = closed_form_planes(rows, cols)
        vals = [0.33325195, -0.125, 0.0009765625]
        row_ptr = np.arange(0, 3 * rows + 1, 3, dtype=np.uint32)
        packed = np.array([(f16_np(v) << 16) | (cols - 1) for _ in range(rows) for v in vals],
                          dtype=np.uint32)
        dense = decode_numpy(rows, cols, padded, cent, scales, words, row_ptr, packed)
        out[f"c{cols}_rows"] = np.array([0, 1, 514], dtype=np.int64)
        out[f"c{cols}_expected"] = dense[[0, 1, 514]]
    return out


def cb4_dup_outlier():
    out = {}
    for rows in (1, 3, 4, 5, 7, 9, 17):
        for cols in (1, 129, 257, 513):
            padded, cent, scales, words = closed_form_planes(rows, cols)
            row_ptr = np.arange(0, 3 * rows + 1, 3, dtype=np.uint32)
            packed = np.array([x for _ in range(rows) for x in (
                f16_np(0.25) << 16, f16_np(-0.125) << 16, (f16_np(0.5) << 16) | (cols - 1))],
                dtype=np.uint32)
            dense = decode_numpy(rows, cols, padded, cent, scales, words, row_ptr, packed)
            out[f"r{rows}_c{cols}"] = dense
    return out


def main():
    with open(os.path.join(HERE, "f16_boundaries.json"), "w") as f:
        json.dump({"source": "crates/vxg-tensor/src/fp16.rs:89-108", "cases": f16_boundaries()},
                  f, indent=1)
    np.savez_compressed(os.path.join(HERE, "cb4_closed_form.npz"), **cb4_closed_form())
    np.savez_compressed(os.path.join(HERE, "cb4_dup_outlier.npz"), **cb4_dup_outlier())


if __name__ == "__main__":
    main()
