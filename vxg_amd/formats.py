"""Host-side weight containers for the compressed-weight matmul path.

These mirror the reference's Rust types field for field so that a caller
holding a ``CodebookMatrix`` (or raw GGUF ``Q8_0`` bytes) can hand it to
:class:`vxg_amd.engine.HipEngine` unchanged:

* :class:`CodebookMatrix` -- ``crates/vxg-tensor/src/codebook.rs:9-24`` with
  ``bits == 4`` ("cb4"): 4-bit indices, 8 per little-endian ``u32`` along K,
  one f16 scale per 128-wide K group, one global 16-entry f32 centroid table,
  and a CSR stream of f16 residual outliers.  :meth:`CodebookMatrix.validate`
  applies the archive reader's checks (``format.rs:421-451``, ``:565-574``).
* :class:`Cb4G64Matrix` -- the decode-benchmark cb4 layout: groups of 64 along
  K, one 16-entry fp16 codebook per (row, group), indices packed two per byte
  (low nibble = even column), no scale and no outliers.  It has no Rust
  counterpart; its nibble packing is the reference's.
* :class:`Q8Matrix` -- rows of 34-byte ``{f16 d; i8 qs[32]}`` blocks, the
  byte layout of ``KvQ8Block`` (``llm_prefill.rs:17-24``) and of GGUF
  ``Q8_0`` (``gguf.rs:223-229``), as ``GgufView::tensor_bytes``
  (``gguf.rs:160-172``) returns them.
* :class:`Q4_0Matrix` -- ``crates/vxg-tensor/src/q4_0.rs:7-14``: blocks of 32
  columns, one f16 scale and four little-endian ``u32`` words (16 bytes) per
  block; byte j holds column j in its low nibble and column j + 16 in its
  high nibble, value ``(q - 8) * d``.  GGUF ``Q4_0`` blocks (``gguf.rs:211-221``)
  carry the same bytes as ``{f16 d; u8 qs[16]}``.

Everything here is plain numpy; no device work happens in this module.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Union

import numpy as np


class FormatError(ValueError):
    """Corrupt or inconsistent planes (the reference's ``Error::Format``)."""


# ---------------------------------------------------------------------------
# Vectorised fp16 / bf16 conversions (host side, numpy).
# ---------------------------------------------------------------------------

def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bits, quiet-NaN preserving.

    Same rule as ``fp16.rs:113-120``: add ``0x7fff + lsb`` and keep the top
    half; NaNs keep their top half with the quiet bit forced on.
    """
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    lsb = (b >> 16) & 1
    out = ((b + np.uint32(0x7FFF) + lsb) >> 16).astype(np.uint16)
    nan = ((b & 0x7F800000) == 0x7F800000) & ((b & 0x007FFFFF) != 0)
    if nan.any():
        out[nan] = ((b[nan] >> 16) | 0x0040).astype(np.uint16)
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact bf16 -> f32 widening (``fp16.rs:81-83``)."""
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_f16_bits(a: np.ndarray) -> np.ndarray:
    """f32 -> IEEE binary16 bits, round-to-nearest-even (numpy's cast)."""
    return np.ascontiguousarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact binary16 -> f32 widening."""
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------
# Containers
# ---------------------------------------------------------------------------

@dataclass
class CodebookMatrix:
    """``CodebookMatrix`` with ``bits == 4`` (``codebook.rs:9-24``).

    ``packed_words[r * padded_cols/8 + c/8]`` holds column ``c`` in nibble
    ``c % 8``; ``scales_f16[r * padded_cols/128 + c/128]``;
    ``outliers_packed[i] = col | f16_residual << 16`` for the CSR range
    ``outlier_row_ptr[r] .. outlier_row_ptr[r+1]``.
    """

    rows: int
    cols: int
    padded_cols: int
    centroids: np.ndarray        # f32[16]
    scales_f16: np.ndarray       # u16[rows * padded_cols/128]
    packed_words: np.ndarray     # u32[rows * padded_cols/8]
    outlier_row_ptr: np.ndarray  # u32[rows + 1]
    outliers_packed: np.ndarray  # u32[nnz]
    bits: int = 4

    def validate(self) -> None:
        """Plane-length and CSR checks of the archive reader.

        ``format.rs:423-440`` (header, plane lengths, terminal pointer) and
        ``format.rs:565-574`` (monotone CSR, in-range columns).  The archive
        requires ``padded_cols == roundup(cols, 256)``; the in-memory type (and
        the reference's own GPU test fixture, ``metal_llm_tests.rs:33``) also
        uses ``roundup(cols, 128)``, so any multiple of 128 >= cols is accepted.
        """
        if self.bits != 4:
            raise FormatError("only bits == 4 (cb4) is on the device path")
        if self.rows <= 0 or self.cols <= 0:
            raise FormatError("rows and cols must be positive")
        if self.padded_cols < self.cols or self.padded_cols % 128 != 0:
            raise FormatError("invalid codebook padded_cols")
        groups = self.rows * (self.padded_cols // 128)
        c = np.asarray(self.centroids)
        if c.shape != (16,):
            raise FormatError("centroids must hold 16 f32 entries")
        rp = np.asarray(self.outlier_row_ptr)
        op = np.asarray(self.outliers_packed)
        if (np.asarray(self.scales_f16).size != groups
                or np.asarray(self.packed_words).size != groups * 4 * self.bits
                or rp.size != self.rows + 1
                or int(rp[-1]) != op.size):
            raise FormatError("corrupt VXT codebook plane lengths")
        if (int(rp[0]) != 0 or np.any(np.diff(rp.astype(np.int64)) < 0)
                or np.any(rp.astype(np.int64) > op.size)
                or (op.size and np.any((op & 0xFFFF) >= self.cols))):
            raise FormatError("invalid VXT outlier CSR indices")

    @property
    def kind(self) -> str:
        return "cb4"


@dataclass
class Cb4G64Matrix:
    """cb4 with a per-(row, 64-group) fp16 codebook.

    ``idx[r * padded_cols/2 + c/2] >> 4*(c%2) & 15`` is the index of column
    ``c``; ``lut_f16[(r * padded_cols/64 + c/64) * 16 + q]`` its value.
    """

    rows: int
    cols: int
    padded_cols: int
    idx: np.ndarray       # u8[rows * padded_cols/2]
    lut_f16: np.ndarray   # u16[rows * padded_cols/64 * 16]

    def validate(self) -> None:
        if self.rows <= 0 or self.cols <= 0:
            raise FormatError("rows and cols must be positive")
        if self.padded_cols < self.cols or self.padded_cols % 64 != 0:
            raise FormatError("invalid g64 padded_cols")
        if (np.asarray(self.idx).size != self.rows * self.padded_cols // 2
                or np.asarray(self.lut_f16).size != self.rows * self.padded_cols // 64 * 16):
            raise FormatError("corrupt g64 plane lengths")

    @property
    def kind(self) -> str:
        return "g64"


@dataclass
class Q8Matrix:
    """Rows of GGUF ``Q8_0`` / ``KvQ8Block`` 34-byte blocks, ceil(cols/32) per row."""

    rows: int
    cols: int
    blocks: np.ndarray    # u8[rows * ceil(cols/32) * 34]

    @property
    def blocks_per_row(self) -> int:
        return (self.cols + 31) // 32

    def validate(self) -> None:
        if self.rows <= 0 or self.cols <= 0:
            raise FormatError("rows and cols must be positive")
        if np.asarray(self.blocks).size != self.rows * self.blocks_per_row * 34:
            raise FormatError("corrupt Q8_0 byte length")

    def scales_f16(self) -> np.ndarray:
        b = np.asarray(self.blocks, dtype=np.uint8).reshape(-1, 34)
        return b[:, 0:2].copy().view(np.uint16).reshape(-1)

    def qs(self) -> np.ndarray:
        b = np.asarray(self.blocks, dtype=np.uint8).reshape(-1, 34)
        return b[:, 2:34].copy().view(np.int8)

    @property
    def kind(self) -> str:
        return "q8"


@dataclass
class Q4_0Matrix:
    """``Q4_0Matrix`` (``q4_0.rs:7-14``): f16 scale + 4 words per 32-column block."""

    rows: int
    cols: int
    padded_cols: int
    scales_f16: np.ndarray   # u16[rows * padded_cols/32]
    qs_words: np.ndarray     # u32[rows * padded_cols/32 * 4]

    @property
    def blocks_per_row(self) -> int:
        return self.padded_cols // 32

    def validate(self) -> None:
        """The archive reader's checks (``format.rs:453-462``)."""
        if self.rows <= 0 or self.cols <= 0:
            raise FormatError("rows and cols must be positive")
        if self.padded_cols != (self.cols + 31) // 32 * 32:
            raise FormatError("invalid VXT Q4_0 padded_cols")
        blocks = self.rows * self.blocks_per_row
        if np.asarray(self.scales_f16).size != blocks or np.asarray(self.qs_words).size != blocks * 4:
            raise FormatError("corrupt VXT Q4_0 plane lengths")

    @classmethod
    def from_gguf_blocks(cls, rows: int, cols: int, blocks: np.ndarray) -> "Q4_0Matrix":
        """Split GGUF ``Q4_0`` 18-byte blocks (``gguf.rs:211-221``; cols % 32 == 0)."""
        if cols % 32:
            raise FormatError("GGUF Q4_0 rows need cols % 32 == 0")
        b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, 18)
        if b.shape[0] != rows * (cols // 32):
            raise FormatError("corrupt GGUF Q4_0 byte length")
        sc = b[:, 0:2].copy().view(np.uint16).reshape(-1)
        qs = b[:, 2:18].copy().view(np.uint32).reshape(-1)
        return cls(rows, cols, cols, sc, qs)

    def gguf_blocks(self) -> np.ndarray:
        """The same blocks as GGUF ``Q4_0`` bytes (18 per block)."""
        n = self.rows * self.blocks_per_row
        out = np.empty((n, 18), dtype=np.uint8)
        out[:, 0:2] = np.asarray(self.scales_f16, np.uint16).reshape(n, 1).view(np.uint8)
        out[:, 2:18] = np.asarray(self.qs_words, np.uint32).reshape(n, 4).view(np.uint8)
        return out.reshape(-1)

    @property
    def kind(self) -> str:
        return "q4_0"


PackedTensor = Union[CodebookMatrix, Cb4G64Matrix, Q8Matrix, Q4_0Matrix]


def q8_from_planes(rows: int, cols: int, qs: np.ndarray, d_f16: np.ndarray) -> Q8Matrix:
    """Assemble GGUF ``Q8_0`` bytes from an int8 plane and an f16-bits scale plane."""
    kb = (cols + 31) // 32
    qs = np.asarray(qs, dtype=np.int8).reshape(rows * kb, 32)
    d = np.asarray(d_f16, dtype=np.uint16).reshape(rows * kb, 1)
    blk = np.empty((rows * kb, 34), dtype=np.uint8)
    blk[:, 0:2] = d.view(np.uint8).reshape(rows * kb, 2)
    blk[:, 2:] = qs.view(np.uint8)
    return Q8Matrix(rows, cols, blk.reshape(-1))


def concat_rows(parts):
    """Stack g64 or Q8 matrices with equal ``cols`` along rows (``[q;k;v]``).

    Their planes are per-row, so stacking needs no rebasing.  Codebook
    matrices carry a per-matrix centroid table and CSR stream; they are
    concatenated on upload instead (``HipEngine.upload_concat``).
    """
    parts = list(parts)
    if not parts:
        raise FormatError("nothing to concatenate")
    first = parts[0]
    if any(type(p) is not type(first) for p in parts):
        raise FormatError("concatenated parts must share one format")
    if any(p.cols != first.cols for p in parts):
        raise FormatError("concatenated parts must share cols")
    rows = sum(p.rows for p in parts)
    if isinstance(first, Q8Matrix):
        return Q8Matrix(rows, first.cols, np.concatenate([np.asarray(p.blocks, np.uint8) for p in parts]))
    if isinstance(first, Cb4G64Matrix):
        if any(p.padded_cols != first.padded_cols for p in parts):
            raise FormatError("concatenated parts must share padded_cols")
        return Cb4G64Matrix(rows, first.cols, first.padded_cols,
                            np.concatenate([np.asarray(p.idx, np.uint8) for p in parts]),
                            np.concatenate([np.asarray(p.lut_f16, np.uint16) for p in parts]))
    raise FormatError(f"concat_rows does not handle {type(first).__name__}")
