"""Writers of the two weight containers, for building test archives.

``write_vxt`` restates the reference writer (``write_vxt_model``,
format.rs:183-294, with the plane encoders of format_io.rs:16-63): 64-byte
aligned sections, u64-counted little-endian planes, an FNV-1a64 tag after
each section and over the whole archive.  Metadata values are written raw
(format.rs's ``store_raw_meta_blob`` path for values under 256 bytes).
``write_gguf`` lays out a GGUF v2/v3 file as gguf.rs:83-158 reads it.
"""
import struct

import numpy as np


def fnv1a64(b: bytes) -> int:
    h = 0xCBF29CE484222325
    for x in b:
        h ^= x
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def _vec(a, dtype) -> bytes:
    a = np.ascontiguousarray(a, dtype=dtype)
    return struct.pack("<Q", a.size) + a.tobytes()


def _hdr(kind, sub, rows, cols, pcols) -> bytes:
    return bytes([kind, sub, 0, 0, 0, 0, 0, 0]) + struct.pack("<QQQ", rows, cols, pcols)


def codebook_section(m) -> tuple:
    """(kind, sub, rows, cols, padded_cols, payload) of a CodebookMatrix."""
    payload = (np.ascontiguousarray(m.centroids, np.float32).tobytes() + _vec(m.scales_f16, np.uint16)
               + _vec(m.packed_words, np.uint32) + _vec(m.outlier_row_ptr, np.uint32)
               + _vec(m.outliers_packed, np.uint32))
    return (2, m.bits, m.rows, m.cols, m.padded_cols, payload)


def raw_f32_section(a) -> tuple:
    a = np.asarray(a, np.float32)
    return (5, 0, a.shape[0], a.shape[1], a.shape[1], _vec(a.reshape(-1), np.float32))


def q4_0_section(rows, cols, m=None) -> tuple:
    """A Q4_0 section (format.rs:243-247): all-zero planes, or those of Q4_0Matrix m."""
    pc = (cols + 31) // 32 * 32
    blocks = rows * pc // 32
    if m is not None:
        return (3, 0, m.rows, m.cols, m.padded_cols, _vec(m.scales_f16, np.uint16) + _vec(m.qs_words, np.uint32))
    return (3, 0, rows, cols, pc, _vec(np.zeros(blocks, np.uint16), np.uint16)
            + _vec(np.zeros(blocks * 4, np.uint32), np.uint32))


def wht2_section(rows, cols) -> tuple:
    pc = (cols + 255) // 256 * 256
    groups = rows * pc // 128
    return (4, 2, rows, cols, pc, np.zeros(16, np.float32).tobytes() + _vec(np.zeros(groups, np.uint16), np.uint16)
            + _vec(np.zeros(rows * pc // 256 * 16, np.uint32), np.uint32)
            + _vec(np.zeros(rows + 1, np.uint32), np.uint32) + _vec(np.zeros(0, np.uint32), np.uint32))


def lossless_section(rows, cols) -> tuple:
    pc = (cols + 255) // 256 * 256
    return (1, 0, rows, cols, pc, bytes(8) + _vec(np.zeros(rows * pc, np.uint8), np.uint8)
            + _vec(np.zeros(rows * pc // 256 * 8 * 3, np.uint32), np.uint32)
            + _vec(np.zeros(rows * pc // 256, np.uint32), np.uint32) + _vec(np.zeros(0, np.uint8), np.uint8))


def write_vxt(entries, meta=(), version=1) -> bytes:
    """entries: [(name, (kind, sub, rows, cols, padded_cols, payload))]."""
    out = bytearray(b"VXT1" + struct.pack("<III", version, len(entries), len(meta)))
    for k, v in meta:
        kb = k.encode()
        out += struct.pack("<I", len(kb)) + kb + struct.pack("<Q", len(v)) + v
    for name, (kind, sub, rows, cols, pcols, payload) in entries:
        while len(out) % 64:
            out.append(0)
        start = len(out)
        nb = name.encode()
        out += struct.pack("<I", len(nb)) + nb + _hdr(kind, sub, rows, cols, pcols) + payload
        out += struct.pack("<Q", fnv1a64(bytes(out[start:])))
    out += struct.pack("<Q", fnv1a64(bytes(out)))
    return bytes(out)


# ---- GGUF ------------------------------------------------------------------

def _gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def gguf_value(vtype, v) -> bytes:
    fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
    if vtype == 8:
        return _gstr(v)
    if vtype == 9:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(gguf_value(et, x) for x in items)
    return struct.pack(fmt[vtype], v)


def write_gguf(tensors, kv=(), version=3, alignment=None) -> bytes:
    """tensors: [(name, ne tuple, ggml type, data bytes)]; kv: [(key, vtype, value)]."""
    kv = list(kv)
    if alignment is not None:
        kv.append(("general.alignment", 4, alignment))
    align = alignment or 32
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv)))
    for key, vt, v in kv:
        out += _gstr(key) + struct.pack("<I", vt) + gguf_value(vt, v)
    offs, off = [], 0
    for _, _, _, data in tensors:
        offs.append(off)
        off += (len(data) + align - 1) // align * align
    for (name, ne, gt, _), o in zip(tensors, offs):
        out += _gstr(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        out += struct.pack("<IQ", gt, o)
    while len(out) % align:
        out.append(0)
    for (_, _, _, data), o in zip(tensors, offs):
        out += data
        while len(out) % align:
            out.append(0)
    return bytes(out)
