"""Weight containers from disk: ``.vxt`` (VXT1) archives and GGUF files.

Both readers are native (``csrc/archive.cpp``, ``vxt_hip_vxt_parse`` and
``vxt_hip_gguf_parse``): they verify and index the bytes, which stay in a
read-only memory map; this module turns the index into host containers
(``formats.CodebookMatrix`` / ``formats.Q8Matrix``, numpy views of the map)
and uploads entries straight from the mapped bytes
(``vxt_hip_upload_vxt_entry``, ``vxt_hip_upload_gguf_q8_0``).

Reference: ``read_vxt_model`` (format.rs:301-451) and ``GgufView``
(gguf.rs:75-172).  Like the reference's device path, only 4-bit codebook
entries and Q8_0 GGUF matrices go to the GPU; other kinds are listed with
their kind id and can be read by the reference's own code.
"""
from __future__ import annotations

import ctypes as C
import mmap
import os
from dataclasses import dataclass

import numpy as np

from . import engine
from .formats import CodebookMatrix, FormatError, Q4_0Matrix, Q8Matrix

KIND_LOSSLESS, KIND_CODEBOOK, KIND_Q4_0, KIND_WHT2, KIND_RAW_F32, KIND_TURBO_WHT, KIND_TURBO_WHT_EC = range(1, 8)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_BF16 = 0, 1, 2, 8, 12, 30


def _raise_from(code: int, buf) -> None:
    msg = buf.value.decode(errors="replace")
    if code == engine.VXT_E_UNSUPPORTED:
        raise engine.UnsupportedError(code, msg)
    raise FormatError(msg) if code == engine.VXT_E_FORMAT else engine.BackendError(code, msg)


class _Bytes:
    """Bytes held for the readers: a read-only map of a file, or a buffer."""

    def __init__(self, src):
        self._map = None
        self._file = None
        if isinstance(src, (str, os.PathLike)):
            self._file = open(src, "rb")
            size = os.fstat(self._file.fileno()).st_size
            if size == 0:
                self.array = np.zeros(0, np.uint8)
            else:
                self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
                self.array = np.frombuffer(self._map, dtype=np.uint8)
        else:
            self.array = np.frombuffer(bytes(src), dtype=np.uint8)
        self.ptr = self.array.ctypes.data if self.array.size else None
        self.len = int(self.array.size)

    def view(self, off: int, dtype, count: int) -> np.ndarray:
        """Elements at a byte offset, copied when not aligned for their type."""
        dt = np.dtype(dtype)
        a = self.array[off: off + count * dt.itemsize]
        if off % dt.itemsize == 0:
            return a.view(dt)
        return a.copy().view(dt)

    def text(self, off: int, n: int) -> str:
        return bytes(self.array[off: off + n]).decode("utf-8", errors="replace")

    def close(self) -> None:
        self.array = None
        if self._map is not None:
            self._map.close()
            self._map = None
        if self._file is not None:
            self._file.close()
            self._file = None


@dataclass
class ArchiveEntry:
    name: str
    kind: int
    sub: int
    rows: int
    cols: int
    padded_cols: int
    raw: engine.VxtArchiveEntry


class VxtArchive:
    """A verified ``.vxt`` archive (path or bytes)."""

    def __init__(self, src):
        self._b = _Bytes(src)
        L = engine.load_library()
        buf = C.create_string_buffer(512)
        n, meta = C.c_uint32(), C.c_uint32()
        rc = L.vxt_hip_vxt_parse(self._b.ptr, self._b.len, None, 0, C.byref(n), C.byref(meta), buf, len(buf))
        if rc != engine.VXT_OK:
            self._b.close()
            _raise_from(rc, buf)
        arr = (engine.VxtArchiveEntry * max(n.value, 1))()
        rc = L.vxt_hip_vxt_parse(self._b.ptr, self._b.len, arr, n.value, C.byref(n), C.byref(meta), buf, len(buf))
        if rc != engine.VXT_OK:
            self._b.close()
            _raise_from(rc, buf)
        self.meta_count = meta.value
        self.entries = [ArchiveEntry(self._b.text(e.name_off, e.name_len), e.kind, e.sub, e.rows, e.cols,
                                     e.padded_cols, e) for e in arr[: n.value]]
        self._by_name = {e.name: e for e in self.entries}

    def __getitem__(self, name: str) -> ArchiveEntry:
        return self._by_name[name]

    def codebook(self, name: str) -> CodebookMatrix:
        """The entry as a host ``CodebookMatrix`` (views of the mapped bytes)."""
        e = self[name]
        if e.kind != KIND_CODEBOOK:
            raise engine.UnsupportedError(engine.VXT_E_UNSUPPORTED, f"{name}: kind {e.kind} is not a codebook")
        r = e.raw
        b = self._b
        return CodebookMatrix(e.rows, e.cols, e.padded_cols, b.view(r.centroids_off, np.float32, 16),
                              b.view(r.scales_off, np.uint16, r.n_scales), b.view(r.words_off, np.uint32, r.n_words),
                              b.view(r.row_ptr_off, np.uint32, r.n_row_ptr),
                              b.view(r.outliers_off, np.uint32, r.n_outliers), bits=e.sub)

    def q4_0(self, name: str) -> Q4_0Matrix:
        """A Q4_0 entry as a host ``Q4_0Matrix`` (views of the mapped bytes)."""
        e = self[name]
        if e.kind != KIND_Q4_0:
            raise engine.UnsupportedError(engine.VXT_E_UNSUPPORTED, f"{name}: kind {e.kind} is not Q4_0")
        r = e.raw
        return Q4_0Matrix(e.rows, e.cols, e.padded_cols, self._b.view(r.scales_off, np.uint16, r.n_scales),
                          self._b.view(r.words_off, np.uint32, r.n_words))

    def upload(self, eng: engine.HipEngine, name: str) -> engine.GpuPackedTensor:
        """Upload a 4-bit codebook or Q4_0 entry from the archive bytes."""
        e = self[name]
        buf = C.create_string_buffer(512)
        h = engine.load_library().vxt_hip_upload_vxt_entry(eng.ctx, self._b.ptr, self._b.len, C.byref(e.raw),
                                                           buf, len(buf))
        if not h:
            engine._upload_failed(buf)
        return engine.GpuPackedTensor(eng, h)

    def close(self) -> None:
        self._b.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


@dataclass
class GgufTensorInfo:
    name: str
    ggml_type: int
    ne: tuple
    supported: bool
    raw: engine.VxtGgufTensor

    def matrix_dims(self):
        """(rows, cols): ne[0] is the contiguous cols (gguf.rs:65-73)."""
        if len(self.ne) < 2:
            return None
        rows = int(np.prod(self.ne[1:], dtype=np.uint64))
        return (rows, self.ne[0]) if rows and self.ne[0] else None


class GgufFile:
    """A parsed GGUF v2/v3 file (path or bytes)."""

    def __init__(self, src):
        self._b = _Bytes(src)
        L = engine.load_library()
        buf = C.create_string_buffer(512)
        n, ver, al = C.c_uint32(), C.c_uint32(), C.c_uint64()
        rc = L.vxt_hip_gguf_parse(self._b.ptr, self._b.len, None, 0, C.byref(n), C.byref(ver), C.byref(al), buf,
                                  len(buf))
        if rc != engine.VXT_OK:
            self._b.close()
            _raise_from(rc, buf)
        arr = (engine.VxtGgufTensor * max(n.value, 1))()
        rc = L.vxt_hip_gguf_parse(self._b.ptr, self._b.len, arr, n.value, C.byref(n), C.byref(ver), C.byref(al),
                                  buf, len(buf))
        if rc != engine.VXT_OK:
            self._b.close()
            _raise_from(rc, buf)
        self.version, self.alignment = ver.value, al.value
        self.tensors = [GgufTensorInfo(self._b.text(t.name_off, t.name_len), t.ggml_type,
                                       tuple(int(t.ne[d]) for d in range(t.n_dims)), bool(t.supported), t)
                        for t in arr[: n.value]]
        self._by_name = {t.name: t for t in self.tensors}

    def __getitem__(self, name: str) -> GgufTensorInfo:
        return self._by_name[name]

    def tensor_bytes(self, name: str) -> np.ndarray:
        """The tensor's bytes as stored (``tensor_bytes``, gguf.rs:160-172)."""
        t = self[name]
        if not t.supported:
            raise engine.UnsupportedError(engine.VXT_E_UNSUPPORTED, f"unsupported GGUF type {t.ggml_type}")
        return self._b.array[t.raw.data_off: t.raw.data_off + t.raw.data_len]

    def q8(self, name: str) -> Q8Matrix:
        """A Q8_0 matrix as a host ``Q8Matrix`` over the file's blocks."""
        t = self[name]
        if t.ggml_type != GGML_Q8_0:
            raise engine.UnsupportedError(engine.VXT_E_UNSUPPORTED, f"{name} is not Q8_0")
        dims = t.matrix_dims()
        if dims is None:
            raise FormatError(f"{name} is not a matrix")
        rows, cols = dims
        return Q8Matrix(rows, cols, self.tensor_bytes(name))

    def q4_0(self, name: str) -> Q4_0Matrix:
        """A Q4_0 matrix (gguf.rs:211-221 blocks) as a host ``Q4_0Matrix``."""
        t = self[name]
        if t.ggml_type != GGML_Q4_0:
            raise engine.UnsupportedError(engine.VXT_E_UNSUPPORTED, f"{name} is not Q4_0")
        dims = t.matrix_dims()
        if dims is None:
            raise FormatError(f"{name} is not a matrix")
        rows, cols = dims
        return Q4_0Matrix.from_gguf_blocks(rows, cols, self.tensor_bytes(name))

    def upload(self, eng: engine.HipEngine, name: str) -> engine.GpuPackedTensor:
        """Upload a Q8_0 matrix from the file bytes (no f32 expansion), or a
        Q4_0 matrix through its planes (``HipEngine.upload_packed``)."""
        t = self[name]
        if t.ggml_type == GGML_Q4_0:
            return eng.upload_packed(self.q4_0(name))
        buf = C.create_string_buffer(512)
        h = engine.load_library().vxt_hip_upload_gguf_q8_0(eng.ctx, self._b.ptr, self._b.len, C.byref(t.raw), buf,
                                                           len(buf))
        if not h:
            engine._upload_failed(buf)
        return engine.GpuPackedTensor(eng, h)

    def close(self) -> None:
        self._b.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
