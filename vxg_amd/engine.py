"""Python mirror of the reference's GPU matmul engine API over the HIP C ABI.

Shape of the API follows ``MetalEngine`` / ``GpuPackedTensor``
(``crates/vxg-tensor/src/metal.rs:393-557``) and the weight dispatch seam
``MatWeight::forward`` / ``forward_multi`` (``llm_cpu.rs:15-71``):

=============================================  ================================
reference (Rust)                               here
=============================================  ================================
``MetalEngine::new()``                         ``HipEngine(device=-1)``
``MetalEngine::device_name()``                 ``HipEngine.device_name``
``MetalEngine::upload_packed(&PackedTensor)``  ``HipEngine.upload_packed(m)``
``MetalEngine::run_multi_same_x(x, jobs)``     ``HipEngine.run_multi_same_x``
``GpuPackedTensor::run_gemv(eng, x, y, it)``   ``GpuPackedTensor.run_gemv``
``PackedTensor::gemm_cpu(x, m, y, threads)``   ``HipEngine.gemm(t, X)``
``CodebookMatrix::decode_row``                 ``HipEngine.dequant_rows``
``Error::Backend(String)``                     :class:`BackendError`
``Error::Unsupported``                         :class:`UnsupportedError`
=============================================  ================================

Device-pointer calls (``matmul_dev`` / ``matmul_multi_dev`` /
``dequant_rows_dev``) take raw device addresses and a ``hipStream_t``.  The
engine owns what they need -- :meth:`HipEngine.alloc` / :class:`DeviceBuffer`,
the context stream (:attr:`HipEngine.stream`) and HIP-graph capture
(:meth:`HipEngine.capture`) -- so no other GPU runtime has to be loaded.  (A
process that also uses PyTorch must import torch first: torch ships its own
copy of the HIP runtime under the same soname, and the first one loaded is the
one both use.)

There is no CPU fallback: if ``libvxt_hip.so`` is missing or no gfx950 device
is present, construction raises.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Iterable, Sequence

import numpy as np

from .formats import Cb4G64Matrix, CodebookMatrix, Q4_0Matrix, Q8Matrix

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvxt_hip.so")

VXT_OK = 0
VXT_E_ARG, VXT_E_SHAPE, VXT_E_FORMAT, VXT_E_DEVICE, VXT_E_UNSUPPORTED = -1, -2, -3, -4, -5
DTYPE_F32, DTYPE_BF16 = 0, 1
ACT_SILU, ACT_GELU_TANH = 0, 1
NORM_PLAIN, NORM_GLU_SILU, NORM_GLU_GELU_TANH = 0, 1, 2
GEMM_AUTO, GEMM_PANEL, GEMM_FUSED, GEMM_LIBRARY = 0, 1, 2, 3
KIND_CB4, KIND_Q4_0, KIND_Q8_0, KIND_CB4_G64 = 2, 4, 8, 9

ABI_SYMBOLS = (
    "vxt_hip_create", "vxt_hip_destroy", "vxt_hip_upload_cb4", "vxt_hip_upload_cb4_concat",
    "vxt_hip_upload_cb4_g64",
    "vxt_hip_upload_q8_0", "vxt_hip_upload_q4_0", "vxt_hip_clone_tensor", "vxt_hip_free_tensor",
    "vxt_hip_tensor_info", "vxt_hip_run_multi", "vxt_hip_gemm", "vxt_hip_dequant_rows",
    "vxt_hip_matmul_dev", "vxt_hip_matmul_multi_dev", "vxt_hip_dequant_rows_dev", "vxt_hip_greedy_dev",
    "vxt_hip_embed_dev", "vxt_hip_ffn_glu_dev", "vxt_hip_rms_norm_dev", "vxt_hip_norm_matmul_dev",
    "vxt_hip_vxt_parse", "vxt_hip_upload_vxt_entry", "vxt_hip_gguf_parse", "vxt_hip_upload_gguf_q8_0",
    "vxt_hip_kv_q8_append_dev", "vxt_hip_attn_q8_dev", "vxt_hip_attn_prep_q8_dev", "vxt_hip_attn_step_q8_dev",
    "vxt_hip_matmul_noalloc_dev", "vxt_hip_read_probe_dev", "vxt_hip_last_kernel_ms", "vxt_hip_set_gemm_path", "vxt_hip_device_alloc", "vxt_hip_device_free", "vxt_hip_memcpy",
    "vxt_hip_stream", "vxt_hip_synchronize", "vxt_hip_capture_begin", "vxt_hip_capture_end",
    "vxt_hip_graph_launch", "vxt_hip_graph_free",
    "vxt_hip_runner_create", "vxt_hip_runner_step", "vxt_hip_runner_generate", "vxt_hip_runner_destroy",
)


class BackendError(RuntimeError):
    """A failed engine call (the reference's ``Error::Backend(String)``)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class UnsupportedError(BackendError):
    """A valid request this build does not support (``Error::Unsupported``)."""


class Cb4View(C.Structure):
    _fields_ = [("bits", C.c_uint32), ("rows", C.c_uint32), ("cols", C.c_uint32),
                ("padded_cols", C.c_uint32),
                ("centroids", C.c_void_p),
                ("scales_f16", C.c_void_p), ("n_scales", C.c_size_t),
                ("packed_words", C.c_void_p), ("n_words", C.c_size_t),
                ("outlier_row_ptr", C.c_void_p), ("n_row_ptr", C.c_size_t),
                ("outliers_packed", C.c_void_p), ("n_outliers", C.c_size_t)]


class Cb4G64View(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("cols", C.c_uint32), ("padded_cols", C.c_uint32),
                ("reserved", C.c_uint32),
                ("idx", C.c_void_p), ("n_idx", C.c_size_t),
                ("lut_f16", C.c_void_p), ("n_lut", C.c_size_t)]


class VxtArchiveEntry(C.Structure):
    _fields_ = [("name_off", C.c_uint64), ("name_len", C.c_uint64), ("kind", C.c_uint32), ("sub", C.c_uint32),
                ("rows", C.c_uint64), ("cols", C.c_uint64), ("padded_cols", C.c_uint64),
                ("section_off", C.c_uint64), ("section_len", C.c_uint64), ("centroids_off", C.c_uint64),
                ("scales_off", C.c_uint64), ("n_scales", C.c_uint64), ("words_off", C.c_uint64),
                ("n_words", C.c_uint64), ("row_ptr_off", C.c_uint64), ("n_row_ptr", C.c_uint64),
                ("outliers_off", C.c_uint64), ("n_outliers", C.c_uint64)]


class VxtGgufTensor(C.Structure):
    _fields_ = [("name_off", C.c_uint64), ("name_len", C.c_uint64), ("ggml_type", C.c_uint32),
                ("n_dims", C.c_uint32), ("ne", C.c_uint64 * 8), ("data_off", C.c_uint64),
                ("data_len", C.c_uint64), ("supported", C.c_uint32), ("reserved", C.c_uint32)]


class KvQ8CacheView(C.Structure):
    _fields_ = [("k_qs", C.c_void_p), ("k_d", C.c_void_p), ("v_qs", C.c_void_p), ("v_d", C.c_void_p),
                ("max_seq", C.c_uint32), ("n_kv", C.c_uint32), ("head_dim", C.c_uint32), ("reserved", C.c_uint32)]


class GqaParams(C.Structure):
    """``VxtGqaParams``: the scalar arguments of step_full_gqa_q8
    (llm_prefill.rs:259-278) and the optional device pointers (0 = none)."""
    _fields_ = [("q_norm", C.c_void_p), ("k_norm", C.c_void_p), ("q_bias", C.c_void_p), ("k_bias", C.c_void_p),
                ("v_bias", C.c_void_p), ("n_head", C.c_uint32), ("gated_q", C.c_uint32), ("rope_dim", C.c_uint32),
                ("rope_neox", C.c_uint32), ("rope_freq_base", C.c_float), ("eps", C.c_float)]


class RunnerLayer(C.Structure):
    """``VxtRunnerLayer``: one decoder layer's tensors (handles) and device
    norm weights (0 = none for q_norm / k_norm)."""
    _fields_ = [("w_in", C.c_void_p), ("w_out", C.c_void_p), ("w_ffn_gu", C.c_void_p), ("w_ffn_dn", C.c_void_p),
                ("attn_norm", C.c_void_p), ("post_attn_norm", C.c_void_p), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p)]


class RunnerConfig(C.Structure):
    """``VxtRunnerConfig``."""
    _fields_ = [("n_layers", C.c_uint32), ("hidden", C.c_uint32), ("n_head", C.c_uint32), ("n_kv", C.c_uint32),
                ("head_dim", C.c_uint32), ("ffn", C.c_uint32), ("vocab", C.c_uint32), ("gated_q", C.c_uint32),
                ("rope_dim", C.c_uint32), ("rope_neox", C.c_uint32), ("activation", C.c_uint32),
                ("max_seq", C.c_uint32), ("max_batch", C.c_uint32), ("rope_freq_base", C.c_float),
                ("eps", C.c_float), ("embed_scale", C.c_float)]


class HipJob(C.Structure):
    _fields_ = [("tensor", C.c_void_p), ("y", C.c_void_p)]


_lib = None


def load_library(path: str = LIB_PATH):
    """Load and type the C ABI.  Raises if the library is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built; run `python -m vxg_amd.build` first")
    L = C.CDLL(path)
    vp, sz, u32, i32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_int32
    cp = C.c_char_p
    L.vxt_hip_create.restype = vp
    L.vxt_hip_create.argtypes = [i32, cp, sz, cp, sz]
    L.vxt_hip_destroy.restype = None
    L.vxt_hip_destroy.argtypes = [vp]
    L.vxt_hip_upload_cb4.restype = vp
    L.vxt_hip_upload_cb4.argtypes = [vp, C.POINTER(Cb4View), cp, sz]
    L.vxt_hip_upload_cb4_concat.restype = vp
    L.vxt_hip_upload_cb4_concat.argtypes = [vp, C.POINTER(Cb4View), u32, cp, sz]
    L.vxt_hip_upload_cb4_g64.restype = vp
    L.vxt_hip_upload_cb4_g64.argtypes = [vp, C.POINTER(Cb4G64View), cp, sz]
    L.vxt_hip_upload_q8_0.restype = vp
    L.vxt_hip_upload_q8_0.argtypes = [vp, u32, u32, vp, sz, cp, sz]
    L.vxt_hip_upload_q4_0.restype = vp
    L.vxt_hip_upload_q4_0.argtypes = [vp, u32, u32, u32, vp, sz, vp, sz, cp, sz]
    L.vxt_hip_clone_tensor.restype = vp
    L.vxt_hip_clone_tensor.argtypes = [vp, cp, sz]
    L.vxt_hip_free_tensor.restype = None
    L.vxt_hip_free_tensor.argtypes = [vp]
    L.vxt_hip_tensor_info.restype = C.c_int
    L.vxt_hip_tensor_info.argtypes = [vp, C.POINTER(u32), C.POINTER(u32), C.POINTER(u32),
                                      C.POINTER(C.c_uint64)]
    L.vxt_hip_run_multi.restype = C.c_int
    L.vxt_hip_run_multi.argtypes = [vp, vp, u32, C.POINTER(HipJob), u32, u32,
                                    C.POINTER(C.c_double), cp, sz]
    L.vxt_hip_gemm.restype = C.c_int
    L.vxt_hip_gemm.argtypes = [vp, vp, vp, u32, vp, C.POINTER(C.c_double), cp, sz]
    L.vxt_hip_dequant_rows.restype = C.c_int
    L.vxt_hip_dequant_rows.argtypes = [vp, vp, u32, u32, vp, cp, sz]
    L.vxt_hip_matmul_dev.restype = C.c_int
    L.vxt_hip_matmul_dev.argtypes = [vp, vp, vp, u32, u32, vp, u32, vp, cp, sz]
    L.vxt_hip_read_probe_dev.restype = C.c_int
    L.vxt_hip_read_probe_dev.argtypes = [vp, vp, sz, u32, vp, cp, sz]
    L.vxt_hip_matmul_noalloc_dev.restype = C.c_int
    L.vxt_hip_matmul_noalloc_dev.argtypes = [vp, vp, vp, u32, u32, vp, u32, vp, cp, sz]
    L.vxt_hip_matmul_multi_dev.restype = C.c_int
    L.vxt_hip_matmul_multi_dev.argtypes = [vp, C.POINTER(vp), u32, vp, u32, u32, C.POINTER(vp),
                                           u32, vp, cp, sz]
    L.vxt_hip_dequant_rows_dev.restype = C.c_int
    L.vxt_hip_dequant_rows_dev.argtypes = [vp, vp, u32, u32, vp, vp, cp, sz]
    L.vxt_hip_greedy_dev.restype = C.c_int
    L.vxt_hip_embed_dev.argtypes = [vp, vp, vp, u32, C.c_float, vp, u32, vp, cp, sz]
    L.vxt_hip_embed_dev.restype = C.c_int
    L.vxt_hip_ffn_glu_dev.argtypes = [vp, vp, vp, u32, u32, vp, u32, u32, u32, vp, cp, sz]
    L.vxt_hip_ffn_glu_dev.restype = C.c_int
    L.vxt_hip_rms_norm_dev.argtypes = [vp, vp, vp, vp, vp, u32, u32, u32, u32, C.c_float, vp, cp, sz]
    L.vxt_hip_rms_norm_dev.restype = C.c_int
    L.vxt_hip_norm_matmul_dev.argtypes = [vp, vp, vp, vp, vp, C.c_float, vp, u32, vp, u32, u32, vp, cp, sz]
    L.vxt_hip_norm_matmul_dev.restype = C.c_int
    L.vxt_hip_kv_q8_append_dev.argtypes = [vp, C.POINTER(KvQ8CacheView), vp, vp, u32, vp, cp, sz]
    L.vxt_hip_kv_q8_append_dev.restype = C.c_int
    L.vxt_hip_attn_q8_dev.argtypes = [vp, C.POINTER(KvQ8CacheView), vp, u32, u32, vp, vp, vp, cp, sz]
    L.vxt_hip_attn_q8_dev.restype = C.c_int
    gqa = [vp, C.POINTER(KvQ8CacheView), C.POINTER(GqaParams), vp, u32, vp, vp, u32, u32, u32, u32]
    L.vxt_hip_attn_prep_q8_dev.argtypes = gqa + [vp, vp, vp, cp, sz]
    L.vxt_hip_attn_prep_q8_dev.restype = C.c_int
    L.vxt_hip_attn_step_q8_dev.argtypes = gqa + [vp, vp, cp, sz]
    L.vxt_hip_attn_step_q8_dev.restype = C.c_int
    L.vxt_hip_vxt_parse.argtypes = [vp, sz, C.POINTER(VxtArchiveEntry), u32, C.POINTER(u32), C.POINTER(u32),
                                    cp, sz]
    L.vxt_hip_vxt_parse.restype = C.c_int
    L.vxt_hip_upload_vxt_entry.argtypes = [vp, vp, sz, C.POINTER(VxtArchiveEntry), cp, sz]
    L.vxt_hip_upload_vxt_entry.restype = vp
    L.vxt_hip_gguf_parse.argtypes = [vp, sz, C.POINTER(VxtGgufTensor), u32, C.POINTER(u32), C.POINTER(u32),
                                     C.POINTER(C.c_uint64), cp, sz]
    L.vxt_hip_gguf_parse.restype = C.c_int
    L.vxt_hip_upload_gguf_q8_0.argtypes = [vp, vp, sz, C.POINTER(VxtGgufTensor), cp, sz]
    L.vxt_hip_upload_gguf_q8_0.restype = vp
    L.vxt_hip_greedy_dev.argtypes = [vp, vp, u32, vp, vp, cp, sz]
    L.vxt_hip_last_kernel_ms.restype = C.c_int
    L.vxt_hip_last_kernel_ms.argtypes = [vp, C.POINTER(C.c_double)]
    L.vxt_hip_set_gemm_path.restype = C.c_int
    L.vxt_hip_set_gemm_path.argtypes = [vp, u32]
    L.vxt_hip_device_alloc.restype = vp
    L.vxt_hip_device_alloc.argtypes = [vp, sz, cp, sz]
    L.vxt_hip_device_free.restype = None
    L.vxt_hip_device_free.argtypes = [vp, vp]
    L.vxt_hip_memcpy.restype = C.c_int
    L.vxt_hip_memcpy.argtypes = [vp, vp, vp, sz, u32, cp, sz]
    L.vxt_hip_stream.restype = vp
    L.vxt_hip_stream.argtypes = [vp]
    L.vxt_hip_synchronize.restype = C.c_int
    L.vxt_hip_synchronize.argtypes = [vp, cp, sz]
    L.vxt_hip_capture_begin.restype = C.c_int
    L.vxt_hip_capture_begin.argtypes = [vp, cp, sz]
    L.vxt_hip_capture_end.restype = vp
    L.vxt_hip_capture_end.argtypes = [vp, cp, sz]
    L.vxt_hip_graph_launch.restype = C.c_int
    L.vxt_hip_graph_launch.argtypes = [vp, vp, u32, C.POINTER(C.c_double), cp, sz]
    L.vxt_hip_graph_free.restype = None
    L.vxt_hip_graph_free.argtypes = [vp]
    L.vxt_hip_runner_create.restype = vp
    L.vxt_hip_runner_create.argtypes = [vp, C.POINTER(RunnerConfig), C.POINTER(RunnerLayer), vp, vp, vp, cp, sz]
    L.vxt_hip_runner_step.restype = C.c_int
    L.vxt_hip_runner_step.argtypes = [vp, C.POINTER(u32), u32, u32, vp, cp, sz]
    L.vxt_hip_runner_generate.restype = C.c_int
    L.vxt_hip_runner_generate.argtypes = [vp, u32, u32, u32, C.POINTER(u32), C.POINTER(u32), cp, sz]
    L.vxt_hip_runner_destroy.restype = None
    L.vxt_hip_runner_destroy.argtypes = [vp]
    _lib = L
    return L


def _errbuf():
    return C.create_string_buffer(512)


def _raise(code: int, buf) -> None:
    msg = buf.value.decode("utf-8", "replace")
    if code == VXT_E_UNSUPPORTED:
        raise UnsupportedError(code, msg)
    raise BackendError(code, msg)


def _upload_failed(buf) -> None:
    """An upload returned NULL: raise with the code its message implies."""
    msg = buf.value
    if b"corrupt" in msg or b"invalid" in msg or b"need" in msg:
        code = VXT_E_FORMAT
    elif b"only" in msg:
        code = VXT_E_UNSUPPORTED
    elif b"must" in msg or b"too large" in msg:
        code = VXT_E_SHAPE
    elif b"null" in msg or b"parts" in msg:
        code = VXT_E_ARG
    else:
        code = VXT_E_DEVICE
    _raise(code, buf)


def _check(code: int, buf) -> None:
    if code != VXT_OK:
        _raise(code, buf)


class GpuPackedTensor:
    """A device-resident weight matrix (``GpuPackedTensor``, metal.rs:527-557)."""

    def __init__(self, engine: "HipEngine", handle: int):
        self._engine = engine
        self.handle = handle
        k, r, c, b = C.c_uint32(), C.c_uint32(), C.c_uint32(), C.c_uint64()
        load_library().vxt_hip_tensor_info(handle, C.byref(k), C.byref(r), C.byref(c), C.byref(b))
        self.kind, self.rows, self.cols, self.device_bytes = k.value, r.value, c.value, b.value

    def run_gemv(self, engine: "HipEngine", x, y: np.ndarray, iters: int = 1) -> float:
        """``y = W x`` (f32, host), ``iters`` times; returns mean kernel ms."""
        return engine.run_multi_same_x(x, [(self, y)], iters=iters)

    def clone(self) -> "GpuPackedTensor":
        buf = _errbuf()
        h = load_library().vxt_hip_clone_tensor(self.handle, buf, len(buf))
        if not h:
            _raise(VXT_E_DEVICE, buf)
        return GpuPackedTensor(self._engine, h)

    def free(self) -> None:
        """Release the device copy (a no-op once the engine is closed:
        closing released it)."""
        if self.handle and self._engine.ctx:
            load_library().vxt_hip_free_tensor(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceBuffer:
    """A device allocation owned by the engine (``vxt_hip_device_alloc``)."""

    def __init__(self, engine: "HipEngine", nbytes: int):
        buf = _errbuf()
        p = load_library().vxt_hip_device_alloc(engine.ctx, int(nbytes), buf, len(buf))
        if not p:
            _raise(VXT_E_DEVICE, buf)
        self._engine = engine
        self.ptr = p
        self.nbytes = int(nbytes)

    def upload(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise BackendError(VXT_E_SHAPE, "array larger than the buffer")
        buf = _errbuf()
        _check(load_library().vxt_hip_memcpy(self._engine.ctx, self.ptr, a.ctypes.data, a.nbytes, 0,
                                             buf, len(buf)), buf)
        return self

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise BackendError(VXT_E_SHAPE, "requested more bytes than the buffer holds")
        buf = _errbuf()
        _check(load_library().vxt_hip_memcpy(self._engine.ctx, out.ctypes.data, self.ptr, out.nbytes,
                                             1, buf, len(buf)), buf)
        return out

    def free(self) -> None:
        if self.ptr and self._engine.ctx:
            load_library().vxt_hip_device_free(self._engine.ctx, self.ptr)
        self.ptr = None


class KvQ8Cache:
    """One layer's Q8_0 KV cache in device memory (``VxtKvQ8Cache``)."""

    def __init__(self, engine: "HipEngine", max_seq: int, n_kv: int, head_dim: int):
        self._engine = engine
        self.max_seq, self.n_kv, self.head_dim = int(max_seq), int(n_kv), int(head_dim)
        per = self.n_kv * self.head_dim
        self.k_qs, self.v_qs = engine.alloc(max_seq * per), engine.alloc(max_seq * per)
        self.k_d, self.v_d = engine.alloc(max_seq * per // 16), engine.alloc(max_seq * per // 16)
        self.view = KvQ8CacheView(self.k_qs.ptr, self.k_d.ptr, self.v_qs.ptr, self.v_d.ptr, self.max_seq,
                                  self.n_kv, self.head_dim, 0)

    def append(self, k_ptr: int, v_ptr: int, pos: int, stream: int = 0) -> None:
        buf = _errbuf()
        _check(load_library().vxt_hip_kv_q8_append_dev(self._engine.ctx, C.byref(self.view), k_ptr or None,
                                                       v_ptr or None, pos, stream or None, buf, len(buf)), buf)

    def attend(self, q_ptr: int, n_head: int, seq_len: int, out_ptr: int, gate_ptr: int = 0,
               stream: int = 0) -> None:
        buf = _errbuf()
        _check(load_library().vxt_hip_attn_q8_dev(self._engine.ctx, C.byref(self.view), q_ptr or None, n_head,
                                                  seq_len, gate_ptr or None, out_ptr or None, stream or None, buf,
                                                  len(buf)), buf)

    def prep(self, params: GqaParams, q_raw: int, k_cur: int, v_cur: int, pos: int, rope_pos: int, q_out: int,
             gate_out: int = 0, batch_m: int = 1, q_stride: int = 0, kv_stride: int = 0, stream: int = 0) -> None:
        """vxt_hip_attn_prep_q8_dev: q / k preparation and the cache writes of
        ``batch_m`` tokens at rows pos .. pos + batch_m - 1."""
        buf = _errbuf()
        _check(load_library().vxt_hip_attn_prep_q8_dev(
            self._engine.ctx, C.byref(self.view), C.byref(params), q_raw or None, q_stride, k_cur or None,
            v_cur or None, kv_stride, batch_m, pos, rope_pos, q_out or None, gate_out or None, stream or None, buf,
            len(buf)), buf)

    def step(self, params: GqaParams, q_raw: int, k_cur: int, v_cur: int, pos: int, rope_pos: int, out: int,
             batch_m: int = 1, q_stride: int = 0, kv_stride: int = 0, stream: int = 0) -> None:
        """vxt_hip_attn_step_q8_dev: the whole attention step of ``batch_m``
        tokens (causal), out [batch_m][n_head * head_dim]."""
        buf = _errbuf()
        _check(load_library().vxt_hip_attn_step_q8_dev(
            self._engine.ctx, C.byref(self.view), C.byref(params), q_raw or None, q_stride, k_cur or None,
            v_cur or None, kv_stride, batch_m, pos, rope_pos, out or None, stream or None, buf, len(buf)), buf)

    def blocks(self, which: str, seq_len: int):
        """Positions [0, seq_len) as KvQ8Block bytes [seq][n_kv * hd / 32][34] (host copy)."""
        import numpy as np
        qs_buf, d_buf = (self.k_qs, self.k_d) if which == "k" else (self.v_qs, self.v_d)
        per = self.n_kv * self.head_dim
        qs = qs_buf.download(np.int8, (seq_len, per // 32, 32))
        d = d_buf.download(np.uint16, (seq_len, per // 32, 1))
        out = np.empty((seq_len, per // 32, 34), np.uint8)
        out[..., :2] = d.view(np.uint8)
        out[..., 2:] = qs.view(np.uint8)
        return out

    def free(self) -> None:
        for b in (self.k_qs, self.v_qs, self.k_d, self.v_d):
            b.free()


class Graph:
    """An instantiated HIP graph captured from the engine stream."""

    def __init__(self, engine: "HipEngine", handle: int):
        self._engine = engine
        self.handle = handle

    def launch(self, replays: int = 1) -> float:
        """Replay back to back, wait, return total GPU ms of all replays."""
        ms = C.c_double()
        buf = _errbuf()
        _check(load_library().vxt_hip_graph_launch(self._engine.ctx, self.handle, int(replays),
                                                   C.byref(ms), buf, len(buf)), buf)
        return ms.value

    def free(self) -> None:
        """Release the graph (a no-op once its engine is closed: closing
        released it)."""
        if self.handle and self._engine.ctx:
            load_library().vxt_hip_graph_free(self.handle)
        self.handle = None


class DecodeRunner:
    """A device-resident decoder (``vxt_hip_runner_*``), the reference's
    device runner (metal_cb4_fast_ffi.rs:134-206): ``step`` is step_batch,
    ``generate`` the ring of enqueue_async / wait_cmd."""

    def __init__(self, engine: "HipEngine", handle: int, cfg: RunnerConfig):
        self._engine = engine
        self.handle = handle
        self.cfg = cfg

    def step(self, tokens, pos_base: int, want_logits: bool = True):
        """Feed ``tokens`` at positions ``pos_base..``; the last token's
        logits (f32 [vocab]) or None."""
        ids = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        buf = _errbuf()
        _check(load_library().vxt_hip_runner_step(
            self.handle, ids.ctypes.data_as(C.POINTER(C.c_uint32)), len(ids), int(pos_base),
            logits.ctypes.data if logits is not None else None, buf, len(buf)), buf)
        return logits

    def generate(self, token: int, pos_base: int, n_steps: int):
        """Greedy ids of ``n_steps`` single-token steps from ``token`` at
        ``pos_base``, and the per-step non-finite-logits flags."""
        ids = np.zeros(n_steps, np.uint32)
        flags = np.zeros(n_steps, np.uint32)
        buf = _errbuf()
        _check(load_library().vxt_hip_runner_generate(
            self.handle, int(token), int(pos_base), int(n_steps), ids.ctypes.data_as(C.POINTER(C.c_uint32)),
            flags.ctypes.data_as(C.POINTER(C.c_uint32)), buf, len(buf)), buf)
        return ids, flags

    def free(self) -> None:
        """Release the runner (a no-op once its engine is closed)."""
        if self.handle and self._engine.ctx:
            load_library().vxt_hip_runner_destroy(self.handle)
        self.handle = None


class HipEngine:
    """HIP compute engine for fused compressed-domain GEMV / GEMM (one GPU)."""

    def __init__(self, device: int = -1):
        L = load_library()
        name = C.create_string_buffer(256)
        buf = _errbuf()
        ctx = L.vxt_hip_create(int(device), name, len(name), buf, len(buf))
        if not ctx:
            _raise(VXT_E_DEVICE, buf)
        self.ctx = ctx
        self.device_name = name.value.decode()

    # -- lifetime -----------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "ctx", None):
            load_library().vxt_hip_destroy(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- upload --------------------------------------------------------------
    def upload_packed(self, m) -> GpuPackedTensor:
        """Copy a host weight matrix to HBM in its device-resident layout."""
        if isinstance(m, CodebookMatrix):
            return self.upload_concat([m])
        L = load_library()
        buf = _errbuf()
        if isinstance(m, Cb4G64Matrix):
            keep = [np.ascontiguousarray(m.idx, np.uint8), np.ascontiguousarray(m.lut_f16, np.uint16)]
            v = Cb4G64View(m.rows, m.cols, m.padded_cols, 0, keep[0].ctypes.data, keep[0].size,
                           keep[1].ctypes.data, keep[1].size)
            h = L.vxt_hip_upload_cb4_g64(self.ctx, C.byref(v), buf, len(buf))
        elif isinstance(m, Q8Matrix):
            b = np.ascontiguousarray(m.blocks, np.uint8)
            h = L.vxt_hip_upload_q8_0(self.ctx, m.rows, m.cols, b.ctypes.data, b.size, buf, len(buf))
        elif isinstance(m, Q4_0Matrix):
            # runs on the Q8_0 kernels: (q - 8) widened to int8, same f16 scales
            sc = np.ascontiguousarray(m.scales_f16, np.uint16)
            qw = np.ascontiguousarray(m.qs_words, np.uint32)
            h = L.vxt_hip_upload_q4_0(self.ctx, m.rows, m.cols, m.padded_cols, sc.ctypes.data, sc.size,
                                      qw.ctypes.data, qw.size, buf, len(buf))
        else:
            raise UnsupportedError(VXT_E_UNSUPPORTED, f"no device path for {type(m).__name__}")
        if not h:
            _upload_failed(buf)
        return GpuPackedTensor(self, h)

    def upload_concat(self, parts: Sequence) -> GpuPackedTensor:
        """Upload matrices with equal ``cols`` as one row-concatenated tensor.

        Codebook parts (1 to 3) keep their own centroid tables and CSR
        streams, as ``VxtCb4FastConcatMat::from_subs`` does
        (``metal_cb4_fast_ffi.rs:89-104``); g64 and Q8 parts are stacked on
        the host (``formats.concat_rows``).
        """
        parts = list(parts)
        if parts and all(isinstance(p, CodebookMatrix) for p in parts):
            L = load_library()
            buf = _errbuf()
            keep, views = [], (Cb4View * len(parts))()
            for i, m in enumerate(parts):
                arrs = [np.ascontiguousarray(m.centroids, np.float32),
                        np.ascontiguousarray(m.scales_f16, np.uint16),
                        np.ascontiguousarray(m.packed_words, np.uint32),
                        np.ascontiguousarray(m.outlier_row_ptr, np.uint32),
                        np.ascontiguousarray(m.outliers_packed, np.uint32)]
                keep.append(arrs)
                views[i] = Cb4View(m.bits, m.rows, m.cols, m.padded_cols, arrs[0].ctypes.data,
                                   arrs[1].ctypes.data, arrs[1].size, arrs[2].ctypes.data, arrs[2].size,
                                   arrs[3].ctypes.data, arrs[3].size,
                                   arrs[4].ctypes.data if arrs[4].size else None, arrs[4].size)
            h = L.vxt_hip_upload_cb4_concat(self.ctx, views, len(parts), buf, len(buf))
            if not h:
                _upload_failed(buf)
            return GpuPackedTensor(self, h)
        if any(isinstance(p, CodebookMatrix) for p in parts):
            raise BackendError(VXT_E_ARG, "concatenated parts must share one format")
        from .formats import concat_rows
        return self.upload_packed(concat_rows(parts))

    # -- host-pointer calls (synchronous) ------------------------------------
    def run_multi_same_x(self, x, jobs: Sequence, iters: int = 1) -> float:
        """All ``(tensor, y)`` GEMVs over one f32 x; returns mean kernel ms."""
        xx = np.ascontiguousarray(x, np.float32).reshape(-1)
        arr = (HipJob * len(jobs))()
        for i, (t, y) in enumerate(jobs):
            if not (isinstance(y, np.ndarray) and y.dtype == np.float32 and y.flags.c_contiguous
                    and y.size == t.rows):
                raise BackendError(VXT_E_SHAPE, "y must be a contiguous f32 array of rows")
            arr[i].tensor = t.handle
            arr[i].y = y.ctypes.data
        ms = C.c_double()
        buf = _errbuf()
        _check(load_library().vxt_hip_run_multi(self.ctx, xx.ctypes.data, xx.size, arr, len(jobs),
                                                max(int(iters), 1), C.byref(ms), buf, len(buf)), buf)
        return ms.value / max(int(iters), 1)

    def gemm(self, t: GpuPackedTensor, X) -> np.ndarray:
        """``Y[M, rows] = X[M, cols] W^T`` with f32 host arrays."""
        X = np.ascontiguousarray(X, np.float32).reshape(-1, t.cols)
        Y = np.empty((X.shape[0], t.rows), np.float32)
        ms = C.c_double()
        buf = _errbuf()
        _check(load_library().vxt_hip_gemm(self.ctx, t.handle, X.ctypes.data, X.shape[0],
                                           Y.ctypes.data, C.byref(ms), buf, len(buf)), buf)
        return Y

    def dequant_rows(self, t: GpuPackedTensor, row0: int = 0, nrows: int | None = None) -> np.ndarray:
        nrows = t.rows - row0 if nrows is None else nrows
        out = np.empty((nrows, t.cols), np.float32)
        buf = _errbuf()
        _check(load_library().vxt_hip_dequant_rows(self.ctx, t.handle, row0, nrows,
                                                   out.ctypes.data, buf, len(buf)), buf)
        return out

    def greedy(self, logits) -> tuple[int, bool]:
        """Greedy token over host f32 logits: ``(id, nonfinite)`` (see
        :meth:`greedy_dev`).  Copies the logits to the device and back."""
        logits = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1)
        src = self.to_device(logits) if logits.size else None
        out = self.alloc(8)
        try:
            self.greedy_dev(src.ptr if src else 0, logits.size, out.ptr, self.stream)
            self.synchronize()
            r = out.download(np.uint32, (2,))
        finally:
            out.free()
            if src:
                src.free()
        return int(r[0]), bool(r[1])

    def set_gemm_path(self, path: int) -> None:
        """Pin the prefill GEMM path (``GEMM_AUTO``, ``GEMM_PANEL``, ``GEMM_FUSED``, ``GEMM_LIBRARY``)."""
        rc = load_library().vxt_hip_set_gemm_path(self.ctx, path)
        if rc != VXT_OK:
            raise BackendError(rc, f"unknown GEMM path {path}")

    def last_kernel_ms(self) -> float:
        ms = C.c_double()
        load_library().vxt_hip_last_kernel_ms(self.ctx, C.byref(ms))
        return ms.value

    # -- device memory, stream, graphs ---------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        return DeviceBuffer(self, a.nbytes).upload(a)

    @property
    def stream(self) -> int:
        return load_library().vxt_hip_stream(self.ctx) or 0

    def synchronize(self) -> None:
        buf = _errbuf()
        _check(load_library().vxt_hip_synchronize(self.ctx, buf, len(buf)), buf)

    def capture(self, enqueue) -> Graph:
        """Record ``enqueue(stream)`` (which issues *_dev calls) into a graph."""
        L = load_library()
        buf = _errbuf()
        _check(L.vxt_hip_capture_begin(self.ctx, buf, len(buf)), buf)
        try:
            enqueue(self.stream)
        finally:
            h = L.vxt_hip_capture_end(self.ctx, buf, len(buf))
        if not h:
            _raise(VXT_E_DEVICE, buf)
        return Graph(self, h)

    def kv_q8_cache(self, max_seq: int, n_kv: int, head_dim: int) -> KvQ8Cache:
        return KvQ8Cache(self, max_seq, n_kv, head_dim)

    def runner(self, cfg: RunnerConfig, layers: Sequence[RunnerLayer], output_norm: int,
               lm_head: GpuPackedTensor, embed: GpuPackedTensor) -> DecodeRunner:
        """``vxt_hip_runner_create`` over uploaded tensors and device norms."""
        arr = (RunnerLayer * max(1, len(layers)))(*layers)
        buf = _errbuf()
        h = load_library().vxt_hip_runner_create(self.ctx, C.byref(cfg), arr, output_norm, lm_head.handle,
                                                 embed.handle, buf, len(buf))
        if not h:
            _upload_failed(buf)
        return DecodeRunner(self, h, cfg)

    # -- device-pointer calls (asynchronous on `stream`) ----------------------
    def matmul_dev(self, t: GpuPackedTensor, x_ptr: int, x_dtype: int, batch_m: int, y_ptr: int,
                   y_dtype: int, stream: int = 0) -> None:
        buf = _errbuf()
        _check(load_library().vxt_hip_matmul_dev(self.ctx, t.handle, x_ptr, x_dtype, batch_m,
                                                 y_ptr, y_dtype, stream or None, buf, len(buf)), buf)

    def read_probe_dev(self, ptr: int, nbytes: int, key: int = 1, stream: int = 0) -> None:
        """``vxt_hip_read_probe_dev``: read nbytes at ptr once (HBM floor probe)."""
        buf = _errbuf()
        _check(load_library().vxt_hip_read_probe_dev(self.ctx, ptr, int(nbytes), int(key), stream or None, buf,
                                                     len(buf)), buf)

    def matmul_noalloc_dev(self, t: GpuPackedTensor, x_ptr: int, x_dtype: int, batch_m: int, y_ptr: int,
                           y_dtype: int, stream: int = 0) -> None:
        """``vxt_hip_matmul_noalloc_dev``: matmul_dev without any device
        allocation (fixed 32 MiB scratch per GPU; larger GEMMs raise)."""
        buf = _errbuf()
        _check(load_library().vxt_hip_matmul_noalloc_dev(self.ctx, t.handle, x_ptr, x_dtype, batch_m,
                                                         y_ptr, y_dtype, stream or None, buf, len(buf)), buf)

    def matmul_multi_dev(self, ts: Sequence[GpuPackedTensor], x_ptr: int, x_dtype: int,
                         batch_m: int, y_ptrs: Iterable[int], y_dtype: int, stream: int = 0) -> None:
        ys = list(y_ptrs)
        ta = (C.c_void_p * len(ts))(*[t.handle for t in ts])
        ya = (C.c_void_p * len(ys))(*ys)
        buf = _errbuf()
        _check(load_library().vxt_hip_matmul_multi_dev(self.ctx, ta, len(ts), x_ptr, x_dtype,
                                                       batch_m, ya, y_dtype, stream or None, buf,
                                                       len(buf)), buf)

    def greedy_dev(self, logits_ptr: int, n: int, out_ptr: int, stream: int = 0) -> None:
        """``out[0]`` = the lowest index of the largest non-NaN logit (0 when
        none is above -inf), ``out[1]`` = 1 if any logit is NaN or +-inf: the
        runner's greedy step (``vxt_greedy_exact``, vxt_llm_ops.metal:569-600)
        and the CPU sampler's greedy branch (llm_ops.rs:318-327).  One launch,
        no allocation; capturable."""
        buf = _errbuf()
        _check(load_library().vxt_hip_greedy_dev(self.ctx, logits_ptr or None, n, out_ptr or None,
                                                 stream or None, buf, len(buf)), buf)

    def ffn_glu_dev(self, t: GpuPackedTensor, x_ptr: int, x_dtype: int, batch_m: int, act_ptr: int,
                    act_dtype: int, act_stride: int | None = None, activation: int = ACT_SILU,
                    stream: int = 0) -> None:
        """Gated FFN projection over a ``[gate; up]`` tensor
        (``vxt_hip_ffn_glu_dev``): ``act = act(gate . x) * (up . x)``, the
        fused gate/up kernel of the device runner (vxt_cb4_fast.metal:212-287)."""
        buf = _errbuf()
        stride = t.rows // 2 if act_stride is None else act_stride
        _check(load_library().vxt_hip_ffn_glu_dev(self.ctx, t.handle, x_ptr or None, x_dtype, batch_m,
                                                  act_ptr or None, act_dtype, stride, activation,
                                                  stream or None, buf, len(buf)), buf)

    def norm_matmul_dev(self, t: GpuPackedTensor, cur_ptr: int, delta_ptr: int, weight_ptr: int, eps: float,
                        cur_out_ptr: int, mode: int, y_ptr: int, y_dtype: int, y_stride: int | None = None,
                        stream: int = 0) -> None:
        """Batch-1 projection of ``bf16(rms_norm(cur [+ delta]) * w)`` in one
        launch (``vxt_hip_norm_matmul_dev``); with ``delta_ptr`` the sum goes
        to ``cur_out_ptr``."""
        buf = _errbuf()
        stride = (t.rows // 2 if mode != NORM_PLAIN else t.rows) if y_stride is None else y_stride
        _check(load_library().vxt_hip_norm_matmul_dev(self.ctx, t.handle, cur_ptr or None, delta_ptr or None,
                                                      weight_ptr or None, eps, cur_out_ptr or None, mode,
                                                      y_ptr or None, y_dtype, stride, stream or None, buf,
                                                      len(buf)), buf)

    def rms_norm_dev(self, cur_ptr: int, delta_ptr: int, weight_ptr: int, out_ptr: int, out_dtype: int,
                     dim: int, stride: int | None = None, batch_m: int = 1, eps: float = 1e-6,
                     stream: int = 0) -> None:
        """``cur += delta`` (when ``delta_ptr``) then ``out = rms_norm(cur) * weight``
        (``vxt_hip_rms_norm_dev``; llm_ops.rs:48-57 after llm_cpu.rs:443-446)."""
        buf = _errbuf()
        _check(load_library().vxt_hip_rms_norm_dev(self.ctx, cur_ptr or None, delta_ptr or None,
                                                   weight_ptr or None, out_ptr or None, out_dtype, dim,
                                                   dim if stride is None else stride, batch_m, eps,
                                                   stream or None, buf, len(buf)), buf)

    def embed_dev(self, t: GpuPackedTensor, tokens_ptr: int, batch_m: int, out_ptr: int,
                  out_stride: int | None = None, embed_scale: float = 1.0, stream: int = 0) -> None:
        """f32 embedding rows of ``batch_m`` device-resident token ids
        (``vxt_hip_embed_dev``): bit-exact ``decode_row``, scaled as
        llm_cpu.rs:224-229, zero-padded to ``out_stride``; ids past the last
        row read the last row."""
        buf = _errbuf()
        stride = t.cols if out_stride is None else out_stride
        _check(load_library().vxt_hip_embed_dev(self.ctx, t.handle, tokens_ptr or None, batch_m,
                                                embed_scale, out_ptr or None, stride, stream or None,
                                                buf, len(buf)), buf)

    def dequant_rows_dev(self, t: GpuPackedTensor, row0: int, nrows: int, out_ptr: int,
                         stream: int = 0) -> None:
        buf = _errbuf()
        _check(load_library().vxt_hip_dequant_rows_dev(self.ctx, t.handle, row0, nrows, out_ptr,
                                                       stream or None, buf, len(buf)), buf)
