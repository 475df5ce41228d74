"""CPU parity oracle for the compressed-weight matmul path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker or the timed CPU
baseline.  The product (``vxg_amd``) never imports it.

The arithmetic lives in ``oracle/vxt_oracle.c`` (built by ``oracle/Makefile``
into ``oracle/liboracle_vxt.so``); each C function cites the reference
(``crates/vxg-tensor``) lines it restates.  This module only marshals numpy
arrays through ctypes.

Parity status of every function, and the checks that pin it, are listed in
``tests/test_oracle_pinning.py``'s module docstring.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle_vxt.so")

KIND_CB4, KIND_G64, KIND_Q8, KIND_Q40 = 1, 2, 3, 4

_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc; runs where gcc exists)."""
    if force and os.path.exists(LIB_PATH):
        os.remove(LIB_PATH)
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle_vxt.so"], check=True)
    return LIB_PATH


class _Cb4(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("cols", C.c_uint32), ("padded_cols", C.c_uint32),
                ("centroids", C.c_void_p), ("scales_f16", C.c_void_p),
                ("packed_words", C.c_void_p), ("outlier_row_ptr", C.c_void_p),
                ("outliers_packed", C.c_void_p)]


class _G64(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("cols", C.c_uint32), ("padded_cols", C.c_uint32),
                ("idx", C.c_void_p), ("lut_f16", C.c_void_p)]


class _Q8(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("cols", C.c_uint32), ("blocks", C.c_void_p)]


class _Q40(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("cols", C.c_uint32), ("padded_cols", C.c_uint32),
                ("scales_f16", C.c_void_p), ("qs_words", C.c_void_p)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
        L.vxo_f16_to_f32.restype = C.c_float
        L.vxo_f16_to_f32.argtypes = [C.c_uint16]
        L.vxo_f32_to_f16.restype = C.c_uint16
        L.vxo_f32_to_f16.argtypes = [C.c_float]
        L.vxo_f32_to_bf16.restype = C.c_uint16
        L.vxo_f32_to_bf16.argtypes = [C.c_float]
        for n in ("vxo_f16_to_f32_n", "vxo_f32_to_f16_n", "vxo_bf16_to_f32_n", "vxo_f32_to_bf16_n"):
            getattr(L, n).argtypes = [vp, vp, sz]
            getattr(L, n).restype = None
        for n in ("vxo_cb4_decode_row", "vxo_g64_decode_row", "vxo_q8_decode_row", "vxo_q40_decode_row"):
            getattr(L, n).argtypes = [vp, sz, vp]
            getattr(L, n).restype = None
        for n in ("vxo_cb4_gemv", "vxo_g64_gemv", "vxo_q8_gemv", "vxo_q40_gemv"):
            getattr(L, n).argtypes = [vp, vp, vp, i32]
            getattr(L, n).restype = None
        L.vxo_q40_encode.argtypes = [C.c_uint32, C.c_uint32, vp, vp, vp]
        L.vxo_q40_encode.restype = None
        L.vxo_q8_quantize.argtypes = [vp, vp]
        L.vxo_q8_quantize.restype = None
        L.vxo_q8_dot_f32.argtypes = [vp, vp]
        L.vxo_q8_dot_f32.restype = C.c_float
        L.vxo_q8_axpy_f32.argtypes = [vp, C.c_float, vp]
        L.vxo_q8_axpy_f32.restype = None
        L.vxo_q8_dequant.argtypes = [vp, sz, vp]
        L.vxo_q8_dequant.restype = None
        L.vxo_gemm.argtypes = [i32, vp, vp, sz, vp, i32]
        L.vxo_gemm.restype = None
        L.vxo_gemv_any.argtypes = [i32, vp, vp, vp, i32]
        L.vxo_gemv_any.restype = None
        L.vxo_hardware_threads.restype = C.c_int
        L.vxo_silu.argtypes = [C.c_float]
        L.vxo_silu.restype = C.c_float
        L.vxo_gelu_tanh.argtypes = [C.c_float]
        L.vxo_gelu_tanh.restype = C.c_float
        L.vxo_glu.argtypes = [vp, vp, sz, i32, vp]
        L.vxo_glu.restype = None
        L.vxo_rms_norm.argtypes = [vp, vp, sz, C.c_float, vp]
        L.vxo_rms_norm.restype = None
        L.vxo_attn_q8.argtypes = [vp, vp, vp, sz, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp]
        L.vxo_attn_q8.restype = None
        L.vxo_apply_rope.argtypes = [vp, sz, sz, sz, C.c_float, i32]
        L.vxo_apply_rope.restype = None
        gqa = [vp, vp, vp, vp, vp, i32, C.c_uint32, C.c_uint32, C.c_uint32, sz, sz, sz, C.c_float, i32, C.c_float,
               vp, vp]
        L.vxo_gqa_prep_q8.argtypes = gqa + [vp, vp]
        L.vxo_gqa_prep_q8.restype = None
        L.vxo_gqa_step_q8.argtypes = gqa + [vp]
        L.vxo_gqa_step_q8.restype = None
        L.vxo_greedy.argtypes = [vp, sz, C.POINTER(C.c_uint32)]
        L.vxo_greedy.restype = C.c_uint32
        _lib = L
    return _lib


def hardware_threads() -> int:
    return int(lib().vxo_hardware_threads())


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# --------------------------------------------------------------------------
# conversions
# --------------------------------------------------------------------------

def f16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().vxo_f16_to_f32_n(_ptr(b), _ptr(out), b.size)
    return out


def f32_to_f16(vals) -> np.ndarray:
    v = np.ascontiguousarray(vals, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint16)
    lib().vxo_f32_to_f16_n(_ptr(v), _ptr(out), v.size)
    return out


def bf16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().vxo_bf16_to_f32_n(_ptr(b), _ptr(out), b.size)
    return out


def f32_to_bf16(vals) -> np.ndarray:
    v = np.ascontiguousarray(vals, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint16)
    lib().vxo_f32_to_bf16_n(_ptr(v), _ptr(out), v.size)
    return out


# --------------------------------------------------------------------------
# matrix views (the arrays are kept alive on the returned object)
# --------------------------------------------------------------------------

class _View:
    def __init__(self, kind, struct, keep):
        self.kind = kind
        self.struct = struct
        self._keep = keep

    @property
    def ptr(self):
        return C.addressof(self.struct)


def view(m) -> _View:
    k = m.kind
    if k == "cb4":
        arrs = [np.ascontiguousarray(m.centroids, dtype=np.float32),
                np.ascontiguousarray(m.scales_f16, dtype=np.uint16),
                np.ascontiguousarray(m.packed_words, dtype=np.uint32),
                np.ascontiguousarray(m.outlier_row_ptr, dtype=np.uint32),
                np.ascontiguousarray(m.outliers_packed, dtype=np.uint32)]
        if arrs[4].size == 0:
            arrs[4] = np.zeros(1, dtype=np.uint32)
        s = _Cb4(m.rows, m.cols, m.padded_cols, *[_ptr(a) for a in arrs])
        return _View(KIND_CB4, s, arrs)
    if k == "g64":
        arrs = [np.ascontiguousarray(m.idx, dtype=np.uint8),
                np.ascontiguousarray(m.lut_f16, dtype=np.uint16)]
        s = _G64(m.rows, m.cols, m.padded_cols, *[_ptr(a) for a in arrs])
        return _View(KIND_G64, s, arrs)
    if k == "q8":
        arrs = [np.ascontiguousarray(m.blocks, dtype=np.uint8)]
        s = _Q8(m.rows, m.cols, _ptr(arrs[0]))
        return _View(KIND_Q8, s, arrs)
    if k == "q4_0":
        arrs = [np.ascontiguousarray(m.scales_f16, dtype=np.uint16),
                np.ascontiguousarray(m.qs_words, dtype=np.uint32)]
        s = _Q40(m.rows, m.cols, m.padded_cols, _ptr(arrs[0]), _ptr(arrs[1]))
        return _View(KIND_Q40, s, arrs)
    raise TypeError(f"unknown matrix kind {k!r}")


_DECODE = {KIND_CB4: "vxo_cb4_decode_row", KIND_G64: "vxo_g64_decode_row",
           KIND_Q8: "vxo_q8_decode_row", KIND_Q40: "vxo_q40_decode_row"}


def decode_rows(m, row0: int = 0, nrows: int | None = None) -> np.ndarray:
    """Dequantised rows [nrows, cols] (``decode_row`` per row)."""
    v = view(m)
    nrows = m.rows - row0 if nrows is None else nrows
    out = np.zeros((nrows, m.cols), dtype=np.float32)
    fn = getattr(lib(), _DECODE[v.kind])
    for i in range(nrows):
        fn(v.ptr, row0 + i, out[i].ctypes.data)
    return out


def gemv(m, x, threads: int = 1) -> np.ndarray:
    """y[rows] = W x for f32 x[cols] (the reference GEMV of that kind)."""
    v = view(m)
    xx = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert xx.size == m.cols
    y = np.empty(m.rows, dtype=np.float32)
    lib().vxo_gemv_any(v.kind, v.ptr, _ptr(xx), _ptr(y), int(threads))
    return y


def gemv_batch(m, X, threads: int = 1) -> np.ndarray:
    """Per-token GEMV: Y[M, rows] with row m = gemv(W, X[m])."""
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, m.cols)
    return np.stack([gemv(m, X[i], threads) for i in range(X.shape[0])])


def gemm(m, X, threads: int = 1) -> np.ndarray:
    """``PackedTensor::gemm_cpu`` for batch_m >= 2: Y[M, rows] (f32)."""
    v = view(m)
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, m.cols)
    Y = np.empty((X.shape[0], m.rows), dtype=np.float32)
    lib().vxo_gemm(v.kind, v.ptr, _ptr(X), X.shape[0], _ptr(Y), int(threads))
    return Y


# --------------------------------------------------------------------------
# Q4_0 encoder
# --------------------------------------------------------------------------

def q40_encode(rows: int, cols: int, w):
    """``Q4_0Matrix::encode`` (``q4_0.rs:17-64``) of f32 weights [rows, cols]."""
    from vxg_amd.formats import Q4_0Matrix
    ww = np.ascontiguousarray(w, dtype=np.float32).reshape(rows, cols)
    bpr = (cols + 31) // 32
    sc = np.empty(rows * bpr, dtype=np.uint16)
    qs = np.empty(rows * bpr * 4, dtype=np.uint32)
    lib().vxo_q40_encode(rows, cols, _ptr(ww), _ptr(sc), _ptr(qs))
    return Q4_0Matrix(rows, cols, bpr * 32, sc, qs)


# --------------------------------------------------------------------------
# Q8 block primitives
# --------------------------------------------------------------------------

def q8_quantize(src32) -> np.ndarray:
    s = np.ascontiguousarray(src32, dtype=np.float32).reshape(32)
    blk = np.empty(34, dtype=np.uint8)
    lib().vxo_q8_quantize(_ptr(s), _ptr(blk))
    return blk


def q8_dot(blk, x32) -> float:
    b = np.ascontiguousarray(blk, dtype=np.uint8).reshape(34)
    x = np.ascontiguousarray(x32, dtype=np.float32).reshape(32)
    return float(np.float32(lib().vxo_q8_dot_f32(_ptr(b), _ptr(x))))


def q8_axpy(blk, weight: float, out32) -> np.ndarray:
    b = np.ascontiguousarray(blk, dtype=np.uint8).reshape(34)
    o = np.array(out32, dtype=np.float32).reshape(32)
    lib().vxo_q8_axpy_f32(_ptr(b), float(weight), _ptr(o))
    return o


def q8_dequant(blocks) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    assert b.size % 34 == 0
    out = np.empty(b.size // 34 * 32, dtype=np.float32)
    lib().vxo_q8_dequant(_ptr(b), b.size // 34, _ptr(out))
    return out


def greedy(logits) -> tuple[int, bool]:
    """``(id, nonfinite)`` of the greedy pick over f32 logits (vxo_greedy)."""
    a = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1)
    nf = C.c_uint32(0)
    i = lib().vxo_greedy(_ptr(a) if a.size else None, a.size, C.byref(nf))
    return int(i), bool(nf.value)


def embed_rows(m, tokens, embed_scale: float = 1.0) -> np.ndarray:
    """Token embedding rows [len(tokens), cols]: ``decode_row(token)``
    (llm_cpu.rs:223), then every value times ``embed_scale`` when
    ``|embed_scale - 1| > 1e-7`` in f32 (llm_cpu.rs:226-229; also llm.rs:
    565-569).  Ids must be < rows (the CPU path rejects others, llm_cpu.rs:
    219-221)."""
    toks = [int(t) for t in np.asarray(tokens).reshape(-1)]
    if any(t >= m.rows for t in toks):
        raise ValueError("token id out of vocab")
    out = np.zeros((len(toks), m.cols), dtype=np.float32)
    for i, t in enumerate(toks):
        out[i] = decode_rows(m, t, 1)[0]
    s = np.float32(embed_scale)
    if abs(s - np.float32(1.0)) > np.float32(1e-7):
        out = out * s
    return out


def glu(g, u, gelu: bool = False) -> np.ndarray:
    """``act(g) * u`` element-wise (vxo_glu; llm_cpu.rs:457-464)."""
    g = np.ascontiguousarray(g, dtype=np.float32).reshape(-1)
    u = np.ascontiguousarray(u, dtype=np.float32).reshape(-1)
    assert g.size == u.size
    out = np.empty_like(g)
    if g.size:
        lib().vxo_glu(_ptr(g), _ptr(u), g.size, int(gelu), _ptr(out))
    return out


def silu(x) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    return np.array([lib().vxo_silu(float(v)) for v in a], dtype=np.float32)


def gelu_tanh(x) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    return np.array([lib().vxo_gelu_tanh(float(v)) for v in a], dtype=np.float32)


def rms_norm(x, w, eps: float) -> np.ndarray:
    """``rms_norm`` of llm_ops.rs:48-57 over one row (vxo_rms_norm)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    assert w.size >= x.size
    out = np.empty_like(x)
    lib().vxo_rms_norm(_ptr(x), _ptr(w), x.size, float(eps), _ptr(out))
    return out


def kv_q8_blocks(x, n_kv: int, hd: int) -> np.ndarray:
    """One position's K or V rows as KvQ8Block bytes [n_kv * hd / 32][34]
    (the quantize loop of llm_prefill.rs:306-312)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(n_kv * hd // 32, 32)
    out = np.empty((x.shape[0], 34), dtype=np.uint8)
    for i in range(x.shape[0]):
        lib().vxo_q8_quantize(_ptr(x[i]), _ptr(out[i]))
    return out


def apply_rope(vec, pos: int, rope_dim: int, freq_base: float, neox: bool) -> np.ndarray:
    """``apply_rope`` of llm_ops.rs:81-99 on a copy of one head's vector."""
    v = np.array(vec, dtype=np.float32).reshape(-1)
    lib().vxo_apply_rope(_ptr(v), v.size, int(pos), int(rope_dim), float(freq_base), int(bool(neox)))
    return v


class GqaStep:
    """Scalar arguments of step_full_gqa_q8 (llm_prefill.rs:259-278)."""

    def __init__(self, n_head, n_kv, hd, gated=False, q_norm=None, k_norm=None, rope_dim=0,
                 freq_base=10000.0, neox=False, eps=1e-6):
        self.n_head, self.n_kv, self.hd = n_head, n_kv, hd
        self.gated, self.rope_dim, self.freq_base, self.neox, self.eps = gated, rope_dim, freq_base, neox, eps
        self.q_norm = None if q_norm is None else np.ascontiguousarray(q_norm, dtype=np.float32)
        self.k_norm = None if k_norm is None else np.ascontiguousarray(k_norm, dtype=np.float32)

    @property
    def q_rows(self):
        return self.n_head * self.hd * (2 if self.gated else 1)

    def _args(self, q_raw, k_cur, v_cur, pos, rope_pos, kb, vb):
        p = self
        return (_ptr(q_raw), _ptr(k_cur), _ptr(v_cur), None if p.q_norm is None else _ptr(p.q_norm),
                None if p.k_norm is None else _ptr(p.k_norm), int(p.gated), p.n_head, p.n_kv, p.hd, int(pos),
                int(rope_pos), int(p.rope_dim), float(p.freq_base), int(p.neox), float(p.eps), _ptr(kb), _ptr(vb))

    def _inputs(self, q_raw, k_cur, v_cur, kb, vb, pos):
        q_raw = np.ascontiguousarray(q_raw, dtype=np.float32).reshape(-1)
        k_cur = np.array(k_cur, dtype=np.float32).reshape(-1)
        v_cur = np.ascontiguousarray(v_cur, dtype=np.float32).reshape(-1)
        kvd = self.n_kv * self.hd
        assert q_raw.size == self.q_rows and k_cur.size == kvd and v_cur.size == kvd
        assert kb.dtype == np.uint8 and vb.dtype == np.uint8 and kb.flags.c_contiguous and vb.flags.c_contiguous
        assert kb.size >= (pos + 1) * kvd // 32 * 34 and vb.size == kb.size
        return q_raw, k_cur, v_cur

    def prep(self, q_raw, k_cur, v_cur, kb, vb, pos: int, rope_pos: int):
        """vxo_gqa_prep_q8: returns (q heads, gates or None, normed and rotated
        k); writes row ``pos`` of the block arrays ``kb`` / ``vb`` in place."""
        q_raw, k_cur, v_cur = self._inputs(q_raw, k_cur, v_cur, kb, vb, pos)
        qh = np.empty(self.n_head * self.hd, dtype=np.float32)
        qg = np.empty(self.n_head * self.hd, dtype=np.float32) if self.gated else None
        lib().vxo_gqa_prep_q8(*self._args(q_raw, k_cur, v_cur, pos, rope_pos, kb, vb), _ptr(qh),
                              None if qg is None else _ptr(qg))
        return qh, qg, k_cur

    def step(self, q_raw, k_cur, v_cur, kb, vb, pos: int, rope_pos: int) -> np.ndarray:
        """vxo_gqa_step_q8: one whole step; writes row ``pos`` of kb / vb."""
        q_raw, k_cur, v_cur = self._inputs(q_raw, k_cur, v_cur, kb, vb, pos)
        out = np.empty(self.n_head * self.hd, dtype=np.float32)
        lib().vxo_gqa_step_q8(*self._args(q_raw, k_cur, v_cur, pos, rope_pos, kb, vb), _ptr(out))
        return out


def attn_q8(q, k_blocks, v_blocks, seq_len: int, n_head: int, n_kv: int, hd: int, gate=None) -> np.ndarray:
    """Attention of one decode step over a Q8 cache (vxo_attn_q8)."""
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
    kb = np.ascontiguousarray(k_blocks, dtype=np.uint8).reshape(-1)
    vb = np.ascontiguousarray(v_blocks, dtype=np.uint8).reshape(-1)
    assert q.size == n_head * hd and kb.size >= seq_len * n_kv * hd // 32 * 34 and vb.size == kb.size
    g = None if gate is None else np.ascontiguousarray(gate, dtype=np.float32).reshape(-1)
    out = np.empty(n_head * hd, dtype=np.float32)
    lib().vxo_attn_q8(_ptr(q), _ptr(kb), _ptr(vb), seq_len, n_head, n_kv, hd,
                      None if g is None else _ptr(g), _ptr(out))
    return out
