"""CPU-side checks of the C ABI library and the host-side containers.

No compute call is made here (there is no GPU in the build container): the
library must load, export every symbol ``include/vxt_hip.h`` declares, and
fail cleanly -- with a message, not a crash -- when no device is present.
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

from vxg_amd import engine, synth
from vxg_amd.formats import CodebookMatrix, FormatError, Q8Matrix

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vxt_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"VXT_API\s+[\w\*\s]+?\b(vxt_hip_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    syms = declared_symbols()
    assert len(syms) == len(engine.ABI_SYMBOLS)
    assert set(syms) == set(engine.ABI_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = engine.load_library()
    for s in declared_symbols():
        assert hasattr(lib, s), s


def _needed(path):
    """DT_NEEDED entries of an ELF shared library built here (readelf -d)."""
    import subprocess
    out = subprocess.run(["readelf", "-d", path], capture_output=True, text=True, check=True).stdout
    return re.findall(r"\(NEEDED\)\s+Shared library: \[([^\]]+)\]", out)


def test_vendor_gemm_library_is_a_separate_plugin():
    # The matmul library does not link hipBLASLt; the pinned comparison
    # path's plugin beside it does, and exports what blas_plugin.cpp looks up.
    lib_dir = os.path.join(ROOT, "vxg_amd")
    main = os.path.join(lib_dir, "libvxt_hip.so")
    plugin = os.path.join(lib_dir, "libvxt_hip_blas.so")
    engine.load_library()
    assert not any("hipblaslt" in n for n in _needed(main)), _needed(main)
    assert any("hipblaslt" in n for n in _needed(plugin))
    import subprocess
    syms = subprocess.run(["nm", "-D", "--defined-only", plugin], capture_output=True, text=True,
                          check=True).stdout
    for s in ("vxt_blas_gemm_f16_tn", "vxt_blas_release_device"):
        assert re.search(rf"\bT {s}$", syms, re.M), s


def test_no_cpu_fallback_without_device():
    # Construction must raise (no silent host path) when no GPU is visible.
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is visible")
    except ImportError:
        pass
    with pytest.raises(engine.BackendError) as ei:
        engine.HipEngine()
    assert ei.value.code == engine.VXT_E_DEVICE


def test_null_handles_are_rejected_without_a_device():
    lib = engine.load_library()
    buf = C.create_string_buffer(256)
    # null context: a clean error code and message, no dereference
    assert lib.vxt_hip_upload_q8_0(None, 1, 32, None, 0, buf, len(buf)) is None
    assert b"null" in buf.value
    rc = lib.vxt_hip_matmul_dev(None, None, None, 0, 1, None, 0, None, buf, len(buf))
    assert rc == engine.VXT_E_ARG and b"null" in buf.value
    rc = lib.vxt_hip_run_multi(None, None, 0, None, 0, 1, None, buf, len(buf))
    assert rc == engine.VXT_E_ARG
    assert lib.vxt_hip_tensor_info(None, None, None, None, None) == engine.VXT_E_ARG
    lib.vxt_hip_free_tensor(None)   # no-ops
    lib.vxt_hip_destroy(None)
    ms = C.c_double()
    assert lib.vxt_hip_last_kernel_ms(None, C.byref(ms)) == engine.VXT_E_ARG


def test_stale_handles_are_rejected_without_a_device():
    """Handles the library never issued (or already released) are looked up,
    not dereferenced: releases are no-ops, calls fail with VXT_E_ARG."""
    lib = engine.load_library()
    buf = C.create_string_buffer(256)
    bogus = C.c_void_p(0x1000)
    lib.vxt_hip_free_tensor(bogus)
    lib.vxt_hip_graph_free(bogus)
    lib.vxt_hip_destroy(bogus)
    lib.vxt_hip_device_free(bogus, bogus)
    assert lib.vxt_hip_stream(bogus) is None
    assert lib.vxt_hip_tensor_info(bogus, None, None, None, None) == engine.VXT_E_ARG
    assert lib.vxt_hip_set_gemm_path(bogus, 0) == engine.VXT_E_ARG
    rc = lib.vxt_hip_matmul_dev(bogus, bogus, bogus, 0, 1, bogus, 0, None, buf, len(buf))
    assert rc == engine.VXT_E_ARG and b"context" in buf.value
    rc = lib.vxt_hip_graph_launch(bogus, bogus, 1, None, buf, len(buf))
    assert rc == engine.VXT_E_ARG


def test_codebook_validation_mirrors_archive_reader():
    m = synth.make_cb4(7, 300, seed=3)
    m.validate()
    bad = CodebookMatrix(**{**m.__dict__, "scales_f16": m.scales_f16[:-1]})
    with pytest.raises(FormatError, match="plane lengths"):
        bad.validate()
    rp = m.outlier_row_ptr.copy()
    rp[2], rp[3] = rp[3] + 1, rp[2]
    with pytest.raises(FormatError):
        CodebookMatrix(**{**m.__dict__, "outlier_row_ptr": rp}).validate()
    if m.outliers_packed.size:
        op = m.outliers_packed.copy()
        op[0] = (op[0] & 0xFFFF0000) | 300     # col == cols
        with pytest.raises(FormatError, match="CSR"):
            CodebookMatrix(**{**m.__dict__, "outliers_packed": op}).validate()
    with pytest.raises(FormatError, match="padded_cols"):
        CodebookMatrix(**{**m.__dict__, "padded_cols": 200}).validate()


def test_q8_container_round_trip():
    m = synth.make_q8(3, 70, seed=1)
    m.validate()
    assert m.blocks.size == 3 * 3 * 34
    assert m.qs().shape == (9, 32)
    assert np.all(m.qs()[:, :][2::3, 6:] == 0)   # padding columns of the tail block
    with pytest.raises(FormatError):
        Q8Matrix(3, 70, m.blocks[:-1]).validate()
