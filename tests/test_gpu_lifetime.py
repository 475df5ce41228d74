"""Handle lifetimes and the context workspace.

* Releasing a tensor, graph or device buffer after its engine was closed is a
  no-op: closing the context released them (the C library keeps a registry of
  live handles and never dereferences a stale one).
* A graph captured before the workspace grows keeps replaying correctly: the
  workspace it recorded stays allocated until the context is destroyed.
* Growing the workspace inside a stream capture is refused with VXT_E_ARG.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from vxg_amd import engine, synth
from vxg_amd.formats import bf16_bits_to_f32

from parity_util import THREADS, assert_bits_equal

pytestmark = pytest.mark.gpu


def test_release_after_close_is_a_no_op():
    print("lifetime: release after close", flush=True)
    eng = engine.HipEngine(0)
    m = synth.make_g64(64, 256, seed=1)
    t = eng.upload_packed(m)
    xd = eng.to_device(synth.make_x_bf16(16, 256, seed=2))
    yd = eng.alloc(16 * 64 * 4)
    eng.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 16, yd.ptr, engine.DTYPE_F32, eng.stream)   # sizes the workspace
    eng.synchronize()
    g = eng.capture(lambda s: eng.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 16, yd.ptr, engine.DTYPE_F32, s))
    g.launch(2)
    handles = (t.handle, g.handle)
    eng.close()
    g.free()
    t.free()
    xd.free()
    yd.free()
    lib = engine.load_library()
    lib.vxt_hip_graph_free(handles[1])   # stale in C too: still a no-op
    lib.vxt_hip_free_tensor(handles[0])
    assert lib.vxt_hip_tensor_info(handles[0], None, None, None, None) == engine.VXT_E_ARG
    buf = C.create_string_buffer(256)
    assert lib.vxt_hip_graph_launch(None, handles[1], 1, None, buf, len(buf)) == engine.VXT_E_ARG


def test_graph_survives_workspace_growth():
    """Capture a small GEMM, run a larger one eagerly (the workspace grows),
    then replay the graph: it still produces the small GEMM's eager bits."""
    print("lifetime: graph after workspace growth", flush=True)
    eng = engine.HipEngine(0)
    try:
        small = synth.make_g64(96, 320, seed=3)
        big = synth.make_cb4(1024, 2048, seed=4)
        ts, tb = eng.upload_packed(small), eng.upload_packed(big)
        xs_h = synth.make_x_bf16(24, 320, seed=5)
        xs = eng.to_device(xs_h)
        ys = eng.alloc(24 * 96 * 4)
        eng.matmul_dev(ts, xs.ptr, engine.DTYPE_BF16, 24, ys.ptr, engine.DTYPE_F32, eng.stream)   # sizes the workspace
        eng.synchronize()
        want = ys.download(np.float32, (24, 96))
        g = eng.capture(lambda s: eng.matmul_dev(ts, xs.ptr, engine.DTYPE_BF16, 24, ys.ptr, engine.DTYPE_F32, s))
        xb = eng.to_device(synth.make_x_bf16(600, 2048, seed=6))
        yb = eng.alloc(600 * 1024 * 4)
        eng.matmul_dev(tb, xb.ptr, engine.DTYPE_BF16, 600, yb.ptr, engine.DTYPE_F32, eng.stream)   # grows it
        eng.synchronize()
        ys.upload(np.zeros(24 * 96, np.float32))
        for _ in range(3):
            g.launch(1)
            got = ys.download(np.float32, (24, 96))
            assert_bits_equal(got, want)
        X = bf16_bits_to_f32(xs_h).reshape(24, 320)
        ref = oracle.gemm(small, X, threads=THREADS)
        assert np.max(np.abs(got - ref)) <= 1e-3 * np.max(np.abs(ref))
        g.free()
    finally:
        eng.close()


def test_workspace_growth_inside_capture_is_refused():
    print("lifetime: growth inside capture", flush=True)
    eng = engine.HipEngine(0)
    try:
        m = synth.make_q8(512, 1024, seed=7)
        t = eng.upload_packed(m)
        xd = eng.to_device(synth.make_x_bf16(300, 1024, seed=8))
        yd = eng.alloc(300 * 512 * 4)
        with pytest.raises(engine.BackendError) as ei:
            eng.capture(lambda s: eng.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 300, yd.ptr, engine.DTYPE_F32, s))
        assert ei.value.code == engine.VXT_E_ARG
        # the context stays usable: size the workspace eagerly, then capture
        eng.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 300, yd.ptr, engine.DTYPE_F32, eng.stream)
        eng.synchronize()
        want = yd.download(np.float32, (300, 512))
        g = eng.capture(lambda s: eng.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 300, yd.ptr, engine.DTYPE_F32, s))
        yd.upload(np.zeros(300 * 512, np.float32))
        g.launch(1)
        assert_bits_equal(yd.download(np.float32, (300, 512)), want)
        g.free()
    finally:
        eng.close()


def test_read_probe_runs_and_checks_sizes():
    """The streaming-floor probe reads a buffer and rejects sizes that are not
    a positive multiple of 16."""
    eng = engine.HipEngine(0)
    try:
        b = eng.alloc(1 << 20)
        eng.read_probe_dev(b.ptr, 1 << 20, 1, eng.stream)
        eng.synchronize()
        for bad in (0, 100):
            with pytest.raises(engine.BackendError) as ei:
                eng.read_probe_dev(b.ptr, bad, 1, eng.stream)
            assert ei.value.code == engine.VXT_E_SHAPE
        b.free()
    finally:
        eng.close()
