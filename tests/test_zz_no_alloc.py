"""The allocation-free matmul entry point (vxt_hip_matmul_noalloc_dev).

It runs the same kernels as vxt_hip_matmul_dev with a fixed scratch array
in device memory instead of the context workspace, so its outputs must equal
matmul_dev's bit for bit.  Checked on two calls in a row (the second with a
smaller input, which reuses the array as the first left it), for the GEMV
and the fused and two-phase GEMM paths, inside a captured graph that no
eager call sized first, and for the clean refusal of a GEMM too large for
the array.
"""
import numpy as np
import pytest

from vxg_amd import engine, synth

from parity_util import assert_bits_equal

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine(0)
    yield e
    e.close()


def both(eng, t, xh, x_dtype, M):
    """(matmul_dev output, matmul_noalloc_dev output) for the same inputs."""
    xd = eng.to_device(xh)
    ya, yb = eng.alloc(M * t.rows * 4), eng.alloc(M * t.rows * 4)
    eng.matmul_dev(t, xd.ptr, x_dtype, M, ya.ptr, engine.DTYPE_F32, eng.stream)
    eng.matmul_noalloc_dev(t, xd.ptr, x_dtype, M, yb.ptr, engine.DTYPE_F32, eng.stream)
    eng.synchronize()
    a, b = ya.download(np.float32, (M, t.rows)), yb.download(np.float32, (M, t.rows))
    for buf in (xd, ya, yb):
        buf.free()
    return a, b


CASES = [
    # kind, rows, cols, x dtype, M of the first call, M of the second (smaller) call
    ("g64", 6144, 2048, "bf16", 128, 40),    # fused GEMM
    ("q8", 2048, 2048, "bf16", 200, 16),     # fused GEMM (Q8)
    ("cb4", 1024, 1536, "bf16", 96, 12),     # two-phase GEMM (panel + own dense kernel)
    ("q8", 512, 768, "f32", 64, 9),          # two-phase, f32 activations (hi/lo)
    ("g64", 6144, 2048, "bf16", 8, 1),       # GEMV (no scratch)
]


@pytest.mark.parametrize("kind,rows,cols,xdt,m1,m2", CASES)
def test_noalloc_matches_matmul_dev_on_two_calls(eng, kind, rows, cols, xdt, m1, m2):
    print(f"noalloc kind={kind} {rows}x{cols} x={xdt} M={m1},{m2}", flush=True)
    gen = {"g64": synth.make_g64, "q8": synth.make_q8, "cb4": synth.make_cb4}[kind]
    t = eng.upload_packed(gen(rows, cols, seed=rows + m1))
    dt = engine.DTYPE_BF16 if xdt == "bf16" else engine.DTYPE_F32
    make_x = synth.make_x_bf16 if xdt == "bf16" else synth.make_x_f32
    for M in (m1, m2):
        a, b = both(eng, t, make_x(M, cols, seed=M), dt, M)
        assert np.all(np.isfinite(a))
        assert_bits_equal(b, a)
    t.free()


def test_noalloc_in_a_graph_without_a_sizing_call():
    """A fresh context: the first call of this shape is captured (matmul_dev
    would refuse to grow its workspace there); replays equal the eager
    matmul_dev result."""
    print("noalloc graph capture", flush=True)
    e = engine.HipEngine(0)
    try:
        t = e.upload_packed(synth.make_g64(2048, 2048, seed=5))
        xh = synth.make_x_bf16(64, 2048, seed=6)
        xd = e.to_device(xh)
        y = e.alloc(64 * 2048 * 4)
        g = e.capture(lambda s: e.matmul_noalloc_dev(t, xd.ptr, engine.DTYPE_BF16, 64, y.ptr, engine.DTYPE_F32, s))
        outs = []
        for _ in range(3):
            y.upload(np.zeros(64 * 2048, np.float32))
            g.launch(1)
            outs.append(y.download(np.float32, (64, 2048)))
        g.free()
        ref = e.alloc(64 * 2048 * 4)
        e.matmul_dev(t, xd.ptr, engine.DTYPE_BF16, 64, ref.ptr, engine.DTYPE_F32, e.stream)
        e.synchronize()
        want = ref.download(np.float32, (64, 2048))
        for o in outs:
            assert_bits_equal(o, want)
    finally:
        e.close()


def test_noalloc_refuses_a_gemm_larger_than_its_scratch(eng):
    print("noalloc too large", flush=True)
    t = eng.upload_packed(synth.make_cb4(6144, 2048, seed=9))
    xd = eng.to_device(synth.make_x_bf16(1024, 2048, seed=9))
    yd = eng.alloc(1024 * 6144 * 4)
    with pytest.raises(engine.BackendError) as ei:
        eng.matmul_noalloc_dev(t, xd.ptr, engine.DTYPE_BF16, 1024, yd.ptr, engine.DTYPE_F32, eng.stream)
    assert ei.value.code == engine.VXT_E_SHAPE and "scratch" in str(ei.value)
    for b in (xd, yd):
        b.free()
    t.free()
