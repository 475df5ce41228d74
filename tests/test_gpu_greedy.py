"""GPU parity of greedy token selection (``vxt_hip_greedy_dev``).

Expected values: the oracle's restatement of the CPU sampler's greedy branch
(llm_ops.rs:318-327) plus the non-finite flag of vxt_greedy_exact
(vxt_llm_ops.metal:569-600), which the oracle pinning tests tie to the
reference's own tie cases (metal_llm_tests.rs:95-117).  Index results are
compared exactly.
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine
from parity_util import GREEDY_REFERENCE_CASES, greedy_reference_logits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


def logits_with_ties(n, seed):
    """Rounded normals (many exact ties), the maximum repeated in distant blocks."""
    g = np.random.default_rng(seed)
    a = np.round(g.standard_normal(n) * 4).astype(np.float32)
    if n > 8:
        top = np.float32(a.max() + 1)
        for i in sorted(set(g.integers(0, n, 3).tolist())):
            a[i] = top
    return a


@pytest.mark.parametrize("case", range(len(GREEDY_REFERENCE_CASES)))
def test_reference_tie_cases(eng, case):
    c = GREEDY_REFERENCE_CASES[case]
    got = eng.greedy(greedy_reference_logits(c))
    assert got == (c[2], c[3])


@pytest.mark.parametrize("n", [0, 1, 2, 3, 4, 5, 7, 8, 255, 256, 1023, 1024, 1025, 4095, 4096, 4097,
                               16383, 151936, 151937, 196608, 196609, 196612, 262147])
def test_sizes_and_ties(eng, n):
    print(f"greedy n={n}", flush=True)
    a = logits_with_ties(n, seed=n)
    assert eng.greedy(a) == oracle.greedy(a)


@pytest.mark.parametrize("n", [1000, 151936])
def test_nonfinite_mixtures(eng, n):
    g = np.random.default_rng(n + 1)
    for trial in range(12):
        a = g.standard_normal(n).astype(np.float32)
        if trial & 1:
            a[g.integers(0, n, 4)] = np.nan
        if trial & 2:
            a[g.integers(0, n, 2)] = np.inf
        if trial & 4:
            a[g.integers(0, n, 5)] = -np.inf
        if trial & 8:
            a[:] = np.nan
            a[g.integers(0, n, 3)] = -np.inf
        assert eng.greedy(a) == oracle.greedy(a), trial


def test_signed_zero_and_denormals(eng):
    a = np.full(5000, -0.0, dtype=np.float32)
    a[4999] = 0.0
    assert eng.greedy(a) == (0, False)
    a = np.zeros(5000, dtype=np.float32)
    a[3000] = np.float32(1e-45)     # the smallest denormal beats +0
    a[4000] = np.float32(1e-45)
    assert eng.greedy(a) == (3000, False) == oracle.greedy(a)
    a = np.full(5000, -np.float32(1e-45))
    a[4321] = -0.0
    assert eng.greedy(a) == (4321, False) == oracle.greedy(a)


def test_grid_stride_beyond_one_pass(eng):
    """More logits than the largest grid covers in one pass (4 Mi floats)."""
    n = 6_000_003
    a = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    a[5_500_000] = a[4_400_000] = a[6_000_001] = 50.0
    assert eng.greedy(a) == (4_400_000, False) == oracle.greedy(a)


@pytest.mark.parametrize("offset", [4, 8, 12])
def test_unaligned_logits(eng, offset):
    n = 70_001
    a = logits_with_ties(n, seed=offset)
    padded = np.zeros(n + 4, dtype=np.float32)
    padded[offset // 4:offset // 4 + n] = a
    src, out = eng.to_device(padded), eng.alloc(8)
    try:
        eng.greedy_dev(src.ptr + offset, n, out.ptr, eng.stream)
        eng.synchronize()
        r = out.download(np.uint32, (2,))
    finally:
        src.free()
        out.free()
    assert (int(r[0]), bool(r[1])) == oracle.greedy(a)


def test_state_resets_between_calls(eng):
    """A call leaves nothing behind: a smaller maximum and no flag next time,
    on both the one-launch path (up to 48 blocks of 4096 logits) and the
    partials path."""
    big = np.zeros(300_000, dtype=np.float32)
    big[7] = 1e30
    big[11] = np.nan
    mid = np.zeros(150_000, dtype=np.float32)
    mid[149_999] = 1e20
    mid[3] = -np.inf
    small = np.full(1000, -5.0, dtype=np.float32)
    small[999] = -1.0
    for _ in range(3):
        assert eng.greedy(big) == (7, True)
        assert eng.greedy(mid) == (149_999, True)
        assert eng.greedy(small) == (999, False)
        assert eng.greedy(np.zeros(0, np.float32)) == (0, False)


@pytest.mark.parametrize("n", [151_936, 262_144])
def test_captured_graph_replays(eng, n):
    src, out = eng.alloc(n * 4), eng.alloc(8)
    try:
        g = eng.capture(lambda s: eng.greedy_dev(src.ptr, n, out.ptr, s))
        try:
            for seed in range(4):
                a = logits_with_ties(n, seed=100 + seed)
                if seed == 2:
                    a[17] = np.nan
                src.upload(a)
                g.launch(1)
                r = out.download(np.uint32, (2,))
                assert (int(r[0]), bool(r[1])) == oracle.greedy(a), seed
                eng.greedy_dev(src.ptr, n, out.ptr, eng.stream)   # eager call between replays
                eng.synchronize()
                r2 = out.download(np.uint32, (2,))
                assert (int(r2[0]), bool(r2[1])) == oracle.greedy(a), seed
        finally:
            g.free()
    finally:
        src.free()
        out.free()


def test_argument_errors(eng):
    buf = eng.alloc(64)
    try:
        with pytest.raises(engine.BackendError) as e:
            eng.greedy_dev(buf.ptr, 4, 0, eng.stream)
        assert e.value.code == engine.VXT_E_ARG
        with pytest.raises(engine.BackendError) as e:
            eng.greedy_dev(buf.ptr + 2, 4, buf.ptr + 32, eng.stream)
        assert e.value.code == engine.VXT_E_ARG
        with pytest.raises(engine.BackendError) as e:
            eng.greedy_dev(buf.ptr, 1 << 31, buf.ptr + 32, eng.stream)
        assert e.value.code == engine.VXT_E_SHAPE
        with pytest.raises(engine.BackendError) as e:
            eng.greedy_dev(0, 5, buf.ptr, eng.stream)
        assert e.value.code == engine.VXT_E_ARG
        eng.greedy_dev(0, 0, buf.ptr, eng.stream)      # empty input needs no logits
        eng.synchronize()
        assert buf.download(np.uint32, (2,)).tolist() == [0, 0]
    finally:
        buf.free()
