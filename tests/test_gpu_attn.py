"""GPU parity of the Q8_0 KV cache (``vxt_hip_kv_q8_append_dev``) and the
decode attention over it (``vxt_hip_attn_q8_dev``).

Append: every value and scale bit-equal to KvQ8Block::quantize (the oracle,
llm_prefill.rs:27-42), special values included.  Attention: against the
oracle's restatement of step_full_gqa_q8's scoring, softmax and
accumulation (llm_prefill.rs:315-367) on the same cache bytes.  The output
of a head is a convex combination of V rows, so the bar is absolute in units
of the largest |V|: |out - ref| <= 1e-4 max|V| (fp32 sums in another order,
expf).
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


def append_all(eng, cache, K, V):
    kd, vd = eng.to_device(K), eng.to_device(V)
    per = cache.n_kv * cache.head_dim
    try:
        for t in range(K.shape[0]):
            cache.append(kd.ptr + 4 * t * per, vd.ptr + 4 * t * per, t, eng.stream)
        eng.synchronize()
    finally:
        kd.free()
        vd.free()


@pytest.mark.parametrize("n_kv,hd", [(1, 32), (4, 64), (16, 128), (2, 256)])
def test_append_bit_exact(eng, n_kv, hd):
    rng = np.random.default_rng(hd)
    seq = 6
    K = rng.standard_normal((seq, n_kv * hd)).astype(np.float32) * 3
    V = rng.standard_normal((seq, n_kv * hd)).astype(np.float32)
    K[1, :32] = 0                                 # zero block: d = 0, q = 0
    K[2, 5] = np.nan                              # NaN ignored by amax, quantises to 0
    V[2, :32] = np.float32(1e-6)                  # subnormal f16 scale
    V[3, min(40, n_kv * hd - 1)] = np.inf       # inf: scale inf, the block quantises to 0
    K[4, :32] = np.float32(3e6)                   # scale overflows f16 to inf
    K[5, 0] = -0.0
    cache = eng.kv_q8_cache(8, n_kv, hd)
    append_all(eng, cache, K, V)
    for which, X in (("k", K), ("v", V)):
        got = cache.blocks(which, seq)
        want = np.stack([oracle.kv_q8_blocks(X[t], n_kv, hd) for t in range(seq)])
        assert np.array_equal(got, want), which
    cache.free()


def f16_boundary_amaxes():
    """Block maxima whose scale amax / 127 lands on, next to and between f16
    rounding boundaries: ties between neighbouring f16 values (normal and
    subnormal, both parities), one f32 ulp either side, the largest finite
    f16 and the overflow threshold, and the underflow threshold 2^-25."""
    h = np.concatenate([np.arange(1, 64), np.arange(1000, 1040), np.arange(0x0400 - 8, 0x0400 + 8),
                        np.arange(0x3bf0, 0x3c10), np.arange(0x5000, 0x5010), np.arange(0x7bf0, 0x7bff)])
    lo = oracle.f16_to_f32(h.astype(np.uint16)).astype(np.float64)
    hi = oracle.f16_to_f32((h + 1).astype(np.uint16)).astype(np.float64)
    mids = np.float32((lo + hi) / 2)
    scales = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0)),
                             np.float32(lo), np.float32([65504.0, 65519.99, 65520.0, 2.0 ** -25,
                                                          np.nextafter(np.float32(2.0 ** -25), np.float32(1))])])
    # amax near 127 * scale, plus its f32 neighbours (the division decides)
    a = np.float32(scales.astype(np.float64) * 127)
    return np.unique(np.concatenate([a, np.nextafter(a, np.float32(np.inf)), np.nextafter(a, np.float32(0))]))


def test_append_scale_rounding_boundaries(eng):
    """Every block's f16 scale and values bit-equal to KvQ8Block::quantize for
    block maxima around f16 rounding boundaries (the scale conversion is the
    hardware's round-to-nearest-even)."""
    amax = f16_boundary_amaxes()
    n_kv, hd = 4, 64
    per_row = n_kv * hd // 32
    seq = (amax.size + per_row - 1) // per_row
    rng = np.random.default_rng(12)
    X = (rng.uniform(-1, 1, (seq * per_row, 32)) * 0.999).astype(np.float32)
    a = np.resize(amax, seq * per_row)
    X *= a[:, None]
    X[np.arange(X.shape[0]), rng.integers(0, 32, X.shape[0])] = a * np.where(rng.random(X.shape[0]) < 0.5, 1, -1)
    K = X.reshape(seq, n_kv * hd)
    V = K[::-1].copy()
    cache = eng.kv_q8_cache(seq, n_kv, hd)
    append_all(eng, cache, K, V)
    for which, M in (("k", K), ("v", V)):
        got = cache.blocks(which, seq)
        want = np.stack([oracle.kv_q8_blocks(M[t], n_kv, hd) for t in range(seq)])
        assert np.array_equal(got, want), which
    cache.free()


@pytest.mark.parametrize("seq,n_head,n_kv,hd", [(1, 4, 4, 128), (7, 8, 2, 64), (100, 16, 16, 128),
                                                (1000, 16, 4, 128), (5000, 8, 1, 32), (300, 4, 4, 256),
                                                (4097, 16, 16, 128)])
@pytest.mark.parametrize("gated", [False, True])
def test_attention_parity(eng, seq, n_head, n_kv, hd, gated):
    print(f"attn seq={seq} heads={n_head}/{n_kv} hd={hd} gated={gated}", flush=True)
    rng = np.random.default_rng(seq + hd)
    K = (rng.standard_normal((seq, n_kv * hd)) * 0.5).astype(np.float32)
    V = rng.standard_normal((seq, n_kv * hd)).astype(np.float32)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    g = rng.standard_normal(n_head * hd).astype(np.float32) if gated else None
    cache = eng.kv_q8_cache(seq + 3, n_kv, hd)
    append_all(eng, cache, K, V)
    kb, vb = cache.blocks("k", seq), cache.blocks("v", seq)
    qd, od = eng.to_device(q), eng.alloc(n_head * hd * 4)
    gd = eng.to_device(g) if gated else None
    try:
        cache.attend(qd.ptr, n_head, seq, od.ptr, gd.ptr if gd else 0, eng.stream)
        eng.synchronize()
        out = od.download(np.float32, (n_head * hd,))
    finally:
        for b in (qd, od, gd):
            if b is not None:
                b.free()
    ref = oracle.attn_q8(q, kb, vb, seq, n_head, n_kv, hd, gate=g)
    vmax = np.abs(oracle.q8_dequant(vb.reshape(-1))).max()
    assert np.abs(out - ref).max() <= 1e-4 * vmax
    cache.free()


def test_attention_prefix_lengths_share_one_cache(eng):
    """Attention at every length of a growing cache (the decode loop)."""
    seq, n_head, n_kv, hd = 40, 8, 2, 64
    rng = np.random.default_rng(1)
    K = rng.standard_normal((seq, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((seq, n_kv * hd)).astype(np.float32)
    cache = eng.kv_q8_cache(seq, n_kv, hd)
    append_all(eng, cache, K, V)
    kb, vb = cache.blocks("k", seq), cache.blocks("v", seq)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    qd, od = eng.to_device(q), eng.alloc(n_head * hd * 4)
    for L in (1, 2, 17, 40):
        cache.attend(qd.ptr, n_head, L, od.ptr, 0, eng.stream)
        eng.synchronize()
        out = od.download(np.float32, (n_head * hd,))
        ref = oracle.attn_q8(q, kb[:L], vb[:L], L, n_head, n_kv, hd)
        assert np.abs(out - ref).max() <= 1e-4 * np.abs(oracle.q8_dequant(vb[:L].reshape(-1))).max(), L
    qd.free()
    od.free()
    cache.free()


def test_attention_errors(eng):
    cache = eng.kv_q8_cache(4, 2, 64)
    buf = eng.alloc(4096)
    try:
        for kw, code in [(dict(n_head=3, seq_len=1), engine.VXT_E_SHAPE),
                         (dict(n_head=2, seq_len=0), engine.VXT_E_SHAPE),
                         (dict(n_head=2, seq_len=5), engine.VXT_E_SHAPE),
                         (dict(n_head=18, seq_len=1), engine.VXT_E_UNSUPPORTED)]:
            with pytest.raises(engine.BackendError) as e:
                cache.attend(buf.ptr, out_ptr=buf.ptr + 2048, stream=eng.stream, **kw)
            assert e.value.code == code
        with pytest.raises(engine.BackendError) as e:
            cache.append(buf.ptr, buf.ptr, 4, eng.stream)
        assert e.value.code == engine.VXT_E_SHAPE
        bad = eng.kv_q8_cache(4, 2, 48)
        with pytest.raises(engine.BackendError) as e:
            bad.append(buf.ptr, buf.ptr, 0, eng.stream)
        assert e.value.code == engine.VXT_E_UNSUPPORTED
        bad.free()
    finally:
        buf.free()
        cache.free()
