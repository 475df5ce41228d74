"""GPU parity of the whole attention step over the Q8_0 KV cache:
``vxt_hip_attn_prep_q8_dev`` (gated q split, per-head q / k RMSNorm, RoPE,
K / V quantised into the cache) and ``vxt_hip_attn_step_q8_dev`` (prep, then
causal attention for a batch of tokens) against the oracle's restatement of
step_full_gqa_q8 (llm_prefill.rs:259-367, apply_rope llm_ops.rs:81-99).

Bars:
* gate halves and the V cache: bit-equal (an f32 bias add at most, then
  KvQ8Block::quantize);
* q: |dq| <= 1e-5 max|q_ref| per token (fp32: the norm's sum of squares runs
  in another order; sine and cosine are rounded once from double);
* K cache: bit-equal when there is neither norm nor rotation; otherwise every
  dequantised value within one quantisation step max(d_dev, d_ref) of the
  oracle's, and at most 2 % of the blocks (at least one) differing at all (a
  last-bit difference of a normed, rotated k can move a rounding);
* attention output: |out - ref| <= 1e-4 max|V| against the oracle's
  attention over the cache the device wrote (the K check above covers the
  cache), and against the oracle's own whole step when the caches agree.
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


class Case:
    """One layer's attention configuration, its weights on host and device."""

    def __init__(self, eng, n_head, n_kv, hd, gated=False, norms=False, neox=False, rope_dim=0, biases=False,
                 freq_base=1e6, seed=0):
        rng = np.random.default_rng(seed)
        self.rng = rng
        self.p = oracle.GqaStep(n_head, n_kv, hd, gated=gated, rope_dim=rope_dim, freq_base=freq_base, neox=neox,
                                eps=1e-6, q_norm=rng.standard_normal(hd) * 0.5 + 1 if norms else None,
                                k_norm=rng.standard_normal(hd) * 0.5 + 1 if norms else None)
        self.kvd = n_kv * hd
        self.qb = rng.standard_normal(self.p.q_rows).astype(np.float32) * 0.1 if biases else None
        self.kb_ = rng.standard_normal(self.kvd).astype(np.float32) * 0.1 if biases else None
        self.vb_ = rng.standard_normal(self.kvd).astype(np.float32) * 0.1 if biases else None
        self.bufs = []

        def dev(a):
            if a is None:
                return 0
            b = eng.to_device(np.ascontiguousarray(a, dtype=np.float32))
            self.bufs.append(b)
            return b.ptr

        self.params = engine.GqaParams(dev(self.p.q_norm), dev(self.p.k_norm), dev(self.qb), dev(self.kb_),
                                       dev(self.vb_), n_head, int(gated), rope_dim, int(neox), freq_base, 1e-6)
        self.exact_k = not norms and min(rope_dim, hd) < 2

    def tokens(self, m, scale=2.0):
        q = (self.rng.standard_normal((m, self.p.q_rows)) * scale).astype(np.float32)
        k = (self.rng.standard_normal((m, self.kvd)) * scale).astype(np.float32)
        v = self.rng.standard_normal((m, self.kvd)).astype(np.float32)
        return q, k, v

    def host_inputs(self, q, k, v):
        """The caller's bias adds (llm_prefill.rs:497-505), in f32."""
        return (q + self.qb if self.qb is not None else q, k + self.kb_ if self.kb_ is not None else k,
                v + self.vb_ if self.vb_ is not None else v)

    def free(self):
        for b in self.bufs:
            b.free()


def empty_blocks(rows, kvd):
    return np.zeros((rows * kvd // 32, 34), np.uint8)


def check_k_cache(got, want, exact):
    got, want = got.reshape(-1, 34), want.reshape(-1, 34)
    if exact:
        assert np.array_equal(got, want)
        return
    step = np.maximum(oracle.f16_to_f32(got[:, :2].copy().view(np.uint16).reshape(-1)),
                      oracle.f16_to_f32(want[:, :2].copy().view(np.uint16).reshape(-1)))
    dk = oracle.q8_dequant(got).reshape(-1, 32)
    rk = oracle.q8_dequant(want).reshape(-1, 32)
    assert np.all(np.abs(dk - rk) <= step[:, None] * (1 + 2.0 ** -20))
    differing = np.any(got != want, axis=1).sum()
    assert differing <= max(1, int(0.02 * got.shape[0])), differing


def run_prep(eng, case, q, k, v, pos, rope_pos, cache):
    m = q.shape[0]
    n_head, hd = case.p.n_head, case.p.hd
    qd, kd, vd = eng.to_device(q), eng.to_device(k), eng.to_device(v)
    qo = eng.alloc(m * n_head * hd * 4)
    go = eng.alloc(m * n_head * hd * 4)
    try:
        cache.prep(case.params, qd.ptr, kd.ptr, vd.ptr, pos, rope_pos, qo.ptr, go.ptr, batch_m=m,
                   q_stride=case.p.q_rows, kv_stride=case.kvd, stream=eng.stream)
        eng.synchronize()
        return qo.download(np.float32, (m, n_head * hd)), go.download(np.float32, (m, n_head * hd))
    finally:
        for b in (qd, kd, vd, qo, go):
            b.free()


PREP_CASES = [
    # n_head, n_kv, hd, gated, norms, neox, rope_dim, biases, batch, pos, rope_pos
    (4, 4, 32, False, False, False, 0, False, 1, 0, 0),
    (8, 2, 64, True, True, True, 64, False, 3, 5, 5),
    (16, 4, 128, True, True, True, 32, True, 5, 100, 30000),
    (8, 8, 128, False, True, False, 128, False, 2, 7, 4095),
    (4, 1, 256, True, False, False, 64, True, 4, 0, 123456),
    (6, 2, 64, False, False, True, 64, True, 1, 9, 9),
    (2, 2, 32, True, True, False, 7, False, 3, 1, 40),
]


@pytest.mark.parametrize("case_args", PREP_CASES)
def test_prep_parity(eng, case_args):
    n_head, n_kv, hd, gated, norms, neox, rope_dim, biases, m, pos, rope_pos = case_args
    print(f"prep {case_args}", flush=True)
    case = Case(eng, n_head, n_kv, hd, gated, norms, neox, rope_dim, biases, seed=hd + m + pos)
    cache = eng.kv_q8_cache(pos + m + 2, n_kv, hd)
    try:
        q, k, v = case.tokens(m)
        q_dev, g_dev = run_prep(eng, case, q, k, v, pos, rope_pos, cache)
        qh_in, kh_in, vh_in = case.host_inputs(q, k, v)
        kb, vb = empty_blocks(pos + m, case.kvd), empty_blocks(pos + m, case.kvd)
        for t in range(m):
            q_ref, g_ref, _ = case.p.prep(qh_in[t], kh_in[t], vh_in[t], kb, vb, pos + t, rope_pos + t)
            assert np.abs(q_dev[t] - q_ref).max() <= 1e-5 * np.abs(q_ref).max(), t
            if gated:
                assert np.array_equal(g_dev[t].view(np.uint32), g_ref.view(np.uint32))
        rows = slice(pos * case.kvd // 32, (pos + m) * case.kvd // 32)
        assert np.array_equal(cache.blocks("v", pos + m).reshape(-1, 34)[rows], vb[rows])
        check_k_cache(cache.blocks("k", pos + m).reshape(-1, 34)[rows], kb[rows], case.exact_k)
    finally:
        cache.free()
        case.free()


def oracle_q(case, q_in, rope_pos):
    """The oracle's prepared q and gate of one token (cache row is scratch)."""
    kb, vb = empty_blocks(1, case.kvd), empty_blocks(1, case.kvd)
    qh, qg, _ = case.p.prep(q_in, np.zeros(case.kvd, np.float32), np.zeros(case.kvd, np.float32), kb, vb, 0,
                            rope_pos)
    return qh, qg


def run_step(eng, case, cache, q, k, v, pos, rope_pos):
    m = q.shape[0]
    qd, kd, vd = eng.to_device(q), eng.to_device(k), eng.to_device(v)
    od = eng.alloc(m * case.p.n_head * case.p.hd * 4)
    try:
        cache.step(case.params, qd.ptr, kd.ptr, vd.ptr, pos, rope_pos, od.ptr, batch_m=m, q_stride=case.p.q_rows,
                   kv_stride=case.kvd, stream=eng.stream)
        eng.synchronize()
        return od.download(np.float32, (m, case.p.n_head * case.p.hd))
    finally:
        for b in (qd, kd, vd, od):
            b.free()


@pytest.mark.parametrize("n_head,n_kv,hd,gated,norms,neox,rope_dim,biases", [
    (8, 2, 128, True, True, True, 64, True),
    (16, 16, 64, False, False, False, 0, False),
    (4, 1, 32, True, True, False, 32, False),
    (8, 1, 256, False, True, True, 256, True),
])
def test_decode_steps_match_oracle(eng, n_head, n_kv, hd, gated, norms, neox, rope_dim, biases):
    """A decode loop of single-token steps (llm_cpu.rs:395-412), rope
    positions offset from cache positions."""
    S, delta = 24, 3
    print(f"decode steps heads={n_head}/{n_kv} hd={hd} gated={gated}", flush=True)
    case = Case(eng, n_head, n_kv, hd, gated, norms, neox, rope_dim, biases, seed=n_head * hd)
    cache = eng.kv_q8_cache(S, n_kv, hd)
    kb, vb = empty_blocks(S, case.kvd), empty_blocks(S, case.kvd)
    try:
        for pos in range(S):
            q, k, v = case.tokens(1)
            out = run_step(eng, case, cache, q, k, v, pos, pos + delta)[0]
            qi, ki, vi = case.host_inputs(q, k, v)
            ref_own = case.p.step(qi[0], ki[0], vi[0], kb, vb, pos, pos + delta)
            kb_dev, vb_dev = cache.blocks("k", pos + 1), cache.blocks("v", pos + 1)
            qh, qg = oracle_q(case, qi[0], pos + delta)
            ref = oracle.attn_q8(qh, kb_dev, vb_dev, pos + 1, n_head, n_kv, hd, gate=qg)
            vmax = np.abs(oracle.q8_dequant(vb_dev.reshape(-1))).max()
            assert np.abs(out - ref).max() <= 1e-4 * vmax, pos
            if np.array_equal(kb_dev.reshape(-1, 34), kb[:(pos + 1) * case.kvd // 32]):
                assert np.abs(out - ref_own).max() <= 1e-4 * vmax, pos
        assert np.array_equal(cache.blocks("v", S).reshape(-1, 34), vb)
        check_k_cache(cache.blocks("k", S), kb, case.exact_k)
    finally:
        cache.free()
        case.free()


@pytest.mark.parametrize("pos0,m,n_head,n_kv,hd", [
    (0, 37, 8, 2, 64), (5, 64, 16, 4, 128), (3000, 150, 16, 2, 128),   # MFMA prefill
    (0, 100, 6, 2, 64), (17, 40, 8, 1, 32), (0, 300, 16, 16, 128), (33, 16, 4, 4, 128),
    (2, 7, 8, 2, 64), (10, 20, 4, 1, 256), (3000, 15, 16, 2, 128)])    # per-token kernels
def test_batched_step_is_causal(eng, pos0, m, n_head, n_kv, hd):
    """A batch of tokens in one call (the prefill loop of llm_prefill.rs:
    505-517): token t attends to rows [0, pos0 + t] only.  Batches of 16 or
    more tokens with head_dim <= 128 take the MFMA prefill kernel (query
    blocks of 128 / group tokens: groups 1, 2, 3, 4, 8 here); smaller ones and
    head_dim 256 the per-token kernels, the last case split into several
    launch groups (partial sums bounded per launch)."""
    print(f"batched step pos0={pos0} m={m} heads={n_head}/{n_kv} hd={hd}", flush=True)
    case = Case(eng, n_head, n_kv, hd, gated=True, norms=True, neox=True, rope_dim=hd // 2, biases=True,
                seed=pos0 + m)
    cache = eng.kv_q8_cache(pos0 + m, n_kv, hd)
    try:
        if pos0:
            q, k, v = case.tokens(pos0)
            run_step(eng, case, cache, q, k, v, 0, 0)
        q, k, v = case.tokens(m)
        out = run_step(eng, case, cache, q, k, v, pos0, pos0)
        qi, _, _ = case.host_inputs(q, k, v)
        kb_dev, vb_dev = cache.blocks("k", pos0 + m), cache.blocks("v", pos0 + m)
        rows = case.kvd // 32
        sample = sorted(set([0, 1, m // 2, m - 2, m - 1] + list(range(min(m, 130) - 3, min(m, 130)))))
        for t in sample:
            L = pos0 + t + 1
            qh, qg = oracle_q(case, qi[t], pos0 + t)
            ref = oracle.attn_q8(qh, kb_dev[:L], vb_dev[:L], L, n_head, n_kv, hd, gate=qg)
            vmax = np.abs(oracle.q8_dequant(vb_dev[:L].reshape(-1))).max()
            assert np.abs(out[t] - ref).max() <= 1e-4 * vmax, t
        # the batch's cache rows against the oracle's sequential prep
        kb, vb = empty_blocks(pos0 + m, case.kvd), empty_blocks(pos0 + m, case.kvd)
        _, ki, vi = case.host_inputs(q, k, v)
        for t in range(m):
            case.p.prep(qi[t], ki[t], vi[t], kb, vb, pos0 + t, pos0 + t)
        assert np.array_equal(vb_dev.reshape(-1, 34)[pos0 * rows:], vb[pos0 * rows:])
        check_k_cache(kb_dev.reshape(-1, 34)[pos0 * rows:], kb[pos0 * rows:], False)
    finally:
        cache.free()
        case.free()


def test_step_graph_replays_match_eager(eng):
    """A decode step recorded into a graph (workspace sized by an eager call
    first); each replay, with eager steps in between, gives the eager bits."""
    n_head, n_kv, hd, pos = 8, 2, 128, 40
    case = Case(eng, n_head, n_kv, hd, gated=True, norms=True, neox=True, rope_dim=128, seed=9)
    cache = eng.kv_q8_cache(pos + 1, n_kv, hd)
    q0, k0, v0 = case.tokens(pos)
    run_step(eng, case, cache, q0, k0, v0, 0, 0)
    q, k, v = case.tokens(1)
    qd, kd, vd = eng.to_device(q), eng.to_device(k), eng.to_device(v)
    od = eng.alloc(n_head * hd * 4)
    try:
        cache.step(case.params, qd.ptr, kd.ptr, vd.ptr, pos, pos, od.ptr, stream=eng.stream)
        eng.synchronize()
        want = od.download(np.float32, (n_head * hd,))
        g = eng.capture(lambda s: cache.step(case.params, qd.ptr, kd.ptr, vd.ptr, pos, pos, od.ptr, stream=s))
        try:
            for r in range(3):
                od.upload(np.zeros(n_head * hd, np.float32))
                g.launch(1)
                got = od.download(np.float32, (n_head * hd,))
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), r
                cache.step(case.params, qd.ptr, kd.ptr, vd.ptr, pos, pos, od.ptr, stream=eng.stream)
                eng.synchronize()
        finally:
            g.free()
    finally:
        for b in (qd, kd, vd, od):
            b.free()
        cache.free()
        case.free()


def test_step_errors(eng):
    cache = eng.kv_q8_cache(4, 2, 64)
    buf = eng.alloc(1 << 16)
    try:
        def params(**kw):
            d = dict(q_norm=0, k_norm=0, q_bias=0, k_bias=0, v_bias=0, n_head=4, gated_q=0, rope_dim=64,
                     rope_neox=0, rope_freq_base=10000.0, eps=1e-6)
            d.update(kw)
            return engine.GqaParams(**d)

        p = buf.ptr
        for fn, kw, code in [
            ("step", dict(params=params(n_head=3)), engine.VXT_E_SHAPE),
            ("step", dict(params=params(n_head=18)), engine.VXT_E_UNSUPPORTED),
            ("step", dict(params=params(), pos=4), engine.VXT_E_SHAPE),
            ("step", dict(params=params(), pos=2, batch_m=3, q_stride=256, kv_stride=128), engine.VXT_E_SHAPE),
            ("step", dict(params=params(), pos=0, batch_m=2, q_stride=100, kv_stride=128), engine.VXT_E_SHAPE),
            ("step", dict(params=params(gated_q=2)), engine.VXT_E_ARG),
            ("prep", dict(params=params(gated_q=1)), engine.VXT_E_ARG),          # gated without gate_out
            ("prep", dict(params=params(n_head=0)), engine.VXT_E_SHAPE),
        ]:
            args = dict(q_raw=p, k_cur=p + 8192, v_cur=p + 16384, pos=kw.pop("pos", 0), rope_pos=0)
            args.update(kw)
            with pytest.raises(engine.BackendError) as e:
                if fn == "step":
                    cache.step(out=p + 32768, stream=eng.stream, **args)
                else:
                    cache.prep(q_out=p + 32768, stream=eng.stream, **args)
            assert e.value.code == code, (fn, kw)
    finally:
        buf.free()
        cache.free()
