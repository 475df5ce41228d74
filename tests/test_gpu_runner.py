"""GPU parity of the decode-step runner (``vxt_hip_runner_*``): a whole
decoder forward -- embedding, per layer RMSNorm, [q|gate; k; v] projection,
step_full_gqa_q8 over the layer's Q8_0 KV cache, output projection, residual
add + RMSNorm, gated FFN, down projection -- then the final norm, the head and
the greedy id (llm_cpu.rs:395-482; the reference's device runner
metal_cb4_fast_run.mm:94-434 behind metal_cb4_fast_ffi.rs:134-206).

Bars:
* against the eager composition of the entry points it is built from (the
  same kernels in the same order -- a single token with each layer's norms
  inside the projections that read them --, attention at host positions,
  separate KV caches): last-token logits bit-equal after a batched prefill
  and after every single-token step, and ``generate`` ids equal to the eager
  greedy loop -- the captured step with the position in device memory
  computes what the entry points compute;
* against the oracle's whole forward (oracle.embed_rows, rms_norm, gemv per
  weight kind, GqaStep.step, glu, the projections' inputs rounded to bf16 as
  the device stores them): |logits - ref| <= 5e-3 max|ref| per step (fp32 sums
  in other orders; a last-bit difference of k can move one K quantisation
  step), and the greedy id equal wherever the reference's top two logits are
  further apart than that bar.
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine, synth
from vxg_amd.formats import bf16_bits_to_f32, f32_to_bf16_bits

pytestmark = pytest.mark.gpu

H, NH, NKV, HD, FFN, VOCAB = 256, 4, 2, 64, 512, 1000
MAX_SEQ, MAX_BATCH, EPS, ROPE_BASE = 64, 16, 1e-6, 10000.0


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


def bf16r(x):
    """f32 -> nearest bf16 -> f32 (how the device stores projection inputs)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.ascontiguousarray(x, dtype=np.float32)))


def make_weight(kind, rows, cols, seed):
    if kind == "g64":
        return synth.make_g64(rows, cols, seed=seed)
    if kind == "cb4":
        return synth.make_cb4(rows, cols, seed=seed, centred=True)
    return synth.make_q8(rows, cols, seed=seed)


class Model:
    """Host weights, their device copies and the runner's arguments."""

    def __init__(self, eng, kinds, gated, rope_dim, neox, norms, act, seed=0):
        rng = np.random.default_rng(seed)
        self.kinds, self.gated, self.act = kinds, gated, act
        self.q_rows = NH * HD * (2 if gated else 1)
        self.kvd = NKV * HD
        self.bufs, self.tensors = [], []

        def dev(a):
            b = eng.to_device(np.ascontiguousarray(a, dtype=np.float32))
            self.bufs.append(b)
            return b

        def up(m):
            t = eng.upload_packed(m)
            self.tensors.append(t)
            return t

        self.layers, self.host = [], []
        for i, kind in enumerate(kinds):
            s = seed * 100 + i * 10
            w = {"in": make_weight(kind, self.q_rows + 2 * self.kvd, H, s + 1),
                 "out": make_weight(kind, H, NH * HD, s + 2),
                 "gu": make_weight(kind, 2 * FFN, H, s + 3),
                 "dn": make_weight(kind, H, FFN, s + 4),
                 "an": (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32),
                 "pn": (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32),
                 "qn": (1.0 + 0.1 * rng.standard_normal(HD)).astype(np.float32) if norms else None,
                 "kn": (1.0 + 0.1 * rng.standard_normal(HD)).astype(np.float32) if norms else None}
            self.host.append(w)
            qn = dev(w["qn"]).ptr if norms else 0
            kn = dev(w["kn"]).ptr if norms else 0
            self.layers.append(engine.RunnerLayer(up(w["in"]).handle, up(w["out"]).handle, up(w["gu"]).handle,
                                                  up(w["dn"]).handle, dev(w["an"]).ptr, dev(w["pn"]).ptr, qn, kn))
        self.out_norm = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        self.out_norm_dev = dev(self.out_norm)
        self.embed_m = synth.make_q8(VOCAB, H, seed=seed * 100 + 91)
        self.head_m = synth.make_q8(VOCAB, H, seed=seed * 100 + 92)
        self.embed, self.head = up(self.embed_m), up(self.head_m)
        self.cfg = engine.RunnerConfig(len(kinds), H, NH, NKV, HD, FFN, VOCAB, int(gated), rope_dim, int(neox), act,
                                       MAX_SEQ, MAX_BATCH, ROPE_BASE, EPS, 1.0)
        self.gqa = oracle.GqaStep(NH, NKV, HD, gated=gated, q_norm=None, k_norm=None, rope_dim=rope_dim,
                                  freq_base=ROPE_BASE, neox=neox, eps=EPS)
        self.params = []
        for i, w in enumerate(self.host):
            p = engine.GqaParams(self.layers[i].q_norm or 0, self.layers[i].k_norm or 0, 0, 0, 0, NH, int(gated),
                                 rope_dim, int(neox), ROPE_BASE, EPS)
            self.params.append(p)

    def runner(self, eng):
        return eng.runner(self.cfg, self.layers, self.out_norm_dev.ptr, self.head, self.embed)

    def free(self):
        for t in self.tensors:
            t.free()
        for b in self.bufs:
            b.free()


class Eager:
    """The runner's sequence through the per-op entry points (host positions)."""

    def __init__(self, eng, model):
        self.eng, self.m = eng, model
        B = MAX_BATCH
        self.caches = [eng.kv_q8_cache(MAX_SEQ, NKV, HD) for _ in model.kinds]
        self.cur, self.delta = eng.alloc(B * H * 4), eng.alloc(B * H * 4)
        self.cur2 = eng.alloc(H * 4)
        self.normed = eng.alloc(B * H * 2)
        self.qkv_rows = model.q_rows + 2 * model.kvd
        self.qkv = eng.alloc(B * self.qkv_rows * 4)
        self.attn = eng.alloc(B * NH * HD * 4)
        self.act = eng.alloc(B * FFN * 2)
        self.logits = eng.alloc(VOCAB * 4)
        self.tok = eng.alloc(B * 4)
        self.g = eng.alloc(8)

    def forward(self, tokens, pos):
        if len(tokens) == 1:
            return self.forward_one(tokens[0], pos)
        e, m, s = self.eng, self.m, self.eng.stream
        bf, f32 = engine.DTYPE_BF16, engine.DTYPE_F32
        n = len(tokens)
        self.tok.upload(np.asarray(tokens, np.uint32))
        e.embed_dev(m.embed, self.tok.ptr, n, self.cur.ptr, H, 1.0, s)
        for i, L in enumerate(m.layers):
            e.rms_norm_dev(self.cur.ptr, self.delta.ptr if i else 0, L.attn_norm, self.normed.ptr, bf, H, H, n,
                           EPS, s)
            e.matmul_dev(m.tensors_by_handle[L.w_in], self.normed.ptr, bf, n, self.qkv.ptr, f32, s)
            k = self.qkv.ptr + m.q_rows * 4
            v = self.qkv.ptr + (m.q_rows + m.kvd) * 4
            self.caches[i].step(m.params[i], self.qkv.ptr, k, v, pos, pos, self.attn.ptr, batch_m=n,
                                q_stride=self.qkv_rows, kv_stride=self.qkv_rows, stream=s)
            e.matmul_dev(m.tensors_by_handle[L.w_out], self.attn.ptr, f32, n, self.delta.ptr, f32, s)
            e.rms_norm_dev(self.cur.ptr, self.delta.ptr, L.post_attn_norm, self.normed.ptr, bf, H, H, n, EPS, s)
            e.ffn_glu_dev(m.tensors_by_handle[L.w_ffn_gu], self.normed.ptr, bf, n, self.act.ptr, bf, FFN,
                          m.act, s)
            e.matmul_dev(m.tensors_by_handle[L.w_ffn_dn], self.act.ptr, bf, n, self.delta.ptr, f32, s)
        last = (n - 1) * H
        e.rms_norm_dev(self.cur.ptr + last * 4, self.delta.ptr + last * 4, m.out_norm_dev.ptr,
                       self.normed.ptr + last * 2, bf, H, H, 1, EPS, s)
        e.matmul_dev(m.head, self.normed.ptr + last * 2, bf, 1, self.logits.ptr, f32, s)
        e.synchronize()
        return self.logits.download(np.float32, (VOCAB,))

    def forward_one(self, token, pos):
        """One token: the two norms of a layer inside the projections that
        read them (vxt_hip_norm_matmul_dev), the residual stream alternating
        between two buffers."""
        e, m, s = self.eng, self.m, self.eng.stream
        bf, f32 = engine.DTYPE_BF16, engine.DTYPE_F32
        self.tok.upload(np.asarray([token], np.uint32))
        e.embed_dev(m.embed, self.tok.ptr, 1, self.cur.ptr, H, 1.0, s)
        res, c = (self.cur.ptr, self.cur2.ptr), 0
        glu = engine.NORM_GLU_GELU_TANH if m.act == engine.ACT_GELU_TANH else engine.NORM_GLU_SILU
        for i, L in enumerate(m.layers):
            e.norm_matmul_dev(m.tensors_by_handle[L.w_in], res[c], self.delta.ptr if i else 0, L.attn_norm, EPS,
                              res[1 - c] if i else 0, engine.NORM_PLAIN, self.qkv.ptr, f32, self.qkv_rows, s)
            if i:
                c = 1 - c
            k = self.qkv.ptr + m.q_rows * 4
            v = self.qkv.ptr + (m.q_rows + m.kvd) * 4
            self.caches[i].step(m.params[i], self.qkv.ptr, k, v, pos, pos, self.attn.ptr, batch_m=1,
                                q_stride=self.qkv_rows, kv_stride=self.qkv_rows, stream=s)
            e.matmul_dev(m.tensors_by_handle[L.w_out], self.attn.ptr, f32, 1, self.delta.ptr, f32, s)
            e.norm_matmul_dev(m.tensors_by_handle[L.w_ffn_gu], res[c], self.delta.ptr, L.post_attn_norm, EPS,
                              res[1 - c], glu, self.act.ptr, bf, FFN, s)
            c = 1 - c
            e.matmul_dev(m.tensors_by_handle[L.w_ffn_dn], self.act.ptr, bf, 1, self.delta.ptr, f32, s)
        e.rms_norm_dev(res[c], self.delta.ptr, m.out_norm_dev.ptr, self.normed.ptr, bf, H, H, 1, EPS, s)
        e.matmul_dev(m.head, self.normed.ptr, bf, 1, self.logits.ptr, f32, s)
        e.synchronize()
        return self.logits.download(np.float32, (VOCAB,))

    def greedy(self):
        self.eng.greedy_dev(self.logits.ptr, VOCAB, self.g.ptr, self.eng.stream)
        self.eng.synchronize()
        r = self.g.download(np.uint32, (2,))
        return int(r[0]), int(r[1])

    def free(self):
        for c in self.caches:
            c.free()
        for b in (self.cur, self.cur2, self.delta, self.normed, self.qkv, self.attn, self.act, self.logits, self.tok,
                  self.g):
            b.free()


class OracleModel:
    """The whole forward on the CPU oracle, one token at a time."""

    def __init__(self, model):
        self.m = model
        per = MAX_SEQ * model.kvd // 32 * 34
        self.kb = [np.zeros(per, np.uint8) for _ in model.kinds]
        self.vb = [np.zeros(per, np.uint8) for _ in model.kinds]
        self.gqa = []
        for w in model.host:
            self.gqa.append(oracle.GqaStep(NH, NKV, HD, gated=model.gated, q_norm=w["qn"], k_norm=w["kn"],
                                           rope_dim=model.gqa.rope_dim, freq_base=ROPE_BASE, neox=model.gqa.neox,
                                           eps=EPS))

    def token(self, tok, pos):
        m = self.m
        cur = oracle.embed_rows(m.embed_m, [tok])[0].astype(np.float32)
        for i, w in enumerate(m.host):
            normed = bf16r(oracle.rms_norm(cur, w["an"], EPS))
            qkv = oracle.gemv(w["in"], normed)
            q_raw, k, v = qkv[:m.q_rows], qkv[m.q_rows:m.q_rows + m.kvd], qkv[m.q_rows + m.kvd:]
            attn = self.gqa[i].step(q_raw, k, v, self.kb[i], self.vb[i], pos, pos)
            cur = (cur + oracle.gemv(w["out"], attn)).astype(np.float32)
            normed = bf16r(oracle.rms_norm(cur, w["pn"], EPS))
            gu = oracle.gemv(w["gu"], normed)
            act = bf16r(oracle.glu(gu[:FFN], gu[FFN:], gelu=m.act == engine.ACT_GELU_TANH))
            cur = (cur + oracle.gemv(w["dn"], act)).astype(np.float32)
        normed = bf16r(oracle.rms_norm(cur, m.out_norm, EPS))
        return oracle.gemv(m.head_m, normed)


CASES = [
    dict(kinds=("g64", "cb4", "q8"), gated=True, rope_dim=64, neox=True, norms=True, act=engine.ACT_SILU),
    dict(kinds=("q8", "g64"), gated=False, rope_dim=32, neox=False, norms=False, act=engine.ACT_GELU_TANH),
]


def _model(eng, case, seed):
    m = Model(eng, seed=seed, **case)
    m.tensors_by_handle = {t.handle: t for t in m.tensors}
    return m


@pytest.mark.parametrize("ci", range(len(CASES)))
def test_runner_matches_entry_points(eng, ci):
    m = _model(eng, CASES[ci], seed=ci + 1)
    r = m.runner(eng)
    ref = Eager(eng, m)
    try:
        prompt = [5, 917, 42, 300, 7]
        a = r.step(prompt, 0)
        b = ref.forward(prompt, 0)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "prefill logits"
        pos = len(prompt)
        tok, _ = ref.greedy()
        for step in range(4):
            a = r.step([tok], pos)
            b = ref.forward([tok], pos)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {step}"
            tok, _ = ref.greedy()
            pos += 1
        # generation: the runner's device loop against the eager greedy loop
        ids, flags = r.generate(tok, pos, 6)
        want = []
        t = tok
        for i in range(6):
            ref.forward([t], pos + i)
            t, _ = ref.greedy()
            want.append(t)
        assert ids.tolist() == want
        assert not flags.any()
        # a replay of the same position range reproduces the same ids
        ids2, _ = r.generate(tok, pos, 6)
        assert ids2.tolist() == want
    finally:
        r.free()
        ref.free()
        m.free()


@pytest.mark.parametrize("ci", range(len(CASES)))
def test_runner_matches_oracle(eng, ci):
    m = _model(eng, CASES[ci], seed=ci + 11)
    r = m.runner(eng)
    ref = OracleModel(m)
    try:
        prompt = [3, 999, 250, 31, 640, 12]
        got = r.step(prompt, 0)
        for p, t in enumerate(prompt):
            want = ref.token(t, p)
        bar = 5e-3 * float(np.abs(want).max())
        assert float(np.abs(got - want).max()) <= bar, "prefill"
        pos = len(prompt)
        tok = int(np.argmax(want))
        for step in range(3):
            got = r.step([tok], pos)
            want = ref.token(tok, pos)
            bar = 5e-3 * float(np.abs(want).max())
            assert float(np.abs(got - want).max()) <= bar, f"step {step}"
            top2 = np.sort(want)[-2:]
            if top2[1] - top2[0] > 2 * bar:
                assert int(np.argmax(got)) == int(np.argmax(want))
            tok = int(np.argmax(want))
            pos += 1
    finally:
        r.free()
        m.free()


def test_runner_errors(eng):
    m = _model(eng, CASES[1], seed=21)
    r = m.runner(eng)
    try:
        with pytest.raises(engine.BackendError):
            r.step([VOCAB], 0)                          # id past the vocabulary
        with pytest.raises(engine.BackendError):
            r.step([1] * (MAX_BATCH + 1), 0)            # more than max_batch
        with pytest.raises(engine.BackendError):
            r.step([1, 2], MAX_SEQ - 1)                 # past the cache
        with pytest.raises(engine.BackendError):
            r.generate(1, MAX_SEQ - 3, 4)               # past the cache
        ids, _ = r.generate(1, MAX_SEQ - 3, 3)          # up to the last row is fine
        assert ids.shape == (3,)
        bad = engine.RunnerConfig(m.cfg.n_layers, H + 8, NH, NKV, HD, FFN, VOCAB, m.cfg.gated_q, 0, 0, 0,
                                  MAX_SEQ, MAX_BATCH, ROPE_BASE, EPS, 1.0)
        with pytest.raises(engine.BackendError):
            eng.runner(bad, m.layers, m.out_norm_dev.ptr, m.head, m.embed)   # shapes do not chain
    finally:
        r.free()
        m.free()


def test_runner_released_with_its_engine():
    e = engine.HipEngine()
    m = _model(e, CASES[1], seed=31)
    r = m.runner(e)
    ids, _ = r.generate(7, 0, 2)
    assert ids.shape == (2,)
    e.close()        # releases the runner, its graph and its caches
    r.free()         # a no-op now
    m.free()
