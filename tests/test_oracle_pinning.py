"""Pin the CPU oracle (oracle/vxt_oracle.c) before trusting it.

Each oracle function is checked against something other than its own formula:

==========================  ====================================================
oracle function             pinned by
==========================  ====================================================
f16_to_f32 (fp16.rs:6)      all 65,536 patterns vs numpy's IEEE float16 widening
f32_to_f16 (fp16.rs:33)     the reference's golden table (fp16.rs:89-108) +
                            2^20 random f32 patterns vs numpy's RNE cast + NaN
                            payload rule
bf16_to_f32 (fp16.rs:81)    all 65,536 patterns vs torch.bfloat16 widening
f32_to_bf16 (fp16.rs:113)   2^20 random f32 patterns vs torch's RNE cast + NaN
cb4 decode_row              closed-form fixture of metal_llm_tests.rs:31-58 and
(codebook.rs:285)           the duplicate-column CSR of llm_gpu_cpu_parity.rs:
                            680-688 (expected values from an independent numpy
                            decoder, tests/golden/make_golden.py), plus hand-
                            derived values
cb4 gemv (codebook.rs:350)  fp64 brute force with a K*u*sum|wx| bound at the
                            reference's tail shapes; 1- vs 4-thread bit identity
                            (tensor_roundtrip_gemv.rs:176); a cancellation case
                            whose answer is fixed by the 4-accumulator
                            interleave; the sc == 0 group skip
g64 decode / gemv           numpy float16 gather; fp64 bound; thread identity
Q8 dequant (gguf.rs:223)    numpy int8 * float16 product (exact in f32)
Q8 dot_f32 (llm_prefill:45) a cancellation case fixed by the two-chain split;
                            fp64 bound
Q8 quantize (llm_prefill:28) amax -> +-127, ties-to-even, |err| <= d/2, zeros
Q8 gemv                     block-dot composition in block order; fp64 bound
gemm (llm_prefill.rs:156)   vs per-token GEMV, cosine > 0.999999 at rows=96,
                            cols=256, M=11 (vxt_roadmap_steps.rs:210-230); fp64
                            bound; 1- vs 4-worker bit identity; equals the dense
                            FMA chain of decoded rows
embed_rows (llm_cpu.rs:223)  decode_rows at scale 1 and at 1 - 2^-24 (under the
                            1e-7 threshold); an exact doubling at scale 2; the
                            f64 product rounded once to f32 at sqrt(2048)
silu / gelu_tanh / glu     f64 formulas (tanh from numpy) within 4 ulp over
(llm_ops.rs:39,             [-90, 90]; the limits silu(+-large), gelu(+-large);
llm_prefill.rs:66)          signs; act(g) * u equals the product of the parts
rms_norm (llm_ops.rs:48)    f64 computation within 1e-6; constant rows (closed
                            form c / sqrt(c^2 + eps)); zero row; weight scaling
attn_q8 (llm_prefill.rs:   one position: exactly the dequantised V block; f64
317-367)                    softmax attention over the dequantised cache within
                            1e-5 max|V|; GQA head-to-KV mapping; q = 0 gives the
                            mean of V; the gate is the sigmoid factor
greedy (llm_ops.rs:318,     the six tie / NaN / inf cases of metal_llm_tests.rs:
vxt_llm_ops.metal:569)      95-117 with hand-derived answers; every array of
                            length <= 4 over {-inf,-1,-0,+0,denormal,1,inf,NaN}
                            and random arrays vs a numpy set formula (first index
                            of numpy.nanmax, 0 when that is -inf or all NaN)
==========================  ====================================================

The macOS ``cblas_sgemm`` branch of dense_tile_gemm (llm_prefill.rs:117-138)
is not restated (parity unpinned, and off the non-mac reference path).
"""
import json
import os

import numpy as np
import pytest

import oracle
from parity_util import GREEDY_REFERENCE_CASES, greedy_reference_logits
from vxg_amd import synth
from vxg_amd.formats import CodebookMatrix, Cb4G64Matrix, f32_to_f16_bits

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def f32_of_bits(b):
    return np.array(b, dtype=np.uint32).view(np.float32)


# ---------------------------------------------------------------- conversions

def test_f16_to_f32_exhaustive_vs_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))
    # reference NaN rule: sign | 0x7f80_0000 | mant << 13 (payload kept)
    b = bits[nan].astype(np.uint32)
    exp = ((b & 0x8000) << 16) | 0x7F800000 | ((b & 0x3FF) << 13)
    assert np.array_equal(got[nan].view(np.uint32), exp)


def test_f32_to_f16_reference_golden_table():
    with open(os.path.join(GOLD, "f16_boundaries.json")) as f:
        cases = json.load(f)["cases"]
    assert len(cases) == 20
    for c in cases:
        v = f32_of_bits([c["f32_bits"]])
        assert int(oracle.f32_to_f16(v)[0]) == c["f16_bits"], c


def test_f32_to_f16_random_patterns_vs_numpy():
    g = np.random.default_rng(5)
    bits = g.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    # concentrate half the sample on the f16 range (|x| < 2^17)
    bits[: 1 << 19] = (bits[: 1 << 19] & 0x80FFFFFF) | (g.integers(0x60, 0x90, size=1 << 19).astype(np.uint32) << 23)
    v = bits.view(np.float32)
    fin = np.isfinite(v)
    got = oracle.f32_to_f16(v[fin])
    with np.errstate(over="ignore"):
        ref = v[fin].astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    # NaN rule: sign | 0x7e00 | mant >> 13 ; inf stays inf
    nanb = np.array([0x7FC00001, 0xFF800001, 0x7F812345], dtype=np.uint32)
    exp = ((nanb >> 16) & 0x8000) | 0x7E00 | ((nanb & 0x7FFFFF) >> 13)
    assert np.array_equal(oracle.f32_to_f16(nanb.view(np.float32)), exp.astype(np.uint16))
    assert list(oracle.f32_to_f16(np.array([np.inf, -np.inf], np.float32))) == [0x7C00, 0xFC00]


def test_bf16_conversions_vs_torch():
    torch = pytest.importorskip("torch")
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.bf16_to_f32(bits)
    ref = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.array_equal(got.view(np.uint32), bits.astype(np.uint32) << 16)

    g = np.random.default_rng(6)
    rb = g.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    v = rb.view(np.float32)
    fin = np.isfinite(v)
    got = oracle.f32_to_bf16(v[fin])
    ref = torch.from_numpy(v[fin].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    nanb = np.array([0x7F800001, 0xFFC00000, 0x7F8F0000], dtype=np.uint32)
    exp = ((nanb >> 16) | 0x0040).astype(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(nanb.view(np.float32)), exp)


# ---------------------------------------------------------------- cb4 decode

def closed_form(rows, cols, row_ptr, packed, pad=128):
    padded = (cols + pad - 1) // pad * pad
    groups = padded // 128
    cent = ((np.arange(16, dtype=np.float32) - np.float32(7.5)) * np.float32(0.1234567)).astype(np.float32)
    scales = f32_to_f16_bits(np.float32(0.125) + (np.arange(rows * groups) % 11).astype(np.float32) * np.float32(0.25))
    rot = np.array([((0x76543210 << s) | (0x76543210 >> (32 - s))) & 0xFFFFFFFF if s else 0x76543210
                    for s in range(0, 32, 4)], dtype=np.uint64).astype(np.uint32)
    words = rot[np.arange(rows * groups * 16) % 8]
    return CodebookMatrix(rows, cols, padded, cent, scales, words,
                          np.asarray(row_ptr, np.uint32), np.asarray(packed, np.uint32))


def f16b(v):
    return int(f32_to_f16_bits(np.array([v], np.float32))[0])


@pytest.mark.parametrize("cols", [1, 129, 257, 385])
def test_cb4_decode_closed_form_fixture(cols):
    gold = np.load(os.path.join(GOLD, "cb4_closed_form.npz"))
    rows = 515
    vals = [0.33325195, -0.125, 0.0009765625]
    packed = [(f16b(v) << 16) | (cols - 1) for _ in range(rows) for v in vals]
    m = closed_form(rows, cols, np.arange(0, 3 * rows + 1, 3), packed)
    m.validate()
    for i, r in enumerate(gold[f"c{cols}_rows"]):
        got = oracle.decode_rows(m, int(r), 1)[0]
        assert np.array_equal(got.view(np.uint32), gold[f"c{cols}_expected"][i].view(np.uint32)), (cols, r)


def test_cb4_decode_hand_values():
    # row 0: word 0 is 0x76543210 (rotation 0) -> column c in 0..7 has index c,
    # scale group 0 is f16(0.125) (a power of two, so sc*cent is exact).
    m = closed_form(2, 256, [0, 0, 0], [])
    row = oracle.decode_rows(m, 0, 1)[0]
    cent = (np.arange(16, dtype=np.float32) - np.float32(7.5)) * np.float32(0.1234567)
    for c in range(8):
        assert row[c] == np.float32(cent[c] * np.float32(0.125))
    # word 1 is rotated left by 4 bits: nibble 0 = 7, nibble 1 = 0, ...
    assert row[8] == np.float32(cent[7] * np.float32(0.125))
    assert row[9] == np.float32(cent[0] * np.float32(0.125))
    # column 128 is group 1: scale f16(0.375)
    q = 0  # word 16 has rotation 0
    assert row[128] == np.float32(np.float32(0.375) * cent[q])


@pytest.mark.parametrize("rows", [1, 3, 4, 5, 7, 9, 17])
@pytest.mark.parametrize("cols", [1, 129, 257, 513])
def test_cb4_decode_duplicate_column_outliers(rows, cols):
    gold = np.load(os.path.join(GOLD, "cb4_dup_outlier.npz"))
    packed = [x for _ in range(rows) for x in
              (f16b(0.25) << 16, f16b(-0.125) << 16, (f16b(0.5) << 16) | (cols - 1))]
    m = closed_form(rows, cols, np.arange(0, 3 * rows + 1, 3), packed)
    got = oracle.decode_rows(m)
    assert np.array_equal(got.view(np.uint32), gold[f"r{rows}_c{cols}"].view(np.uint32))


# ---------------------------------------------------------------- GEMVs

def fp64_check(W, x, y, slack=4.0):
    """|y - W@x| <= slack * K * 2^-24 * sum|W||x| (+ tiny floor), per row."""
    W64 = W.astype(np.float64)
    x64 = x.astype(np.float64)
    exact = W64 @ x64
    bound = slack * max(W.shape[1], 1) * 2.0 ** -24 * (np.abs(W64) @ np.abs(x64)) + 1e-30
    err = np.abs(y.astype(np.float64) - exact)
    assert np.all(err <= bound), float(np.max(err / bound))


TAIL_ROWS = [1, 2, 3, 5, 7, 9, 16, 17]
TAIL_COLS = [1, 129, 257, 513, 544]


@pytest.mark.parametrize("cols", TAIL_COLS)
def test_cb4_gemv_fp64_bound_tail_shapes(cols):
    for rows in TAIL_ROWS:
        m = synth.make_cb4(rows, cols, seed=rows * 1000 + cols, outlier_frac=0.02)
        m.validate()
        x = synth.make_x_f32(1, cols, seed=cols)[0]
        y = oracle.gemv(m, x, threads=1)
        fp64_check(oracle.decode_rows(m), x, y)


def test_cb4_gemv_thread_count_invariance():
    m = synth.make_cb4(197, 544, seed=11)
    x = synth.make_x_f32(1, 544, seed=999)[0]
    y1 = oracle.gemv(m, x, threads=1)
    y4 = oracle.gemv(m, x, threads=4)
    y7 = oracle.gemv(m, x, threads=7)
    assert np.array_equal(y1.view(np.uint32), y4.view(np.uint32))
    assert np.array_equal(y1.view(np.uint32), y7.view(np.uint32))


def _order_case(shift):
    """One 128-group, scale 1.0; four columns starting at `shift` carry
    2^24, 1, 1, -2^24.  Interleaved acc[c % 4] + (a0+a1)+(a2+a3) decides."""
    cent = np.zeros(16, np.float32)
    cent[1], cent[2], cent[3] = 1.0, 2.0 ** 24, -(2.0 ** 24)
    words = np.zeros(32, np.uint32)  # padded 256 -> 2 groups * 16 words
    x = np.zeros(256, np.float32)
    for j, q in enumerate([2, 1, 1, 3]):
        c = shift + j
        words[c // 8] |= np.uint32(q << (4 * (c % 8)))
        x[c] = 1.0
    scales = np.array([f16b(1.0), 0], np.uint16)
    return CodebookMatrix(1, 256, 256, cent, scales, words, np.zeros(2, np.uint32),
                          np.zeros(0, np.uint32)), x


def test_cb4_gemv_accumulator_interleave_pinned():
    # shift 0: a0=2^24,a1=1,a2=1,a3=-2^24 -> (2^24+1)+(1-2^24) = 2^24 + -(2^24-1) = 1
    m, x = _order_case(0)
    assert oracle.gemv(m, x)[0] == 1.0
    # shift 1: a1=2^24,a2=1,a3=1,a0=-2^24 -> (-2^24+2^24)+(1+1) = 2
    m, x = _order_case(1)
    assert oracle.gemv(m, x)[0] == 2.0
    # shift 4 maps onto the same accumulators as shift 0
    m, x = _order_case(4)
    assert oracle.gemv(m, x)[0] == 1.0


def test_cb4_gemv_zero_scale_group_is_skipped():
    # codebook.rs:384-386: a zero scale skips the group, so an inf in x there
    # does not poison the row.
    m, x = _order_case(0)
    x[200] = np.inf  # group 1, scale 0
    assert oracle.gemv(m, x)[0] == 1.0


def test_cb4_gemv_outliers_after_interleave():
    m, x = _order_case(0)
    # one outlier on column 0 with residual 0.5: sum = fma(0.5, x[0]=1, 1) = 1.5
    m.outlier_row_ptr = np.array([0, 1], np.uint32)
    m.outliers_packed = np.array([(f16b(0.5) << 16) | 0], np.uint32)
    assert oracle.gemv(m, x)[0] == 1.5


@pytest.mark.parametrize("cols", [1, 63, 64, 65, 2048 + 64])
def test_g64_decode_and_gemv(cols):
    rows = 9
    m = synth.make_g64(rows, cols, seed=cols)
    m.validate()
    dec = oracle.decode_rows(m)
    idx = m.idx.reshape(rows, -1)
    c = np.arange(cols)
    q = (idx[:, c // 2] >> (4 * (c % 2)).astype(np.uint8)) & 0xF
    lut = m.lut_f16.reshape(rows, -1, 16).view(np.float16).astype(np.float32)
    ref = lut[np.arange(rows)[:, None], (c // 64)[None, :], q]
    assert np.array_equal(dec.view(np.uint32), ref.view(np.uint32))
    x = synth.make_x_f32(1, cols, seed=3)[0]
    y1 = oracle.gemv(m, x, threads=1)
    fp64_check(dec, x, y1)


def test_g64_gemv_thread_invariance():
    m = synth.make_g64(257, 2048, seed=4)
    x = synth.make_x_f32(1, 2048, seed=4)[0]
    assert np.array_equal(oracle.gemv(m, x, 1), oracle.gemv(m, x, 5))


# ---------------------------------------------------------------- Q8

def test_q8_dequant_exact_vs_numpy():
    m = synth.make_q8(33, 130, seed=0)
    deq = oracle.q8_dequant(m.blocks)
    ref = (m.qs().astype(np.float32) * m.scales_f16().view(np.float16).astype(np.float32)[:, None]).reshape(-1)
    assert np.array_equal(deq.view(np.uint32), ref.view(np.uint32))
    rows = oracle.decode_rows(m)
    assert np.array_equal(rows, ref.reshape(33, -1)[:, :130])


def test_q8_dot_two_chain_split_pinned():
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.array([f16b(1.0)], np.uint16).view(np.uint8)
    qs = np.zeros(32, np.int8)
    x = np.zeros(32, np.float32)
    # s0 chain (even): 2^24, then +1 (rounds away); s1 chain (odd): 1, then -2^24
    qs[0], x[0] = 1, 2.0 ** 24
    qs[2], x[2] = 1, 1.0
    qs[1], x[1] = 1, 1.0
    qs[3], x[3] = -1, 2.0 ** 24
    blk[2:] = qs.view(np.uint8)
    # (s0 + s1) * d = (2^24 + (1 - 2^24)) * 1 = 1 ; a single chain would give 0
    assert oracle.q8_dot(blk, x) == 1.0


def test_q8_dot_and_axpy_fp64():
    g = np.random.default_rng(8)
    for _ in range(50):
        src = g.standard_normal(32).astype(np.float32)
        blk = oracle.q8_quantize(src)
        w = oracle.q8_dequant(blk)
        x = g.standard_normal(32).astype(np.float32)
        fp64_check(w[None, :], x, np.array([oracle.q8_dot(blk, x)], np.float32))
        out = g.standard_normal(32).astype(np.float32)
        got = oracle.q8_axpy(blk, 0.37, out)
        exact = out.astype(np.float64) + w.astype(np.float64) * 0.37
        assert np.all(np.abs(got - exact) <= 1e-6 * (1 + np.abs(exact)))


def test_q8_quantize_properties():
    g = np.random.default_rng(9)
    for _ in range(200):
        src = (g.standard_normal(32) * g.uniform(0.01, 10)).astype(np.float32)
        blk = oracle.q8_quantize(src)
        d = float(np.array(blk[0:2]).view(np.uint16).view(np.float16).astype(np.float32)[0])
        qs = blk[2:].view(np.int8).astype(np.float64)
        amax = float(np.max(np.abs(src)))
        assert abs(d - amax / 127) <= amax / 127 * 2 ** -10
        assert np.max(np.abs(qs)) >= 126
        assert np.all(np.abs(qs * d - src) <= d / 2 * (1 + 2 ** -8) + 1e-12)
    # ties to even with d == 1.0 exactly (amax = 127)
    src = np.zeros(32, np.float32)
    src[0], src[1], src[2], src[3], src[4] = 127.0, 2.5, 3.5, -2.5, 0.5
    qs = oracle.q8_quantize(src)[2:].view(np.int8)
    assert list(qs[:5]) == [127, 2, 4, -2, 0]
    # all-zero block: d = 0, inv = 0, all q = 0
    z = oracle.q8_quantize(np.zeros(32, np.float32))
    assert not z.any()


@pytest.mark.parametrize("cols", [32, 33, 4096])
def test_q8_gemv_composition_and_bound(cols):
    rows = 17
    m = synth.make_q8(rows, cols, seed=cols)
    x = synth.make_x_f32(1, cols, seed=1)[0]
    y = oracle.gemv(m, x, threads=3)
    kb = m.blocks_per_row
    xp = np.zeros(kb * 32, np.float32)
    xp[:cols] = x
    blocks = m.blocks.reshape(rows, kb, 34)
    for r in range(rows):
        acc = np.float32(0.0)
        for b in range(kb):
            acc = np.float32(acc + np.float32(oracle.q8_dot(blocks[r, b], xp[32 * b:32 * b + 32])))
        assert acc == y[r]
    fp64_check(oracle.decode_rows(m), x, y)


# ---------------------------------------------------------------- GEMM

def _cos(a, b):
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    return a @ b / (np.linalg.norm(a) * np.linalg.norm(b))


@pytest.mark.parametrize("make", [
    lambda: synth.make_cb4(96, 256, seed=901),
    lambda: synth.make_g64(96, 256, seed=901),
    lambda: synth.make_q8(96, 256, seed=901),
])
def test_gemm_matches_per_token_gemv(make):
    m = make()
    X = synth.make_x_f32(11, 256, seed=902)
    ref = oracle.gemv_batch(m, X, threads=2)
    got = oracle.gemm(m, X, threads=2)
    assert _cos(ref, got) > 0.999999
    W = oracle.decode_rows(m)
    for i in range(11):
        fp64_check(W, X[i], got[i])


def test_gemm_worker_invariance_and_dense_chain():
    m = synth.make_g64(133, 320, seed=5)
    X = synth.make_x_f32(5, 320, seed=6)
    y1 = oracle.gemm(m, X, threads=1)
    y4 = oracle.gemm(m, X, threads=4)
    assert np.array_equal(y1.view(np.uint32), y4.view(np.uint32))
    # small integer-valued case: every partial sum is exact, so the chain's
    # result equals the exact product (pins indexing / operand orientation)
    rows, cols = 40, 96
    qs = np.random.default_rng(1).integers(-3, 4, size=(rows, cols)).astype(np.int8)
    from vxg_amd.formats import q8_from_planes
    q = q8_from_planes(rows, cols, qs, np.full(rows * 3, f16b(1.0), np.uint16))
    Xi = np.random.default_rng(2).integers(-5, 6, size=(3, cols)).astype(np.float32)
    got = oracle.gemm(q, Xi, threads=2)
    assert np.array_equal(got, (Xi.astype(np.int64) @ qs.T.astype(np.int64)).astype(np.float32))


# ---------------------------------------------------------------- greedy

def greedy_by_sets(a):
    """First index of numpy's nanmax; 0 when nothing is above -inf."""
    a = np.asarray(a, dtype=np.float32)
    ok = ~np.isnan(a)
    nf = bool((~np.isfinite(a)).any())
    if not ok.any():
        return 0, nf
    m = a[ok].max()
    if m == -np.inf:
        return 0, nf
    return int(np.flatnonzero(a == m)[0]), nf


@pytest.mark.parametrize("case", range(len(GREEDY_REFERENCE_CASES)))
def test_greedy_reference_cases(case):
    c = GREEDY_REFERENCE_CASES[case]
    assert oracle.greedy(greedy_reference_logits(c)) == (c[2], c[3])


def test_greedy_exhaustive_small_alphabet():
    import itertools
    alphabet = np.array([-np.inf, -1.0, -0.0, 0.0, 1e-45, 1.0, np.inf, np.nan], dtype=np.float32)
    assert oracle.greedy([]) == (0, False)
    for n in range(1, 5):
        for combo in itertools.product(range(len(alphabet)), repeat=n):
            a = alphabet[list(combo)]
            assert oracle.greedy(a) == greedy_by_sets(a), a


def test_greedy_random_vs_sets():
    g = np.random.default_rng(11)
    for trial in range(200):
        n = int(g.integers(1, 3000))
        a = g.standard_normal(n).astype(np.float32)
        if trial % 3 == 0:      # many exact ties
            a = np.round(a * 2).astype(np.float32)
        if trial % 5 == 0:
            a[g.integers(0, n, 3)] = np.nan
        if trial % 7 == 0:
            a[g.integers(0, n, 2)] = np.inf
        assert oracle.greedy(a) == greedy_by_sets(a)


# ---------------------------------------------------------------- embedding rows

def test_embed_rows_scale_rule():
    m = synth.make_cb4(40, 300, seed=3, outlier_frac=0.02)
    toks = [0, 39, 7, 7]
    base = oracle.decode_rows(m)[toks]
    assert np.array_equal(oracle.embed_rows(m, toks).view(np.uint32), base.view(np.uint32))
    below = np.float32(1.0) - np.float32(2.0 ** -24)           # |s - 1| < 1e-7: unscaled
    assert np.array_equal(oracle.embed_rows(m, toks, below).view(np.uint32), base.view(np.uint32))
    assert np.array_equal(oracle.embed_rows(m, toks, 2.0), base * 2)
    s = np.float32(np.sqrt(2048.0))
    want = (base.astype(np.float64) * np.float64(s)).astype(np.float32)   # one rounding (48-bit product)
    assert np.array_equal(oracle.embed_rows(m, toks, s).view(np.uint32), want.view(np.uint32))
    above = np.float32(1.0) + np.float32(2.0 ** -23)           # |s - 1| > 1e-7: scaled
    assert not np.array_equal(oracle.embed_rows(m, toks, above), base)
    with pytest.raises(ValueError):
        oracle.embed_rows(m, [40])


# ---------------------------------------------------------------- activations, rms_norm

def ulp_dist(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, np.int64(-2**31) - a, a)
    b = np.where(b < 0, np.int64(-2**31) - b, b)
    return np.abs(a - b)


def test_silu_and_gelu_vs_f64():
    x = np.concatenate([np.linspace(-90, 90, 20001), np.linspace(-1e-3, 1e-3, 2001)]).astype(np.float32)
    x = x[x != 0]
    xd = x.astype(np.float64)
    silu64 = (xd / (1.0 + np.exp(-xd))).astype(np.float32)
    fin = x > -88.0                        # exp(-x) finite in f32
    assert ulp_dist(oracle.silu(x[fin]), silu64[fin]).max() <= 4
    assert np.all(oracle.silu(x[x < -88.8]) == 0)   # f32 exp overflows: x / inf = -0
    # 1 + th cancels for large negative g (th rounds to -1 in f32): an absolute
    # error of 0.5 |g| ulp(1) on top of a relative 1e-6.
    g = oracle.gelu_tanh(x)
    ref = 0.5 * xd * (1.0 + np.tanh(0.7978846 * (xd + 0.044715 * xd ** 3)))
    assert np.all(np.abs(g - ref) <= 1e-6 * np.abs(ref) + 0.5 * np.abs(xd) * 2.0 ** -23)
    assert oracle.silu([0.0])[0] == 0 and oracle.gelu_tanh([0.0])[0] == 0
    assert oracle.silu([100.0])[0] == np.float32(100.0)
    assert oracle.silu([-200.0])[0] == 0 and np.signbit(oracle.silu([-200.0])[0])
    assert oracle.gelu_tanh([50.0])[0] == np.float32(50.0)
    assert np.all(oracle.silu(x[x < 0]) <= 0) and np.all(oracle.silu(x[x > 0]) > 0)


def test_glu_is_activation_times_up():
    g = np.random.default_rng(0).standard_normal(5000).astype(np.float32) * 4
    u = np.random.default_rng(1).standard_normal(5000).astype(np.float32)
    assert np.array_equal(oracle.glu(g, u), oracle.silu(g) * u)
    assert np.array_equal(oracle.glu(g, u, gelu=True), oracle.gelu_tanh(g) * u)


def test_rms_norm_pins():
    rng = np.random.default_rng(4)
    for n in (1, 7, 2048, 6144):
        x = rng.standard_normal(n).astype(np.float32) * 3
        w = rng.standard_normal(n).astype(np.float32)
        eps = 1e-6
        xd = x.astype(np.float64)
        ref = xd / np.sqrt((xd * xd).sum() / n + eps) * w.astype(np.float64)
        got = oracle.rms_norm(x, w, eps)
        assert np.all(np.abs(got - ref) <= 1e-6 * np.abs(ref) + 1e-30)
    c = np.full(100, 0.5, np.float32)
    got = oracle.rms_norm(c, np.ones(100, np.float32), 1e-5)
    assert np.allclose(got, 0.5 / np.sqrt(0.25 + 1e-5), rtol=1e-7, atol=0)
    assert np.array_equal(oracle.rms_norm(np.zeros(9, np.float32), np.ones(9, np.float32), 1e-6), np.zeros(9))
    x = rng.standard_normal(64).astype(np.float32)
    assert np.array_equal(oracle.rms_norm(x, np.full(64, 2.0, np.float32), 1e-6),
                          oracle.rms_norm(x, np.ones(64, np.float32), 1e-6) * 2)


# ---------------------------------------------------------------- attention over a Q8 cache

def q8_cache(seq, n_kv, hd, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    K = (rng.standard_normal((seq, n_kv * hd)) * scale).astype(np.float32)
    V = rng.standard_normal((seq, n_kv * hd)).astype(np.float32)
    kb = np.concatenate([oracle.kv_q8_blocks(K[t], n_kv, hd) for t in range(seq)])
    vb = np.concatenate([oracle.kv_q8_blocks(V[t], n_kv, hd) for t in range(seq)])
    return kb, vb


def attn_f64(q, kb, vb, seq, n_head, n_kv, hd):
    Kd = oracle.q8_dequant(kb).reshape(seq, n_kv, hd).astype(np.float64)
    Vd = oracle.q8_dequant(vb).reshape(seq, n_kv, hd).astype(np.float64)
    out = np.zeros((n_head, hd))
    for h in range(n_head):
        kv = h // (n_head // n_kv)
        s = Kd[:, kv, :] @ q.reshape(n_head, hd)[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ Vd[:, kv, :]
    return out.reshape(-1), np.abs(Vd).max()


def test_attn_q8_single_position_is_the_v_block():
    kb, vb = q8_cache(1, 2, 64, seed=1)
    q = np.random.default_rng(2).standard_normal(4 * 64).astype(np.float32)
    out = oracle.attn_q8(q, kb, vb, 1, 4, 2, 64).reshape(4, 64)
    vd = oracle.q8_dequant(vb).reshape(2, 64)
    for h in range(4):
        assert np.array_equal(out[h].view(np.uint32), vd[h // 2].view(np.uint32))


@pytest.mark.parametrize("seq,n_head,n_kv,hd", [(7, 4, 4, 32), (100, 8, 2, 128), (513, 4, 1, 64)])
def test_attn_q8_vs_f64(seq, n_head, n_kv, hd):
    kb, vb = q8_cache(seq, n_kv, hd, seed=seq, scale=0.3)
    q = np.random.default_rng(seq).standard_normal(n_head * hd).astype(np.float32)
    got = oracle.attn_q8(q, kb, vb, seq, n_head, n_kv, hd)
    ref, vmax = attn_f64(q, kb, vb, seq, n_head, n_kv, hd)
    assert np.abs(got - ref).max() <= 1e-5 * vmax


def test_attn_q8_gqa_mapping_uniform_scores_and_gate():
    seq, n_kv, hd = 9, 2, 32
    kb, vb = q8_cache(seq, n_kv, hd, seed=5)
    vb = vb.reshape(seq, n_kv, 1, 34).copy()
    vb[:, 1, :, 2:] = 0                                    # kv head 1: all-zero values
    vb = vb.reshape(-1, 34)
    q = np.random.default_rng(3).standard_normal(4 * hd).astype(np.float32)
    out = oracle.attn_q8(q, kb, vb, seq, 4, n_kv, hd).reshape(4, hd)
    assert np.all(out[2:] == 0) and np.any(out[:2] != 0)   # heads 2, 3 read kv head 1
    zero = oracle.attn_q8(np.zeros(4 * hd, np.float32), kb, vb, seq, 4, n_kv, hd).reshape(4, hd)
    vmean = oracle.q8_dequant(vb).reshape(seq, n_kv, hd).astype(np.float64).mean(axis=0)
    assert np.abs(zero[0] - vmean[0]).max() <= 1e-6 * np.abs(vmean[0]).max()
    g = np.random.default_rng(4).standard_normal(4 * hd).astype(np.float32)
    gated = oracle.attn_q8(q, kb, vb, seq, 4, n_kv, hd, gate=g).reshape(4, hd)
    sig = 1 / (1 + np.exp(-g.astype(np.float64)))
    assert np.allclose(gated, out * sig.reshape(4, hd), rtol=1e-6, atol=1e-30)


# ---------------------------------------------------------------- RoPE and the whole GQA step

def rope_f64(x, pos, rope_dim, base, neox):
    """The rotation of llm_ops.rs:81-99 as complex multiplication in f64; the
    angle is formed the reference's way (f32 exponent, f32 power rounded from
    f64, f32 product with the position) so the test sees the same angles."""
    x = np.asarray(x, np.float32).astype(np.float64).copy()
    rdim = min(rope_dim, x.size)
    half = rdim // 2
    for i in range(half):
        e = np.float32(-(np.float32(2.0) * np.float32(i))) / np.float32(rdim)
        freq = np.float32(np.float64(np.float32(base)) ** np.float64(e))
        theta = np.float64(np.float32(np.float32(pos) * freq))
        i0, i1 = (i, i + half) if neox else (2 * i, 2 * i + 1)
        z = complex(x[i0], x[i1]) * complex(np.cos(theta), np.sin(theta))
        x[i0], x[i1] = z.real, z.imag
    return x


@pytest.mark.parametrize("neox", [False, True])
@pytest.mark.parametrize("n,rope_dim", [(32, 32), (64, 32), (128, 128), (128, 64), (64, 7), (32, 0), (32, 1),
                                        (16, 40)])
@pytest.mark.parametrize("pos", [0, 1, 37, 4095, 40000])
def test_apply_rope_vs_complex_rotation(neox, n, rope_dim, pos):
    rng = np.random.default_rng(n * 7 + rope_dim + pos)
    x = (rng.standard_normal(n) * 2).astype(np.float32)
    for base in (10000.0, 1e6):
        got = oracle.apply_rope(x, pos, rope_dim, base, neox)
        ref = rope_f64(x, pos, rope_dim, base, neox)
        # two f32 products per output plus 1-ulp sin / cos, on |x| <= max|x|
        assert np.abs(got - ref).max() <= 2.0 ** -21 * np.abs(x).max()
        rdim = min(rope_dim, n)
        touched = np.zeros(n, bool)
        half = rdim // 2
        for i in range(half):
            touched[[i, i + half] if neox else [2 * i, 2 * i + 1]] = True
        assert np.array_equal(got[~touched].view(np.uint32), x[~touched].view(np.uint32))
        if pos == 0:
            assert np.array_equal(got, x)
        # a rotation keeps each pair's length
        i0 = np.arange(half) if neox else 2 * np.arange(half)
        i1 = i0 + half if neox else i0 + 1
        r_in = np.hypot(x[i0].astype(np.float64), x[i1].astype(np.float64))
        r_out = np.hypot(got[i0].astype(np.float64), got[i1].astype(np.float64))
        assert np.all(np.abs(r_out - r_in) <= 1e-6 * np.abs(x).max())


def gqa_inputs(p, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    q_raw = (rng.standard_normal(p.q_rows) * scale).astype(np.float32)
    k = (rng.standard_normal(p.n_kv * p.hd) * scale).astype(np.float32)
    v = rng.standard_normal(p.n_kv * p.hd).astype(np.float32)
    return q_raw, k, v


def prep_f64(p, q_raw, k, rope_pos):
    """Independent split / norm / rotation in f64 (llm_prefill.rs:284-309)."""
    hd = p.hd
    qs = np.asarray(q_raw, np.float64).reshape(p.n_head, (2 if p.gated else 1) * hd)
    q, gate = qs[:, :hd], (qs[:, hd:] if p.gated else None)

    def norm(x, w):
        if w is None:
            return x
        return x / np.sqrt((x * x).sum(axis=1, keepdims=True) / hd + p.eps) * w.astype(np.float64)

    qn, kn = norm(q, p.q_norm), norm(np.asarray(k, np.float64).reshape(p.n_kv, hd), p.k_norm)
    qr = np.stack([rope_f64(r.astype(np.float32), rope_pos, p.rope_dim, p.freq_base, p.neox) for r in qn])
    kr = np.stack([rope_f64(r.astype(np.float32), rope_pos, p.rope_dim, p.freq_base, p.neox) for r in kn])
    return qr.reshape(-1), gate, kr.reshape(-1)


@pytest.mark.parametrize("gated,norms,neox,rope_dim,hd", [
    (False, False, False, 0, 32), (True, True, True, 64, 64), (True, False, False, 32, 128),
    (False, True, True, 128, 128), (True, True, False, 16, 256)])
def test_gqa_prep_vs_f64_parts(gated, norms, neox, rope_dim, hd):
    rng = np.random.default_rng(hd + rope_dim)
    n_head, n_kv, pos, rope_pos = 8, 2, 5, 1234
    p = oracle.GqaStep(n_head, n_kv, hd, gated=gated, rope_dim=rope_dim, freq_base=1e6, neox=neox, eps=1e-6,
                       q_norm=rng.standard_normal(hd) if norms else None,
                       k_norm=rng.standard_normal(hd) if norms else None)
    q_raw, k, v = gqa_inputs(p, seed=hd, scale=3.0)
    blk = n_kv * hd // 32
    kb = np.zeros(((pos + 1) * blk, 34), np.uint8)
    vb = np.zeros_like(kb)
    qh, qg, k_rot = p.prep(q_raw, k, v, kb, vb, pos, rope_pos)
    q_ref, g_ref, k_ref = prep_f64(p, q_raw, k, rope_pos)
    qmax = np.abs(q_ref).max()
    assert np.abs(qh - q_ref).max() <= 2e-6 * qmax
    assert np.abs(k_rot - k_ref).max() <= 2e-6 * np.abs(k_ref).max()
    if gated:
        assert np.array_equal(qg, g_ref.reshape(-1).astype(np.float32))
    else:
        assert qg is None
    # row pos holds K (normed, rotated) and V, each KvQ8Block::quantize'd; rows below untouched
    assert np.array_equal(kb[pos * blk:], oracle.kv_q8_blocks(k_rot, n_kv, hd))
    assert np.array_equal(vb[pos * blk:], oracle.kv_q8_blocks(v, n_kv, hd))
    assert not kb[:pos * blk].any() and not vb[:pos * blk].any()


def test_gqa_step_is_prep_then_attention_over_positions_up_to_pos():
    n_head, n_kv, hd, S = 8, 2, 64, 40
    rng = np.random.default_rng(11)
    p = oracle.GqaStep(n_head, n_kv, hd, gated=True, rope_dim=64, freq_base=10000.0, neox=True, eps=1e-6,
                       q_norm=rng.standard_normal(hd), k_norm=rng.standard_normal(hd))
    blk = n_kv * hd // 32
    kb = np.zeros((S * blk, 34), np.uint8)
    vb = np.zeros_like(kb)
    for pos in range(S):
        q_raw, k, v = gqa_inputs(p, seed=100 + pos)
        kb2, vb2 = kb.copy(), vb.copy()
        out = p.step(q_raw, k, v, kb, vb, pos, pos + 3)
        qh, qg, _ = p.prep(q_raw, k, v, kb2, vb2, pos, pos + 3)
        assert np.array_equal(kb, kb2) and np.array_equal(vb, vb2)
        assert np.array_equal(out, oracle.attn_q8(qh, kb, vb, pos + 1, n_head, n_kv, hd, gate=qg))
        if pos in (0, S - 1):
            # brute force over the dequantised cache, the gate as the sigmoid factor
            ref, vmax = attn_f64(qh, kb[:(pos + 1) * blk], vb[:(pos + 1) * blk], pos + 1, n_head, n_kv, hd)
            sig = 1 / (1 + np.exp(-qg.astype(np.float64)))
            assert np.abs(out - ref * sig).max() <= 1e-5 * vmax
