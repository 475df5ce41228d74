"""Config 4 at full size: the decode-step linear stack of 24 layers (hidden
2048, FFN 6144, q/k/v 16 heads x 128) with the 151,936-row Q8 LM head, on the
g64 layout and on the reference cb4 layout (per-part centroid tables, f16
group scales, CSR outliers; concatenated [q;k;v] and [gate;up] as the
reference's device packer builds them, metal_cb4_fast.mm:140-194).

Per projection against the oracle on the GPU's own inputs for layers 0 and
23 (layer 23's input is the output of the first 23 layers run on the
device), the LM head's logits against the oracle, and the captured graph of
the whole token replayed bit-identically to the eager launches.  Layers 1-22
share one set of host weights (each layer still has its own device copy);
layers 0 and 23 have their own.  The cb4 centroid tables are centred: with
no norms between the projections, a table with a non-zero mean makes the
activations grow about 150x per layer and overflow f32 by layer 18.
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine, stack, synth
from vxg_amd.formats import bf16_bits_to_f32

from parity_util import THREADS, assert_bf16_close, assert_bits_equal, floor_scale, q8_floor

pytestmark = pytest.mark.gpu

LAYERS, HIDDEN, FFN, VOCAB = 24, 2048, 6144, 151936


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine(0)
    yield e
    e.close()


def host_layer(kind, seed):
    gen = {"g64": lambda r, c, s: synth.make_g64(r, c, seed=s),
           "cb4": lambda r, c, s: synth.make_cb4(r, c, seed=s, outlier_frac=0.0074, centred=True)}[kind]
    qkv = [gen(HIDDEN, HIDDEN, seed + i) for i in range(3)]
    return qkv, gen(HIDDEN, HIDDEN, seed + 3), [gen(FFN, HIDDEN, seed + 4), gen(FFN, HIDDEN, seed + 5)], \
        gen(HIDDEN, FFN, seed + 6)


def upload(eng, h):
    qkv, o, gu, dn = h
    return stack.LayerWeights(eng.upload_concat(qkv), eng.upload_packed(o), eng.upload_concat(gu),
                              eng.upload_packed(dn))


def check(parts, x_bits, y_bits):
    x = bf16_bits_to_f32(x_bits)
    yref = np.concatenate([oracle.gemv(p, x, threads=THREADS) for p in parts])
    W = np.concatenate([oracle.decode_rows(p) for p in parts])
    assert_bf16_close(y_bits, yref, floor_scale(W, x[None])[0])


def check_layer(eng, lw, h, head, x_bits):
    """Run one layer (and the head) from x_bits; check each projection."""
    st = stack.DecodeStack(eng, [lw], head)
    st.set_input(x_bits)
    st.enqueue()
    eng.synchronize()
    qkv, o, gu, dn = h
    qkv_y = st.qkv_out.download(np.uint16, 3 * HIDDEN)
    check(qkv, x_bits, qkv_y)
    o_y = st.o_out.download(np.uint16, HIDDEN)
    check([o], qkv_y[:HIDDEN], o_y)
    gu_y = st.gu_out.download(np.uint16, 2 * FFN)
    check(gu, o_y, gu_y)
    dn_y = st.dn_out.download(np.uint16, HIDDEN)
    check([dn], gu_y[:FFN], dn_y)
    st.free()


@pytest.mark.parametrize("kind", ["g64", "cb4"])
def test_config4_stack_full_size(eng, kind):
    print(f"config 4 full stack kind={kind}", flush=True)
    h0, hmid, h23 = host_layer(kind, 100), host_layer(kind, 200), host_layer(kind, 300)
    head_h = synth.make_q8(VOCAB, HIDDEN, seed=5)
    head = eng.upload_packed(head_h)
    layers = [upload(eng, h0)] + [upload(eng, hmid) for _ in range(LAYERS - 2)] + [upload(eng, h23)]
    x0 = synth.make_x_bf16(1, HIDDEN, seed=4)[0]

    # layer 0 on the token's input
    check_layer(eng, layers[0], h0, head, x0)
    # layer 23 on the output of layers 0..22 computed on the device
    pre = stack.DecodeStack(eng, layers[:LAYERS - 1], head)
    pre.set_input(x0)
    pre.enqueue()
    eng.synchronize()
    x23 = pre.dn_out.download(np.uint16, HIDDEN)
    pre.free()
    check_layer(eng, layers[-1], h23, head, x23)

    # the whole token: eager, then the captured graph replayed
    st = stack.DecodeStack(eng, layers, head)
    st.set_input(x0)
    st.enqueue()
    eng.synchronize()
    logits = st.logits.download(np.float32, VOCAB)
    dn = st.dn_out.download(np.uint16, HIDDEN)
    x = bf16_bits_to_f32(dn)
    ref = oracle.gemv(head_h, x, threads=THREADS)
    fl = q8_floor(head_h, x)
    print(f"  final hidden: max |x| {np.max(np.abs(x)):.3e}, nonfinite {int((~np.isfinite(x)).sum())}; logits "
          f"max {np.max(np.abs(logits)):.3e} nonfinite {int((~np.isfinite(logits)).sum())}; ref nonfinite "
          f"{int((~np.isfinite(ref)).sum())}; floor min {fl.min():.3e}", flush=True)
    assert np.all(np.isfinite(logits)) and np.all(fl > 0)
    assert np.max(np.abs(logits - ref) / np.maximum(np.abs(ref), fl)) <= 1e-3
    g = st.capture()
    for _ in range(2):
        st.logits.upload(np.zeros(VOCAB, np.float32))
        g.launch(1)
        assert_bits_equal(st.logits.download(np.float32, VOCAB), logits)
        assert np.array_equal(st.dn_out.download(np.uint16, HIDDEN), dn)
    g.free()
    st.free()
    for L in layers:
        for t in (L.qkv, L.o, L.gate_up, L.down):
            t.free()
    head.free()
