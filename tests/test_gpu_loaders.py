"""GPU: tensors uploaded straight from container bytes.

A ``.vxt`` codebook entry (``vxt_hip_upload_vxt_entry``) and a GGUF Q8_0
matrix (``vxt_hip_upload_gguf_q8_0``) must dequantise bit-exactly to the
oracle's ``decode_row`` of the matrices that were written, and multiply like
them (the GEMV bar).
"""
import numpy as np
import pytest

import oracle
from vxg_amd import engine, loaders, synth
from vxg_amd.formats import CodebookMatrix, bf16_bits_to_f32
from archive_util import codebook_section, raw_f32_section, write_gguf, write_vxt
from parity_util import THREADS, assert_bits_equal, floor_scale, max_rel, run_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = engine.HipEngine()
    print(f"device: {e.device_name}", flush=True)
    yield e
    e.close()


def test_vxt_codebook_entries_upload(eng):
    cbs = {"blk.0.ffn_up": synth.make_cb4(40, 300, seed=1, outlier_frac=0.03),
           "x" * 13: synth.make_cb4(17, 2048, seed=2, outlier_frac=0.01),
           "blk.1.attn_o": synth.make_cb4(3, 1, seed=3)}
    data = write_vxt([("raw", raw_f32_section(np.ones((2, 2), np.float32)))]
                     + [(n, codebook_section(m)) for n, m in cbs.items()])
    with loaders.VxtArchive(data) as ar:
        for name, m in cbs.items():
            t = ar.upload(eng, name)
            assert (t.rows, t.cols) == (m.rows, m.cols)
            assert_bits_equal(eng.dequant_rows(t), oracle.decode_rows(m))
            x = synth.make_x_bf16(1, m.cols, seed=5)
            y = run_dev(eng, t, x, engine.DTYPE_BF16, 1, engine.DTYPE_F32)[0]
            xf = bf16_bits_to_f32(x)[0]
            ref = oracle.gemv(m, xf, threads=THREADS)
            assert max_rel(y, ref, floor_scale(oracle.decode_rows(m), xf[None])[0]) <= 1e-3
            t.free()
        with pytest.raises(engine.UnsupportedError):
            ar.upload(eng, "raw")


def test_vxt_three_bit_codebook_is_listed_not_uploaded(eng):
    m = synth.make_cb4(2, 256, seed=4)
    groups = m.rows * m.padded_cols // 128
    cb3 = CodebookMatrix(m.rows, m.cols, m.padded_cols, m.centroids, m.scales_f16,
                         np.zeros(groups * 12, np.uint32), m.outlier_row_ptr, m.outliers_packed, bits=3)
    with loaders.VxtArchive(write_vxt([("w3", codebook_section(cb3))])) as ar:
        assert ar["w3"].sub == 3
        with pytest.raises(engine.UnsupportedError):
            ar.upload(eng, "w3")


def test_gguf_q8_upload(eng):
    g = np.random.default_rng(0)
    mats = {}
    tensors = []
    for name, rows, cols in (("blk.0.attn_q.weight", 96, 2048), ("output.weight", 1000, 256), ("t", 1, 32)):
        m = synth.make_q8(rows, cols, seed=rows)
        mats[name] = m
        tensors.append((name, (cols, rows), 8, m.blocks.tobytes()))
    tensors.append(("norm", (256,), 0, g.standard_normal(256).astype(np.float32).tobytes()))
    with loaders.GgufFile(write_gguf(tensors, alignment=64)) as gf:
        for name, m in mats.items():
            t = gf.upload(eng, name)
            assert (t.rows, t.cols) == (m.rows, m.cols)
            assert_bits_equal(eng.dequant_rows(t), oracle.decode_rows(m))
            X = synth.make_x_bf16(2, m.cols, seed=1)
            Y = run_dev(eng, t, X, engine.DTYPE_BF16, 2, engine.DTYPE_F32)
            Xf = bf16_bits_to_f32(X)
            W = oracle.decode_rows(m)
            for i in range(2):
                assert max_rel(Y[i], oracle.gemv(m, Xf[i], threads=THREADS), floor_scale(W, Xf[i][None])[0]) <= 1e-3
            t.free()
        with pytest.raises(engine.UnsupportedError):
            gf.upload(eng, "norm")
