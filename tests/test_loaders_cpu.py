"""CPU checks of the container readers (``vxt_hip_vxt_parse``,
``vxt_hip_gguf_parse``; no device needed).

Archives are written with ``archive_util`` (a restatement of the reference
writer) and read back through the native reader; the rejection cases are the
reference's own (archive_structure_validation.rs:76-128, format.rs:301-451,
gguf.rs:83-172).
"""
import struct

import numpy as np
import pytest

from vxg_amd import engine, loaders, synth
from vxg_amd.formats import CodebookMatrix, FormatError, Q4_0Matrix, q8_from_planes
from archive_util import (codebook_section, lossless_section, q4_0_section, raw_f32_section, wht2_section,
                          write_gguf, write_vxt)


def same_codebook(a, b):
    assert (a.rows, a.cols, a.padded_cols, a.bits) == (b.rows, b.cols, b.padded_cols, b.bits)
    for f in ("centroids", "scales_f16", "packed_words", "outlier_row_ptr", "outliers_packed"):
        assert np.array_equal(np.asarray(getattr(a, f)).view(np.uint8), np.asarray(getattr(b, f)).view(np.uint8)), f


def test_vxt_round_trip_mixed_kinds_and_metadata():
    cbs = [synth.make_cb4(r, c, seed=r + c, outlier_frac=0.05) for r, c in ((7, 300), (33, 1024), (1, 1))]
    entries = [("blk.0.raw", raw_f32_section(np.arange(12, dtype=np.float32).reshape(3, 4))),
               ("blk.0.ffn_up", codebook_section(cbs[0])),
               ("blk.0.q4", q4_0_section(2, 40)),
               ("a" * 77, codebook_section(cbs[1])),        # odd name length: misaligned planes
               ("wht", wht2_section(2, 3)),
               ("ll", lossless_section(1, 10)),
               ("tiny", codebook_section(cbs[2]))]
    meta = [("general.name", b"demo"), ("tokenizer", bytes(range(256)) * 3)]
    data = write_vxt(entries, meta)
    with loaders.VxtArchive(data) as ar:
        assert ar.meta_count == 2
        assert [e.name for e in ar.entries] == [n for n, _ in entries]
        assert [e.kind for e in ar.entries] == [5, 2, 3, 2, 4, 1, 2]
        same_codebook(ar.codebook("blk.0.ffn_up"), cbs[0])
        same_codebook(ar.codebook("a" * 77), cbs[1])
        same_codebook(ar.codebook("tiny"), cbs[2])
        assert ar["blk.0.ffn_up"].raw.section_off % 64 == 0
        with pytest.raises(engine.UnsupportedError):
            ar.codebook("wht")


def test_vxt_from_a_file(tmp_path):
    cb = synth.make_cb4(5, 256, seed=1)
    p = tmp_path / "m.vxt"
    p.write_bytes(write_vxt([("w", codebook_section(cb))]))
    with loaders.VxtArchive(str(p)) as ar:
        same_codebook(ar.codebook("w"), cb)


def tiny_codebook(ptr, outliers):
    """archive_structure_validation.rs:76-88: 2 x 3, padded 256."""
    return CodebookMatrix(2, 3, 256, np.zeros(16, np.float32), np.zeros(4, np.uint16), np.zeros(64, np.uint32),
                          np.array(ptr, np.uint32), np.array(outliers, np.uint32))


@pytest.mark.parametrize("ptr,outliers", [([1, 1, 1], [0]), ([0, 2, 1], [0]), ([0, 0xFFFFFFFF, 1], [0]),
                                          ([0, 0, 1], [3])])
def test_vxt_rejects_bad_outlier_csr(ptr, outliers):
    """archive_structure_validation.rs:102-116 (both tags valid)."""
    with pytest.raises(FormatError, match="CSR|plane lengths"):
        loaders.VxtArchive(write_vxt([("w", codebook_section(tiny_codebook(ptr, outliers)))]))


def test_vxt_accepts_valid_tiny_csr():
    with loaders.VxtArchive(write_vxt([("w", codebook_section(tiny_codebook([0, 0, 1], [2])))])) as ar:
        assert ar.codebook("w").outliers_packed.tolist() == [2]


def test_vxt_header_and_plane_rules():
    cb = synth.make_cb4(4, 300, seed=3, pad_to=128)          # padded 384: not the archive's 512
    with pytest.raises(FormatError, match="codebook header"):
        loaders.VxtArchive(write_vxt([("w", codebook_section(cb))]))
    good = synth.make_cb4(4, 300, seed=3)
    kind, sub, rows, cols, pcols, payload = codebook_section(good)
    with pytest.raises(FormatError, match="codebook header"):
        loaders.VxtArchive(write_vxt([("w", (kind, 5, rows, cols, pcols, payload))]))
    short = CodebookMatrix(good.rows, good.cols, good.padded_cols, good.centroids, good.scales_f16[:-1],
                           good.packed_words, good.outlier_row_ptr, good.outliers_packed)
    with pytest.raises(FormatError, match="plane lengths"):
        loaders.VxtArchive(write_vxt([("w", codebook_section(short))]))
    for r, c, p in ((0, 3, 256), (2, 0, 256), (2, 300, 256), (2 ** 63, 3, 256), (2, 2 ** 63, 2 ** 63)):
        with pytest.raises(FormatError, match="dimensions"):
            loaders.VxtArchive(write_vxt([("w", (2, 4, r, c, p, b""))]))


def test_vxt_checksums_magic_version_truncation():
    data = bytearray(write_vxt([("w", codebook_section(synth.make_cb4(3, 256, seed=2)))]))
    bad = bytearray(data)
    bad[200] ^= 1
    with pytest.raises(FormatError, match="archive checksum"):
        loaders.VxtArchive(bytes(bad))
    # corrupt the section but re-tag the archive: the section tag must catch it
    from archive_util import fnv1a64
    bad2 = bytearray(data)
    bad2[200] ^= 1
    bad2[-8:] = struct.pack("<Q", fnv1a64(bytes(bad2[:-8])))
    with pytest.raises(FormatError, match="integrity"):
        loaders.VxtArchive(bytes(bad2))
    with pytest.raises(FormatError, match="magic"):
        loaders.VxtArchive(b"VXT2" + bytes(data[4:]))
    with pytest.raises(engine.UnsupportedError):
        loaders.VxtArchive(write_vxt([], version=2))
    with pytest.raises(FormatError, match="truncated"):
        loaders.VxtArchive(bytes(data[:20]))
    with pytest.raises(FormatError):
        loaders.VxtArchive(write_vxt([("w", (9, 0, 1, 1, 1, b""))]))       # unknown kind
    with pytest.raises(engine.UnsupportedError):
        loaders.VxtArchive(write_vxt([("w", (7, 4, 1, 1, 256, b""))]))     # entropy-coded section


def test_vxt_truncated_plane_count_is_rejected():
    """A plane count larger than the rest of the archive (both tags valid)."""
    payload = np.zeros(16, np.float32).tobytes() + struct.pack("<Q", 2 ** 61)
    with pytest.raises(FormatError, match="truncated"):
        loaders.VxtArchive(write_vxt([("w", (2, 4, 1, 1, 256, payload))]))


# ---------------------------------------------------------------- GGUF

def q8_bytes(rows, cols, seed):
    g = np.random.default_rng(seed)
    kb = cols // 32
    qs = g.integers(-127, 128, size=rows * kb * 32).astype(np.int8)
    d = np.float16(g.uniform(0.002, 0.02, size=rows * kb)).view(np.uint16)
    return q8_from_planes(rows, cols, qs, d)


ALL_KV = [("general.architecture", 8, "qwen35"), ("a.u8", 0, 7), ("a.i8", 1, -3), ("a.u16", 2, 500),
          ("a.i16", 3, -500), ("a.u32", 4, 70000), ("a.i32", 5, -70000), ("a.f32", 6, 1.5), ("a.bool", 7, True),
          ("a.arr", 9, (4, [1, 2, 3])), ("a.strs", 9, (8, ["x", "yy"])), ("a.nest", 9, (9, [(4, [5]), (4, [])])),
          ("a.u64", 10, 2 ** 40), ("a.i64", 11, -(2 ** 40)), ("a.f64", 12, 2.5)]


@pytest.mark.parametrize("version,alignment", [(3, None), (2, 64), (3, 256)])
def test_gguf_tensor_table_and_q8_bytes(version, alignment):
    qa, qb = q8_bytes(6, 64, 1), q8_bytes(3, 32, 2)
    f32 = np.arange(10, dtype=np.float32)
    tensors = [("blk.0.attn_q.weight", (64, 6), 8, qa.blocks.tobytes()),
               ("output_norm.weight", (10,), 0, f32.tobytes()),
               ("blk.0.ffn.weight", (32, 3, 1), 8, qb.blocks.tobytes()),
               ("odd", (4, 4), 99, b"\x00" * 16)]
    data = write_gguf(tensors, ALL_KV, version=version, alignment=alignment)
    with loaders.GgufFile(data) as gf:
        assert gf.version == version and gf.alignment == (alignment or 32)
        assert [t.name for t in gf.tensors] == [t[0] for t in tensors]
        assert gf["blk.0.attn_q.weight"].matrix_dims() == (6, 64)
        assert gf["blk.0.ffn.weight"].matrix_dims() == (3, 32)
        assert np.array_equal(gf.tensor_bytes("output_norm.weight").view(np.float32), f32)
        m = gf.q8("blk.0.attn_q.weight")
        assert (m.rows, m.cols) == (6, 64) and np.array_equal(m.blocks, qa.blocks)
        assert np.array_equal(gf.q8("blk.0.ffn.weight").blocks, qb.blocks)
        assert not gf["odd"].supported
        with pytest.raises(engine.UnsupportedError):
            gf.tensor_bytes("odd")
        for t in gf.tensors:
            if t.supported:
                assert t.raw.data_off % gf.alignment == 0


def test_gguf_errors():
    good = write_gguf([("w", (32, 2), 8, q8_bytes(2, 32, 0).blocks.tobytes())])
    with pytest.raises(FormatError, match="magic"):
        loaders.GgufFile(b"GGUG" + good[4:])
    with pytest.raises(engine.UnsupportedError):
        loaders.GgufFile(write_gguf([], version=1))
    with pytest.raises(FormatError, match="past EOF"):
        loaders.GgufFile(good[:-40])      # 68 tensor bytes padded to 96: cut into the tensor
    with pytest.raises(FormatError, match="value type"):
        loaders.GgufFile(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13))
    with pytest.raises(FormatError, match="n_dims"):
        loaders.GgufFile(write_gguf([("w", tuple([1] * 9), 0, b"\x00" * 4)]))
    with pytest.raises(FormatError, match="truncated|larger"):
        loaders.GgufFile(good[:30])


def _q40(rows, cols, seed):
    g = np.random.default_rng(seed)
    kb = (cols + 31) // 32
    sc = g.integers(0, 0x7C00, rows * kb, dtype=np.uint16)
    qw = g.integers(0, 2**32, rows * kb * 4, dtype=np.uint64).astype(np.uint32)
    return Q4_0Matrix(rows, cols, kb * 32, sc, qw)


def test_vxt_q4_0_planes_and_rules():
    m = _q40(3, 70, 4)
    with loaders.VxtArchive(write_vxt([("q", q4_0_section(0, 0, m))])) as ar:
        e = ar["q"]
        assert (e.kind, e.rows, e.cols, e.padded_cols) == (3, 3, 70, 96)
        got = ar.q4_0("q")
        assert np.array_equal(got.scales_f16, m.scales_f16) and np.array_equal(got.qs_words, m.qs_words)
        with pytest.raises(engine.UnsupportedError):
            ar.codebook("q")
    kind, sub, rows, cols, pcols, payload = q4_0_section(0, 0, m)
    with pytest.raises(FormatError, match="invalid VXT Q4_0 padded_cols"):
        loaders.VxtArchive(write_vxt([("q", (kind, sub, rows, cols, 128, payload))]))
    short = Q4_0Matrix(m.rows, m.cols, m.padded_cols, m.scales_f16[:-1], m.qs_words)
    with pytest.raises(FormatError, match="corrupt VXT Q4_0 plane lengths"):
        loaders.VxtArchive(write_vxt([("q", q4_0_section(0, 0, short))]))


def test_gguf_q4_0_blocks_to_planes():
    m = _q40(4, 64, 5)
    data = write_gguf([("w", (64, 4), 2, m.gguf_blocks().tobytes())])
    with loaders.GgufFile(data) as gf:
        got = gf.q4_0("w")
        assert (got.rows, got.cols, got.padded_cols) == (4, 64, 64)
        assert np.array_equal(got.scales_f16, m.scales_f16) and np.array_equal(got.qs_words, m.qs_words)
        with pytest.raises(engine.UnsupportedError):
            gf.q8("w")
