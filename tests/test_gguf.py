"""GGUF files (no GPU): asmllm_amd.gguf_file against the reference's own
loader (src/loader/gguf_loader.c, built unchanged into oracle/_ref) and
against what the writer put in.

The reference loader honours general.alignment only when it is a uint32
(gguf_loader.c:151-155), so the files compared with it record it that way.
"""

import numpy as np
import pytest

from asmllm_amd import gguf
from asmllm_amd import gguf_file as gf
from oracle import gguf_ref

META = {
    "general.architecture": (gf.T_STRING, "llama"),
    "general.name": (gf.T_STRING, "synthetic"),
    "a.u8": (gf.T_UINT8, 200), "a.i8": (gf.T_INT8, -5), "a.u16": (gf.T_UINT16, 60000),
    "a.i16": (gf.T_INT16, -30000), "a.u32": (gf.T_UINT32, 4000000000), "a.i32": (gf.T_INT32, -7),
    "a.f32": (gf.T_FLOAT32, 0.5), "a.bool": (gf.T_BOOL, True), "a.u64": (gf.T_UINT64, 2 ** 40),
    "a.i64": (gf.T_INT64, -(2 ** 40)), "a.f64": (gf.T_FLOAT64, 1e-300),
    "a.ints": (gf.T_ARRAY, (gf.T_INT32, [1, -2, 3])),
    "tokenizer.ggml.tokens": (gf.T_ARRAY, (gf.T_STRING, ["<unk>", "<s>", "héllo", ""])),
}


def _tensors(rng):
    w4 = gguf.quantize_q4_0((rng.standard_normal((24, 96)) * 0.02).astype(np.float32))
    w8 = gguf.quantize_q8_0((rng.standard_normal((5, 64)) * 0.02).astype(np.float32))
    norm = rng.standard_normal(96).astype(np.float32)
    h = rng.standard_normal((3, 7)).astype(np.float16)
    w5 = gguf.pack_q5_0(rng.integers(0, 256, (6, 2, 16), dtype=np.uint8), rng.integers(0, 256, (6, 2, 4), dtype=np.uint8),
                        (rng.standard_normal((6, 2)) * 0.01).astype(np.float16))
    return {
        "blk.0.attn_q.weight": (gf.Q4_0, (96, 24), w4),
        "blk.0.ffn_down.weight": (gf.Q8_0, (64, 5), w8),
        "blk.0.attn_v.weight": (gf.Q5_0, (64, 6), w5),
        "output_norm.weight": (gf.F32, (96,), norm),
        "odd.f16": (gf.F16, (7, 3), h),
    }


@pytest.mark.parametrize("alignment", [32, 64, 4096, 8])
@pytest.mark.parametrize("version", [2, 3])
def test_round_trip(tmp_path, alignment, version):
    rng = np.random.default_rng(alignment + version)
    tensors = _tensors(rng)
    path = tmp_path / "m.gguf"
    gf.write_gguf(path, META, tensors, alignment=alignment, version=version)
    with gf.GGUFFile(path) as g:
        assert g.version == version and g.alignment == alignment
        assert g.data_offset % alignment == 0
        for key, (t, v) in META.items():
            got = g.metadata[key]
            if t == gf.T_ARRAY:
                assert got == list(v[1])
            elif t == gf.T_FLOAT32:
                assert got == np.float32(v)
            else:
                assert got == v
            assert g.metadata_types[key] == t
        assert g.vocab() == ["<unk>", "<s>", "héllo", ""]
        for name, (t, dims, data) in tensors.items():
            info = g.tensors[name]
            assert info.dims == dims and info.type == t and info.offset % alignment == 0
            np.testing.assert_array_equal(g.tensor(name), data.reshape(g.tensor(name).shape))
        assert g.tensor("blk.0.attn_q.weight").shape == (24, 3, 18)
        assert g.tensor("blk.0.ffn_down.weight").shape == (5, 2, 34)
        assert g.tensor("blk.0.attn_v.weight").shape == (6, 2, 22)
        assert g.tensor("odd.f16").shape == (3, 7)


needs_ref = pytest.mark.skipif(gguf_ref.lib() is None, reason="oracle/_ref/libgguf_ref.so not built "
                                                                "(the reference tree was not present at build)")


@needs_ref
@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_matches_the_reference_loader(tmp_path, alignment):
    rng = np.random.default_rng(7)
    tensors = _tensors(rng)
    path = tmp_path / "m.gguf"
    gf.write_gguf(path, META, tensors, alignment=alignment)
    ref = gguf_ref.load(path)
    assert ref is not None
    with gf.GGUFFile(path) as g:
        assert (ref["version"], ref["tensor_count"], ref["kv_count"]) == (g.version, len(g.tensors), len(g.metadata))
        assert ref["data_offset"] == g.data_offset
        assert ref["file_size"] == g.size
        assert set(ref["tensors"]) == set(g.tensors)
        for name, (dims, t, off, data_pos) in ref["tensors"].items():
            info = g.tensors[name]
            assert (dims, t, off) == (info.dims, info.type, info.offset)
            assert data_pos == g.data_offset + info.offset
            # the bytes the reference would hand out are the bytes of our view
            raw = np.fromfile(path, dtype=np.uint8, count=info.nbytes, offset=data_pos)
            np.testing.assert_array_equal(raw, g.tensor(name).view(np.uint8).reshape(-1))


@needs_ref
def test_reference_and_reader_refuse_the_same_files(tmp_path):
    good = tmp_path / "good.gguf"
    gf.write_gguf(good, META, _tensors(np.random.default_rng(1)))
    data = good.read_bytes()
    bad_magic = tmp_path / "magic.gguf"
    bad_magic.write_bytes(b"GGUX" + data[4:])
    v1 = tmp_path / "v1.gguf"
    v1.write_bytes(data[:4] + (1).to_bytes(4, "little") + data[8:])
    tiny = tmp_path / "tiny.gguf"
    tiny.write_bytes(data[:20])
    for p in (bad_magic, v1, tiny):
        assert gguf_ref.load(p) is None
        with pytest.raises(gf.GGUFError):
            gf.GGUFFile(p)


def test_truncated_tensor_data_is_an_error(tmp_path):
    path = tmp_path / "m.gguf"
    gf.write_gguf(path, META, _tensors(np.random.default_rng(2)))
    data = path.read_bytes()
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(data[:-200])
    with pytest.raises(gf.GGUFError):
        gf.GGUFFile(cut)


def test_alignment_defaults_to_32_and_any_integer_type_is_honoured(tmp_path):
    rng = np.random.default_rng(3)
    path = tmp_path / "m.gguf"
    meta = {**META, "general.alignment": (gf.T_UINT64, 128)}
    gf.write_gguf(path, meta, _tensors(rng), alignment=128)
    with gf.GGUFFile(path) as g:
        assert g.alignment == 128 and g.data_offset % 128 == 0
        np.testing.assert_array_equal(g.tensor("output_norm.weight"), _tensors(np.random.default_rng(3))[
            "output_norm.weight"][2])


def test_llama_shape_from_metadata(tmp_path):
    from asmllm_amd.engine import shape_from_gguf

    rng = np.random.default_rng(4)
    emb = gguf.quantize_q4_0((rng.standard_normal((300, 128)) * 0.02).astype(np.float32))
    meta = {"general.architecture": (gf.T_STRING, "llama"),
            "llama.embedding_length": (gf.T_UINT32, 128), "llama.block_count": (gf.T_UINT32, 3),
            "llama.feed_forward_length": (gf.T_UINT32, 256), "llama.attention.head_count": (gf.T_UINT32, 2),
            "llama.attention.head_count_kv": (gf.T_UINT32, 1),
            "llama.attention.layer_norm_rms_epsilon": (gf.T_FLOAT32, 1e-6),
            "llama.rope.freq_base": (gf.T_FLOAT32, 500000.0)}
    path = tmp_path / "m.gguf"
    gf.write_gguf(path, meta, {"token_embd.weight": (gf.Q4_0, (128, 300), emb)})
    with gf.GGUFFile(path) as g:
        s = shape_from_gguf(g)
    assert (s.dim, s.n_layers, s.hidden_dim, s.n_heads, s.n_kv_heads, s.vocab) == (128, 3, 256, 2, 1, 300)
    assert s.eps == np.float32(1e-6) and s.theta == 500000.0 and s.head_dim == 64
