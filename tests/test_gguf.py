"""The GGUF reader (cuinfer::GGUFParser through cri_gguf_*) on files written by
tests/gguf_writer.py: the reference's parser test cases
(ref:tests/test_gguf_parser.cpp:149-930) restated, every metadata type, every
weight format's tensor layout, alignment, and malformed files.  Host code only:
no GPU needed."""
import numpy as np
import pytest

import cretif_amd as cri
from gguf_writer import (GGUFWriter, T_ARR, T_BOOL, T_F32, T_F64, T_I8, T_I16, T_I32, T_I64, T_STR, T_U8, T_U16,
                         T_U32, T_U64)

FILE_ERR, SHAPE_ERR = -6, -2


def write(tmp_path, w, name="m.gguf"):
    p = tmp_path / name
    w.write(str(p))
    return str(p)


def opens_with_error(path, text):
    with pytest.raises(cri.CretifError) as e:
        cri.GGUFFile(path)
    assert e.value.status == FILE_ERR
    assert text in str(e.value)


def test_minimal_file(tmp_path):
    with cri.GGUFFile(write(tmp_path, GGUFWriter())) as f:
        assert (f.version, f.tensor_count, f.metadata_count) == (3, 0, 0)


def test_version2(tmp_path):
    with cri.GGUFFile(write(tmp_path, GGUFWriter(version=2))) as f:
        assert f.version == 2


@pytest.mark.parametrize("v", [1, 4])
def test_unsupported_version(tmp_path, v):
    opens_with_error(write(tmp_path, GGUFWriter(version=v)), "Unsupported GGUF version")


def test_invalid_magic(tmp_path):
    opens_with_error(write(tmp_path, GGUFWriter(magic=b"GGML")), "magic")


def test_truncated_header(tmp_path):
    p = tmp_path / "t.gguf"
    p.write_bytes(b"GGUF" + (3).to_bytes(4, "little"))  # no counts
    opens_with_error(str(p), "too small")


def test_file_not_found(tmp_path):
    opens_with_error(str(tmp_path / "missing.gguf"), "cannot open")


def test_every_metadata_type(tmp_path):
    w = GGUFWriter()
    w.add("u8", T_U8, 200).add("i8", T_I8, -100).add("u16", T_U16, 60000).add("i16", T_I16, -30000)
    w.add("llama.context_length", T_U32, 4096).add("test.negative", T_I32, -42).add("f32", T_F32, 0.125)
    w.add("flag", T_BOOL, True).add("general.architecture", T_STR, "llama")
    w.add("test.big_number", T_U64, 0xDEADBEEFCAFE0000).add("i64", T_I64, -(1 << 40)).add("f64", T_F64, 2.5)
    w.add("arr", T_ARR, (T_U32, [10, 20, 30]))
    w.add("nested", T_ARR, (T_ARR, [(T_STR, ["a", "bc"]), (T_STR, [])]))
    w.add("strs", T_ARR, (T_STR, ["x" * 100, "", "é"]))
    with cri.GGUFFile(write(tmp_path, w)) as f:
        assert f.metadata_count == 15
        for key, tag in (("u8", T_U8), ("i8", T_I8), ("u16", T_U16), ("i16", T_I16), ("f32", T_F32),
                         ("flag", T_BOOL), ("i64", T_I64), ("f64", T_F64), ("arr", T_ARR), ("nested", T_ARR)):
            assert f.metadata_type(key) == tag
        assert f.get_u32("llama.context_length") == 4096
        assert f.get_i32("test.negative") == -42
        assert f.get_u64("test.big_number") == 0xDEADBEEFCAFE0000
        assert f.get_f32("f32") == 0.125
        assert f.get_string("general.architecture") == "llama"
        assert f.array_length("arr") == 3 and f.array_length("nested") == 2 and f.array_length("strs") == 3
        assert f.metadata_type("absent") == -1


def test_type_mismatch_and_missing_key(tmp_path):
    w = GGUFWriter().add("test.value", T_U32, 100)
    with cri.GGUFFile(write(tmp_path, w)) as f:
        assert f.get_u32("test.value") == 100
        for getter in (f.get_string, f.get_f32, f.get_i32, f.get_u64, f.array_length):
            with pytest.raises(cri.CretifError) as e:
                getter("test.value")
            assert e.value.status == SHAPE_ERR and "mismatch" in str(e.value)
        with pytest.raises(cri.CretifError) as e:
            f.get_string("nonexistent.key")
        assert "not found" in str(e.value)


BLOCK = {"f32": (4, 1), "f16": (2, 1), "q4_0": (18, 32), "q4_1": (20, 32), "q5_0": (22, 32), "q8_0": (34, 32),
         "q4_k": (144, 256), "q6_k": (210, 256), "q2_k": (84, 256), "q3_k": (110, 256), "q5_k": (176, 256)}
FORMAT = {"f32": 6, "f16": 5, "q4_0": 1, "q5_0": 2, "q8_0": 0, "q4_k": 3, "q6_k": 4}


@pytest.mark.parametrize("alignment", [32, 64])
def test_tensors_of_every_layout(tmp_path, alignment):
    rng = np.random.default_rng(1)
    w = GGUFWriter(alignment=alignment)
    if alignment != 32:
        w.add("general.alignment", T_U32, alignment)
    expect = {}
    for i, (t, (bb, be)) in enumerate(BLOCK.items()):
        K, N = 512, 3 + i
        data = rng.integers(0, 256, size=N * K // be * bb, dtype=np.uint8)
        w.add_tensor("blk.%d.%s.weight" % (i, t), [K, N], t, data)
        expect["blk.%d.%s.weight" % (i, t)] = (t, K, N, data)
    w.add_tensor("norm", [8], "f32", np.arange(8, dtype=np.float32))
    path = write(tmp_path, w)
    with cri.GGUFFile(path) as f:
        assert f.tensor_count == len(expect) + 1
        for name, (t, K, N, data) in expect.items():
            i = f.find_tensor(name)
            info = f.tensor(i)
            assert info["dims"] == [K, N] and info["n_elements"] == K * N
            assert info["byte_size"] == data.size
            assert info["format"] == FORMAT.get(t, -1)
            assert info["data_offset"] % alignment == 0
            assert info["data_offset"] == w.data_start + w.offsets[i]
            assert np.array_equal(f.tensor_bytes(i), data)
        n = f.tensor(f.find_tensor("norm"))
        assert n["dims"] == [8] and np.array_equal(f.tensor_bytes(f.find_tensor("norm")).view(np.float32),
                                                   np.arange(8, dtype=np.float32))
        assert f.find_tensor("nonexistent") is None


def test_unknown_tensor_type_is_listed(tmp_path):
    w = GGUFWriter().add_tensor("odd", [16], 99, b"\0" * 16)
    with cri.GGUFFile(write(tmp_path, w)) as f:
        info = f.tensor(0)
        assert info["byte_size"] == -1 and info["format"] == -1


def test_tensor_past_end_of_file_rejected(tmp_path):
    w = GGUFWriter().add_tensor("w", [256, 4], "q4_k", b"\0" * (4 * 144))
    b = w.tobytes()
    p = tmp_path / "short.gguf"
    p.write_bytes(b[:-10])
    opens_with_error(str(p), "past the end")


def test_overflowing_dimensions_rejected(tmp_path):
    # {2^62 + 1, 4}: the element count wraps to 4 in 64 bits and the byte size to 16, which would
    # pass the end-of-file check; the reader must refuse the product instead
    w = GGUFWriter().add_tensor("w", [(1 << 62) + 1, 4], "f32", b"\0" * 16)
    opens_with_error(write(tmp_path, w), "overflows")
    # a Q8_0 tensor whose element count (31 * 2^59) fits but whose byte size (n / 32 * 34) does not
    w = GGUFWriter().add_tensor("w", [32, 31 << 54], "q8_0", b"\0" * 34)
    opens_with_error(write(tmp_path, w, "b.gguf"), "overflows")


def test_unknown_type_with_overflowing_dims_is_listed(tmp_path):
    w = GGUFWriter().add_tensor("odd", [1 << 40, 1 << 40], 99, b"\0" * 16)
    with cri.GGUFFile(write(tmp_path, w)) as f:
        info = f.tensor(0)
        assert info["n_elements"] == -1 and info["byte_size"] == -1


def test_partial_block_rejected(tmp_path):
    w = GGUFWriter().add_tensor("w", [100], "q8_0", b"\0" * 136)
    opens_with_error(write(tmp_path, w), "not a multiple")


def test_absurd_counts_rejected(tmp_path):
    import struct

    b = bytearray(GGUFWriter().add("arr", T_ARR, (T_U8, [1, 2])).tobytes())
    # patch the array length (after magic, version, counts, key, type tag, element type) to 2^60
    key_end = 4 + 4 + 8 + 8 + 8 + len("arr") + 4 + 4
    b[key_end:key_end + 8] = struct.pack("<Q", 1 << 60)
    p = tmp_path / "huge.gguf"
    p.write_bytes(bytes(b))
    opens_with_error(str(p), "array of")
    c = bytearray(GGUFWriter().tobytes())
    c[8:16] = struct.pack("<Q", 1 << 40)  # tensor count
    p.write_bytes(bytes(c))
    opens_with_error(str(p), "counts exceed")


def test_unknown_metadata_type_rejected(tmp_path):
    import struct

    b = GGUFWriter().tobytes()[:16] + struct.pack("<Q", 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13)
    p = tmp_path / "bad.gguf"
    p.write_bytes(b + b"\0" * 16)
    opens_with_error(str(p), "unknown metadata value type")


def test_full_model_like_file(tmp_path):
    # ref:tests/test_gguf_parser.cpp:507-633 (FullModelLikeFile)
    w = GGUFWriter().add("general.architecture", T_STR, "llama").add("llama.context_length", T_U32, 512)
    w.add("llama.embedding_length", T_U32, 8).add("llama.block_count", T_U32, 2)
    w.add("llama.attention.head_count", T_U32, 4).add("llama.attention.head_count_kv", T_U32, 2)
    w.add("llama.feed_forward_length", T_U32, 32).add("llama.rope.dimension_count", T_U32, 2)
    w.add("tokenizer.ggml.tokens", T_ARR, (T_STR, ["<s>", "</s>", "a", "b", "c"]))
    w.add_tensor("token_embd.weight", [8, 5], "f32", np.zeros(40, np.float32))
    w.add_tensor("output_norm.weight", [8], "f32", np.ones(8, np.float32))
    with cri.GGUFFile(write(tmp_path, w)) as f:
        m = f.model_params()
        assert m["architecture"] == "llama"
        assert (m["context_length"], m["embedding_length"], m["block_count"], m["head_count"], m["head_count_kv"],
                m["feed_forward_length"], m["rope_dimension_count"]) == (512, 8, 2, 4, 2, 32, 2)
        assert m["vocab_size"] == 5                          # from the tokens array
        assert m["rope_freq_base"] == 10000.0                # default
        assert m["rms_norm_eps"] == np.float32(1e-5)         # default
        assert m["tie_word_embeddings"] is True              # no output.weight


def test_model_params_explicit_and_missing(tmp_path):
    w = GGUFWriter().add("general.architecture", T_STR, "llama").add("llama.vocab_size", T_U32, 49152)
    w.add("llama.rope.freq_base", T_F32, 500000.0).add("llama.attention.layer_norm_rms_epsilon", T_F32, 1e-6)
    w.add_tensor("output.weight", [256, 2], "q6_k", b"\0" * 420)
    with cri.GGUFFile(write(tmp_path, w)) as f:
        m = f.model_params()
        assert m["vocab_size"] == 49152 and m["rope_freq_base"] == 500000.0
        assert m["rms_norm_eps"] == np.float32(1e-6) and m["tie_word_embeddings"] is False
        assert m["context_length"] is None and m["block_count"] is None
    with cri.GGUFFile(write(tmp_path, GGUFWriter(), "empty.gguf")) as f:
        with pytest.raises(cri.CretifError):
            f.model_params()  # no general.architecture
