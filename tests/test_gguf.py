"""GGUF reader (C++ parser in libqmm.so, Python mirror inference_amd.gguf) on the CPU.

Pinned by the reference reader's own tests (crates/llm/mlx-llm/src/gguf/reader.rs:
parse_minimal_gguf_roundtrip :380-436, rejects_bad_magic :438-446, rejects_v1
:448-456, oversized_header_count :458-467, parses_int_and_float_and_array_metadata
:469-500 -- the same byte images, built here), the engine's key-remap and q/k
un-permute tests (crates/llm/candle-llm/src/gguf.rs:528-605), the GGML block
table (mlx-llm/src/gguf/dequant.rs:114-140), and round trips through an
independent writer (tests/gguf_writer.py) that cover every value type,
alignments, offsets and truncations.
"""
import struct

import numpy as np
import pytest

from inference_amd import qmm
from inference_amd.gguf import GgufFile, MetaValue, is_ignorable, remap_key, tensor_byte_len, type_size, \
    unpermute_rows
import gguf_writer as W

MAGIC = W.MAGIC


def push_str(b, s):
    b += struct.pack("<Q", len(s)) + s.encode()


# -- the reference reader's tests, same images -------------------------------
def test_parse_minimal_gguf_roundtrip():
    b = bytearray(struct.pack("<IIQQ", MAGIC, 3, 1, 2))
    push_str(b, "general.architecture")
    b += struct.pack("<I", W.T_STRING)
    push_str(b, "llama")
    push_str(b, "llama.block_count")
    b += struct.pack("<II", W.T_UINT32, 7)
    push_str(b, "w")
    b += struct.pack("<IQQIQ", 2, 3, 2, 0, 0)  # n_dims, ne[0]=3, ne[1]=2, F32, offset 0
    while len(b) % 32:
        b.append(0)
    vals = [1.0, 2.0, 3.0, 4.0, 5.0, 6.0]
    b += struct.pack("<6f", *vals)
    g = GgufFile.parse(bytes(b))
    assert g.meta_str("general.architecture") == "llama"
    assert g.meta_u64("llama.block_count") == 7
    assert len(g.tensors) == 1
    t = g.tensors[0]
    assert t.name == "w" and t.shape == (2, 3) and t.num_elements() == 6
    assert list(g.tensor_data(t).view(np.float32)) == vals


def test_rejects_bad_magic():
    with pytest.raises(qmm.QmmError) as e:
        GgufFile.parse(struct.pack("<IIQQ", 0xDEADBEEF, 3, 0, 0))
    assert e.value.status == qmm.QMM_ERR_INVALID and "magic" in str(e.value)


def test_rejects_v1():
    with pytest.raises(qmm.QmmError) as e:
        GgufFile.parse(struct.pack("<IIQQ", MAGIC, 1, 0, 0))
    assert e.value.status == qmm.QMM_ERR_UNSUPPORTED


def test_oversized_header_count_is_an_error_without_preallocation():
    with pytest.raises(qmm.QmmError) as e:
        GgufFile.parse(struct.pack("<IIQQ", MAGIC, 3, 2 ** 64 - 1, 0))
    assert e.value.status == qmm.QMM_ERR_INVALID


def test_parses_int_and_float_and_array_metadata():
    b = bytearray(struct.pack("<IIQQ", MAGIC, 3, 0, 3))
    push_str(b, "a.f32")
    b += struct.pack("<If", W.T_FLOAT32, 1.5)
    push_str(b, "a.i64")
    b += struct.pack("<Iq", W.T_INT64, -42)
    push_str(b, "a.arr")
    b += struct.pack("<IIQII", W.T_ARRAY, W.T_UINT32, 2, 10, 20)
    g = GgufFile.parse(bytes(b))
    assert g.meta_f64("a.f32") == 1.5
    assert g.meta("a.i64").as_i64() == -42
    arr = g.meta("a.arr").as_array()
    assert [a.as_u64() for a in arr] == [10, 20]


# -- the engine's GGUF-load tests ---------------------------------------------
def test_remaps_keys():
    assert remap_key("token_embd.weight") == "model.embed_tokens.weight"
    assert remap_key("output_norm.weight") == "model.norm.weight"
    assert remap_key("output.weight") == "lm_head.weight"
    assert remap_key("blk.0.attn_q.weight") == "model.layers.0.self_attn.q_proj.weight"
    assert remap_key("blk.13.ffn_down.weight") == "model.layers.13.mlp.down_proj.weight"
    assert remap_key("blk.5.attn_norm.weight") == "model.layers.5.input_layernorm.weight"
    assert remap_key("blk.2.attn_q_norm.weight") == "model.layers.2.self_attn.q_norm.weight"
    assert remap_key("blk.0.some_future_tensor.weight") is None
    assert remap_key("rope_freqs.weight") is None
    assert remap_key("blk.x.attn_q.weight") is None
    assert is_ignorable("rope_freqs.weight") and is_ignorable("blk.0.rope_freqs.weight")
    assert not is_ignorable("blk.0.attn_q.weight")


def test_unpermute_inverts_llama_cpp_forward():
    n_head, head_dim, in_dim = 2, 4, 3
    out = n_head * head_dim
    hf = np.arange(out * in_dim, dtype=np.float32).reshape(out, in_dim)
    gguf = W.permute_rows(hf, n_head)
    assert not np.array_equal(gguf, hf)
    np.testing.assert_array_equal(gguf[unpermute_rows(out, n_head)], hf)
    for nh, hd in ((8, 128), (32, 64), (1, 2)):
        rows = np.arange(nh * hd)
        np.testing.assert_array_equal(W.permute_rows(rows[:, None], nh)[unpermute_rows(nh * hd, nh), 0], rows)


# -- GGML block table (dequant.rs:114-140) ------------------------------------
def test_type_sizes():
    table = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
             10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 20: (32, 18),
             23: (256, 136), 16: (256, 66), 17: (256, 74), 22: (256, 82), 18: (256, 98), 21: (256, 110),
             19: (256, 50), 29: (256, 56)}
    for tag, want in table.items():
        assert type_size(tag) == want
    for bad in (4, 5, 9, 15, 24, 31, 99):  # no block table entry (Q8_1 / Q8_K / removed tags included)
        with pytest.raises(qmm.QmmError):
            type_size(bad)
    assert tensor_byte_len(12, 14336 * 4096) == 33030144
    with pytest.raises(qmm.QmmError):
        tensor_byte_len(12, 255)


# -- writer round trips ---------------------------------------------------------
ALL_META = [
    ("u8", W.T_UINT8, 255), ("i8", W.T_INT8, -128), ("u16", W.T_UINT16, 65535), ("i16", W.T_INT16, -2),
    ("u32", W.T_UINT32, 4000000000), ("i32", W.T_INT32, -7), ("f32", W.T_FLOAT32, 0.25), ("bool", W.T_BOOL, True),
    ("str", W.T_STRING, "héllo"), ("empty", W.T_STRING, ""), ("u64", W.T_UINT64, 2 ** 64 - 1),
    ("i64", W.T_INT64, -(2 ** 63)), ("f64", W.T_FLOAT64, -1.0e300),
    ("arr.str", W.T_ARRAY, (W.T_STRING, ["a", "", "ccc"])), ("arr.bool", W.T_ARRAY, (W.T_BOOL, [True, False])),
    ("arr.f32", W.T_ARRAY, (W.T_FLOAT32, [1.0, -2.5])), ("arr.empty", W.T_ARRAY, (W.T_INT32, [])),
    ("arr.i8", W.T_ARRAY, (W.T_INT8, [-1, 0, 1])),
]


def tensors_of(rng):
    t = []
    for name, shape, tag in (("a.f32", (3, 5), 0), ("b.q4k", (4, 512), 12), ("c.q6k", (2, 256), 14),
                             ("d.q8_0", (3, 64), 8), ("e.f16", (7,), 1), ("f.bf16", (2, 2, 2), 30),
                             ("g.q5k", (1, 256), 13)):
        n = int(np.prod(shape))
        t.append((name, shape, tag, rng.integers(0, 256, tensor_byte_len(tag, n), dtype=np.uint8).tobytes()))
    return t


@pytest.mark.parametrize("alignment,version", [(32, 3), (64, 3), (1, 2), (256, 3)])
def test_writer_round_trip(alignment, version, tmp_path):
    rng = np.random.default_rng(alignment)
    meta = list(ALL_META)
    if alignment != 32:
        meta.append(("general.alignment", W.T_UINT32, alignment))
    tens = tensors_of(rng)
    img = W.build(meta, tens, alignment=alignment, version=version, pad_byte=0xAB)
    p = tmp_path / "m.gguf"
    p.write_bytes(img)
    for g in (GgufFile.parse(img), GgufFile.open(p)):
        assert g.version == version and g.alignment == alignment
        for k, t, v in meta:
            mv = g.meta(k)
            assert mv.type == t
            if t == W.T_ARRAY:
                et, items = v
                assert [x.type for x in mv.as_array()] == [et] * len(items)
                got = [x.value for x in mv.as_array()]
                assert got == (pytest.approx(items) if et == W.T_FLOAT32 else items)
            elif t == W.T_FLOAT32:
                assert mv.value == pytest.approx(v)
            else:
                assert mv.value == v
        assert [t.name for t in g.tensors] == [t[0] for t in tens]
        for info, (name, shape, tag, data) in zip(g.tensors, tens):
            assert info.shape == shape and info.ggml_type == tag and info.offset % alignment == 0
            assert g.tensor_data(info).tobytes() == data


def test_meta_value_coercions():
    mv = MetaValue
    assert mv(W.T_INT32, -1).as_u64() is None and mv(W.T_INT32, 5).as_u64() == 5
    assert mv(W.T_BOOL, True).as_u64() == 1 and mv(W.T_BOOL, True).as_i64() is None
    assert mv(W.T_UINT64, 2 ** 64 - 1).as_i64() == -1
    assert mv(W.T_FLOAT32, 1.5).as_u64() is None and mv(W.T_UINT8, 3).as_f64() is None
    assert mv(W.T_STRING, "x").as_str() == "x" and mv(W.T_UINT8, 1).as_str() is None
    img = W.build([("k", W.T_INT8, -3), ("k", W.T_UINT8, 9)], [])  # a repeated key keeps its last value
    assert GgufFile.parse(img).meta_u64("k") == 9
    img = W.build([("general.alignment", W.T_STRING, "64")], [("t", (32,), 0, bytes(128))])
    assert GgufFile.parse(img).alignment == 32  # a non-integer alignment keeps the default


def test_errors():
    good = W.build([("a", W.T_UINT32, 1), ("s", W.T_ARRAY, (W.T_STRING, ["xy", "z"]))],
                   [("t", (4, 256), 12, bytes(4 * 144))])
    g = GgufFile.parse(good)
    assert g.tensor_data(g.tensors[0]).size == 576
    header_end = len(good) - 576
    # every truncation: a header cut fails to parse; a data cut fails at tensor_data
    for cut in range(len(good)):
        try:
            g = GgufFile.parse(good[:cut])
        except qmm.QmmError as e:
            assert e.status == qmm.QMM_ERR_INVALID
            assert cut < header_end + 1
            continue
        assert cut >= header_end - 31  # parsed: the tables are whole
        with pytest.raises(qmm.QmmError):
            g.tensor_data(g.tensors[0])
    bad = [
        W.build([("n", W.T_ARRAY, (W.T_ARRAY, []))], []),  # nested array
        struct.pack("<IIQQ", MAGIC, 3, 0, 1) + W.gstr("k") + struct.pack("<I", 13),  # unknown value type
        struct.pack("<IIQQ", MAGIC, 3, 1, 0) + W.gstr("t") + struct.pack("<I", 0),  # 0 dims
        struct.pack("<IIQQ", MAGIC, 3, 1, 0) + W.gstr("t") + struct.pack("<I", 5),  # 5 dims
        struct.pack("<IIQQ", MAGIC, 3, 0, 1) + struct.pack("<Q", 2 ** 60),  # string longer than the file
    ]
    for img in bad:
        with pytest.raises(qmm.QmmError):
            GgufFile.parse(img)
    # elements not a multiple of the block, an unknown type, an offset past the end
    for shape, tag, off in (((100,), 12, 0), ((256,), 99, 0), ((256,), 12, 1 << 40)):
        img = bytearray(W.build([], [("t", shape, tag, bytes(64))]))
        if off:
            i = img.index(struct.pack("<I", tag) + struct.pack("<Q", 0))
            img[i + 4:i + 12] = struct.pack("<Q", off)
        g = GgufFile.parse(bytes(img))
        with pytest.raises(qmm.QmmError):
            g.tensor_data(g.tensors[0])
    with pytest.raises(qmm.QmmError):
        GgufFile.open("/nonexistent/file.gguf")
    # metadata-only files may end before the aligned data boundary
    assert GgufFile.parse(W.build([("x", W.T_UINT8, 1)], [])[:-1] if len(W.build([("x", W.T_UINT8, 1)], [])) % 32
                          else W.build([("x", W.T_UINT8, 1)], [])).meta_u64("x") == 1


def test_huge_alignment_is_rejected_not_wrapped():
    # general.alignment near 2^64: rounding the data start up must not wrap to
    # a small offset (the reference's div_ceil rejects such a file as a data
    # section past the end of the file)
    for a in (2 ** 64 - 1, 2 ** 63 + 1, 1 << 40):
        img = W.build([("general.alignment", W.T_UINT64, a)], [("t", (256,), 12, bytes(144))])
        with pytest.raises(qmm.QmmError) as e:
            GgufFile.parse(img)
        assert "past end of file" in str(e.value)


def test_resident_load_rejects_an_empty_dimension_before_any_device_work():
    # a 0 x 256 Q4_K tensor with a q/k un-permute: refused by the shape check
    # (the per-row byte count would otherwise divide by zero)
    import ctypes
    img = W.build([], [("t", (0, 256), 12, b"")])
    g = GgufFile.parse(img)
    out = ctypes.c_void_p()
    for heads in (0, 4):
        rc = qmm.lib().qmm_gguf_load_qtensor(g.handle, 0, heads, None, ctypes.byref(out))
        assert rc == qmm.QMM_ERR_INVALID and "empty dimension" in qmm.last_error()
        assert not out.value
