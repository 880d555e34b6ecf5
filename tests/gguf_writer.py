"""GGUF v2/v3 image writer for the tests (test infrastructure, not part of the package).

Writes the container as the GGUF spec lays it out (little-endian header,
typed key/value table, tensor-info table with ne dims fastest-first, data
section at the first `alignment` boundary, each tensor's data at an offset
that is a multiple of the alignment) so the reader can be checked against
independently built images.
"""
import struct

import numpy as np

T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY, T_UINT64, T_INT64, \
    T_FLOAT64 = range(13)
_FMT = {T_UINT8: "<B", T_INT8: "<b", T_UINT16: "<H", T_INT16: "<h", T_UINT32: "<I", T_INT32: "<i",
        T_FLOAT32: "<f", T_BOOL: "<?", T_UINT64: "<Q", T_INT64: "<q", T_FLOAT64: "<d"}
MAGIC = 0x46554747


def gstr(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def value(t, v):
    if t == T_STRING:
        return gstr(v)
    if t == T_ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def build(metadata, tensors, alignment=32, version=3, pad_byte=0):
    """metadata: list of (key, type, value) (arrays: value = (elem_type, items)); tensors: list of
    (name, torch_shape, ggml_type, data bytes). Returns the image bytes."""
    out = bytearray(struct.pack("<IIQQ", MAGIC, version, len(tensors), len(metadata)))
    for k, t, v in metadata:
        out += gstr(k) + struct.pack("<I", t) + value(t, v)
    offs, off = [], 0
    for _, _, _, data in tensors:
        offs.append(off)
        off += -(-len(data) // alignment) * alignment
    for (name, shape, gt, _), o in zip(tensors, offs):
        out += gstr(name) + struct.pack("<I", len(shape))
        for d in reversed(shape):
            out += struct.pack("<Q", d)
        out += struct.pack("<IQ", gt, o)
    while len(out) % alignment:
        out.append(pad_byte)
    for (_, _, _, data), o in zip(tensors, offs):
        out += bytes(data)
        while len(out) % alignment:
            out.append(pad_byte)
    return bytes(out)


def llama_image(cfg, exported, permute_qk=True):
    """A llama-architecture GGUF image of exported decode weights (LlamaWeights.export()): GGUF tensor
    names, q/k rows in llama.cpp's interleaved order (the inverse of the loader's un-permute), f32
    embedding and norms, Q4_K/Q6_K projection blocks as stored."""
    meta = [("general.architecture", T_STRING, "llama"),
            ("llama.block_count", T_UINT32, cfg.layers), ("llama.embedding_length", T_UINT32, cfg.hidden),
            ("llama.feed_forward_length", T_UINT32, cfg.ffn), ("llama.attention.head_count", T_UINT32, cfg.heads),
            ("llama.attention.head_count_kv", T_UINT32, cfg.kv_heads),
            ("llama.rope.freq_base", T_FLOAT32, cfg.rope_theta),
            ("llama.attention.layer_norm_rms_epsilon", T_FLOAT32, cfg.eps),
            ("llama.rope.scaling.type", T_STRING, "llama3"), ("llama.rope.scaling.factor", T_FLOAT32, cfg.rope_factor),
            ("llama.rope.scaling.low_freq_factor", T_FLOAT32, cfg.rope_low),
            ("llama.rope.scaling.high_freq_factor", T_FLOAT32, cfg.rope_high),
            ("llama.rope.scaling.original_context_length", T_UINT32, int(cfg.rope_orig_ctx))]
    gtype = {12: 12, 14: 14, 8: 8}
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate", "up": "ffn_up",
             "down": "ffn_down"}
    sh = cfg.shapes()
    tensors = [("token_embd.weight", (cfg.vocab, cfg.hidden), 0, exported["embed"].astype(np.float32).tobytes())]
    for li, lw in enumerate(exported["layers"]):
        tensors.append((f"blk.{li}.attn_norm.weight", (cfg.hidden,), 0, exported["attn_norm"][li].tobytes()))
        tensors.append((f"blk.{li}.ffn_norm.weight", (cfg.hidden,), 0, exported["ffn_norm"][li].tobytes()))
        for key, gname in names.items():
            n, k = sh[key]
            raw = np.asarray(lw[key], np.uint8)
            if permute_qk and key in ("q", "k"):
                nh = cfg.heads if key == "q" else cfg.kv_heads
                raw = permute_rows(raw.reshape(n, -1), nh).reshape(-1)
            tensors.append((f"blk.{li}.{gname}.weight", (n, k), gtype[int(cfg.dtypes[key])], raw.tobytes()))
    tensors.append(("output_norm.weight", (cfg.hidden,), 0, exported["final_norm"].tobytes()))
    n, k = sh["head"]
    tensors.append(("output.weight", (n, k), gtype[int(cfg.dtypes["head"])],
                    np.asarray(exported["head"], np.uint8).tobytes()))
    return build(meta, tensors)


def permute_rows(rows, n_head):
    """llama.cpp's convert step for q/k (the reference test's `forward`): GGUF row h*hd + 2j + k holds
    torch row h*hd + k*hd/2 + j."""
    n = rows.shape[0]
    hd = n // n_head
    half = hd // 2
    out = np.empty_like(rows)
    for h in range(n_head):
        for k in range(2):
            for j in range(half):
                out[h * hd + 2 * j + k] = rows[h * hd + k * half + j]
    return out
