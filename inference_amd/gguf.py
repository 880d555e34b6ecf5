"""GGUF files: the reference reader's API over the library's C++ parser, and resident loads.

`GgufFile` mirrors crates/llm/mlx-llm/src/gguf/reader.rs (GgufFile::open/parse,
metadata, tensors, alignment, meta/meta_str/meta_u64/meta_f64, tensor_data;
MetaValue::as_u64/as_i64/as_f64/as_str/as_bool/as_array; TensorInfo with the
torch-order shape), `Content` mirrors candle's gguf_file::Content as the
engine uses it (crates/llm/candle-llm/src/gguf.rs:68, 101-103: read, the
metadata and tensor-info tables, tensor(name, device) -> QTensor). The
difference is where a tensor lands: `Content.tensor` copies the quantized
blocks straight into a device QTensor (qmm_gguf_load_qtensor), where the
engine dequantizes and re-quantizes. `remap_key` and the q/k row un-permute
follow candle-llm gguf.rs:293-318 and :333-356.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Any, Dict, List, Optional

import numpy as np
import torch

from . import qmm
from .qmm import GgmlDType, QTensor

# GGUF metadata value types
T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY, T_UINT64, T_INT64, \
    T_FLOAT64 = range(13)
_UNSIGNED = (T_UINT8, T_UINT16, T_UINT32, T_UINT64)
_SIGNED = (T_INT8, T_INT16, T_INT32, T_INT64)

# GGML type tags of the formats a resident load takes
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4K, GGML_Q6K, GGML_BF16 = 0, 1, 8, 12, 14, 30


@dataclass(frozen=True)
class MetaValue:
    """A typed metadata value (reader.rs:44-71): `type` is the GGUF tag, `value` the Python value
    (int / float / bool / str, or a list of MetaValue for arrays)."""
    type: int
    value: Any

    def as_u64(self) -> Optional[int]:
        if self.type in _UNSIGNED:
            return int(self.value)
        if self.type in _SIGNED and self.value >= 0:
            return int(self.value)
        if self.type == T_BOOL:
            return int(self.value)
        return None

    def as_i64(self) -> Optional[int]:
        if self.type == T_UINT64:
            v = int(self.value)
            return v - (1 << 64) if v >= 1 << 63 else v  # `as i64` wraps
        return int(self.value) if self.type in _UNSIGNED + _SIGNED else None

    def as_f64(self) -> Optional[float]:
        return float(self.value) if self.type in (T_FLOAT32, T_FLOAT64) else None

    def as_str(self) -> Optional[str]:
        return self.value if self.type == T_STRING else None

    def as_bool(self) -> Optional[bool]:
        return bool(self.value) if self.type == T_BOOL else None

    def as_array(self) -> Optional[List["MetaValue"]]:
        return self.value if self.type == T_ARRAY else None


@dataclass(frozen=True)
class TensorInfo:
    """One tensor-info entry: name, torch-order shape ([out, in] for a linear weight), GGML type tag,
    offset within the data section, and its index in the file."""
    name: str
    shape: tuple
    ggml_type: int
    offset: int
    index: int

    def num_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


def type_size(ggml_type: int) -> tuple:
    """(elements, bytes) per block of a GGML type tag (dequant.rs:86-140)."""
    be, bb = ctypes.c_uint64(), ctypes.c_uint64()
    qmm._check(qmm.lib().qmm_gguf_type_size(ggml_type, ctypes.byref(be), ctypes.byref(bb)))
    return int(be.value), int(bb.value)


def tensor_byte_len(ggml_type: int, num_elements: int) -> int:
    """Bytes of a tensor's data (dequant.rs:144-153); raises for a partial block."""
    be, bb = type_size(ggml_type)
    if num_elements % be:
        raise qmm.QmmError(qmm.QMM_ERR_INVALID, f"gguf: {num_elements} elements not a multiple of {be}")
    return num_elements // be * bb


class GgufFile:
    """A parsed GGUF file (reader.rs GgufFile). Files are memory-mapped by the library; in-memory
    images are copied into it. Tensor data views stay valid while the object lives."""

    def __init__(self, handle: ctypes.c_void_p):
        self._h = handle
        L = qmm.lib()
        self.version = int(L.qmm_gguf_version(handle))
        self.alignment = int(L.qmm_gguf_alignment(handle))
        self.metadata: Dict[str, MetaValue] = {}
        for i in range(int(L.qmm_gguf_metadata_count(handle))):
            key, mv = self._meta(i)
            self.metadata[key] = mv
        self.tensors: List[TensorInfo] = [self._tensor(i) for i in range(int(L.qmm_gguf_tensor_count(handle)))]

    @classmethod
    def open(cls, path) -> "GgufFile":
        h = ctypes.c_void_p()
        qmm._check(qmm.lib().qmm_gguf_open(os.fsencode(path), ctypes.byref(h)))
        return cls(h)

    @classmethod
    def parse(cls, data: bytes) -> "GgufFile":
        h = ctypes.c_void_p()
        buf = bytes(data)
        qmm._check(qmm.lib().qmm_gguf_open_memory(buf, len(buf), ctypes.byref(h)))
        return cls(h)

    def close(self):
        if getattr(self, "_h", None):
            qmm.lib().qmm_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    # -- metadata ----------------------------------------------------------
    def _value(self, i: int, elem: int, t: int):
        L = qmm.lib()
        if t == T_STRING:
            p, n = ctypes.c_void_p(), ctypes.c_uint64()
            qmm._check(L.qmm_gguf_meta_string(self._h, i, elem, ctypes.byref(p), ctypes.byref(n)))
            return ctypes.string_at(p.value, n.value).decode("utf-8") if n.value else ""
        if t in (T_FLOAT32, T_FLOAT64):
            v = ctypes.c_double()
            qmm._check(L.qmm_gguf_meta_f64(self._h, i, elem, ctypes.byref(v)))
            return v.value
        if t == T_BOOL:
            v = ctypes.c_uint64()
            qmm._check(L.qmm_gguf_meta_u64(self._h, i, elem, ctypes.byref(v)))
            return bool(v.value)
        if t == T_UINT64:
            v = ctypes.c_uint64()
            qmm._check(L.qmm_gguf_meta_u64(self._h, i, elem, ctypes.byref(v)))
            return int(v.value)
        v = ctypes.c_int64()
        qmm._check(L.qmm_gguf_meta_i64(self._h, i, elem, ctypes.byref(v)))
        return int(v.value)

    def _meta(self, i: int):
        key, t, et, cnt = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int(), ctypes.c_uint64()
        qmm._check(qmm.lib().qmm_gguf_meta_info(self._h, i, ctypes.byref(key), ctypes.byref(t), ctypes.byref(et),
                                                ctypes.byref(cnt)))
        k = key.value.decode("utf-8")
        if t.value == T_ARRAY:
            return k, MetaValue(T_ARRAY, [MetaValue(et.value, self._value(i, e, et.value))
                                          for e in range(cnt.value)])
        return k, MetaValue(t.value, self._value(i, -1, t.value))

    def meta(self, key: str) -> Optional[MetaValue]:
        return self.metadata.get(key)

    def meta_str(self, key: str) -> Optional[str]:
        m = self.metadata.get(key)
        return m.as_str() if m is not None else None

    def meta_u64(self, key: str) -> Optional[int]:
        m = self.metadata.get(key)
        return m.as_u64() if m is not None else None

    def meta_f64(self, key: str) -> Optional[float]:
        m = self.metadata.get(key)
        return m.as_f64() if m is not None else None

    # -- tensors -----------------------------------------------------------
    def _tensor(self, i: int) -> TensorInfo:
        name, nd, ty, off = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int(), ctypes.c_uint64()
        shape = (ctypes.c_int64 * 4)()
        qmm._check(qmm.lib().qmm_gguf_tensor_info(self._h, i, ctypes.byref(name), ctypes.byref(nd), shape,
                                                  ctypes.byref(ty), ctypes.byref(off)))
        return TensorInfo(name.value.decode("utf-8"), tuple(int(shape[d]) for d in range(nd.value)), ty.value,
                          int(off.value), i)

    def tensor_data(self, info: TensorInfo) -> np.ndarray:
        """Read-only uint8 view of the tensor's bytes (bounds-checked against the file)."""
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        qmm._check(qmm.lib().qmm_gguf_tensor_data(self._h, info.index, ctypes.byref(p), ctypes.byref(n)))
        if n.value == 0:
            return np.zeros(0, np.uint8)
        buf = (ctypes.c_uint8 * n.value).from_address(p.value)
        buf._owner = self  # the mapping lives as long as any view of it
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def load_qtensor(self, info: TensorInfo, device: torch.device, unpermute_heads: int = 0) -> QTensor:
        """Resident load of a 2-D Q8_0 / Q4_K / Q6_K tensor into a device QTensor (blocks copied as is;
        unpermute_heads > 0 restores the half-split q/k row order of llama.cpp files)."""
        with torch.cuda.device(device):
            h = ctypes.c_void_p()
            qmm._check(qmm.lib().qmm_gguf_load_qtensor(self._h, info.index, unpermute_heads, qmm._stream(device),
                                                       ctypes.byref(h)))
        return QTensor(h, device)

    def load_dense(self, info: TensorInfo, device: torch.device) -> torch.Tensor:
        """F32 / F16 / BF16 tensor as f32 on the device; Q8_0 / Q4_K / Q6_K dequantized on the device."""
        if info.ggml_type in (GGML_Q8_0, GGML_Q4K, GGML_Q6K):
            qt = self.load_qtensor(info, device)
            return qt.dequantize().reshape(info.shape)
        raw = self.tensor_data(info)
        if info.ggml_type == GGML_F32:
            a = torch.from_numpy(raw.view(np.float32).copy())
        elif info.ggml_type == GGML_F16:
            a = torch.from_numpy(raw.view(np.float16).astype(np.float32))
        elif info.ggml_type == GGML_BF16:
            a = torch.from_numpy((raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32))
        else:
            raise qmm.QmmError(qmm.QMM_ERR_UNSUPPORTED, f"gguf: tensor {info.name!r} has type {info.ggml_type}")
        return a.reshape(info.shape).to(device)


class Content:
    """candle's gguf_file::Content as the engine uses it: read(), metadata, tensor_infos, tensor()."""

    def __init__(self, f: GgufFile):
        self.file = f
        self.metadata = f.metadata
        self.tensor_infos: Dict[str, TensorInfo] = {t.name: t for t in f.tensors}
        self.tensor_data_offset = None

    @classmethod
    def read(cls, path) -> "Content":
        return cls(GgufFile.open(path))

    def tensor(self, name: str, device: torch.device, unpermute_heads: int = 0) -> QTensor:
        info = self.tensor_infos.get(name)
        if info is None:
            raise qmm.QmmError(qmm.QMM_ERR_INVALID, f"gguf: no tensor {name!r}")
        return self.file.load_qtensor(info, device, unpermute_heads)


def remap_key(name: str) -> Optional[str]:
    """GGUF tensor name -> transformers key (candle-llm gguf.rs:293-318); None when unmapped."""
    fixed = {"token_embd.weight": "model.embed_tokens.weight", "output_norm.weight": "model.norm.weight",
             "output.weight": "lm_head.weight"}
    if name in fixed:
        return fixed[name]
    if not name.startswith("blk."):
        return None
    idx, dot, suffix = name[4:].partition(".")
    digits = idx[1:] if idx.startswith("+") else idx  # usize::from_str takes an optional '+'
    if not dot or not digits.isascii() or not digits.isdigit():
        return None
    hf = {"attn_q.weight": "self_attn.q_proj.weight", "attn_k.weight": "self_attn.k_proj.weight",
          "attn_v.weight": "self_attn.v_proj.weight", "attn_output.weight": "self_attn.o_proj.weight",
          "attn_norm.weight": "input_layernorm.weight", "ffn_norm.weight": "post_attention_layernorm.weight",
          "ffn_gate.weight": "mlp.gate_proj.weight", "ffn_up.weight": "mlp.up_proj.weight",
          "ffn_down.weight": "mlp.down_proj.weight", "attn_q_norm.weight": "self_attn.q_norm.weight",
          "attn_k_norm.weight": "self_attn.k_norm.weight"}.get(suffix)
    return f"model.layers.{idx}.{hf}" if hf else None


def is_ignorable(name: str) -> bool:
    """Tensors the engine recomputes and skips (gguf.rs:321-324): precomputed RoPE frequencies."""
    return name == "rope_freqs.weight" or name.endswith(".rope_freqs.weight")


def unpermute_rows(n_rows: int, n_head: int) -> np.ndarray:
    """Source row of each torch row for llama.cpp's q/k order (gguf.rs:346-353): torch row
    h * hd + k * hd/2 + j comes from GGUF row h * hd + 2j + k."""
    hd = n_rows // n_head
    half = hd // 2
    r = np.arange(hd)
    per = 2 * (r % half) + r // half
    return (np.arange(n_head)[:, None] * hd + per[None, :]).reshape(-1)
