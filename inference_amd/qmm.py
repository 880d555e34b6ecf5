"""Candle-shaped host API over the libqmm C ABI (include/qmm.h).

Mirrors the surface the reference engine uses for its quantized projections:

* ``GgmlDType``             -- candle ``quantized::GgmlDType`` (Q8_0, Q4K, Q6K; Q8K as vec-dot type)
* ``QTensor``               -- ``QTensor::{quantize, new(QStorage::from_data), dequantize, dtype}``
* ``QMatMul``               -- ``QMatMul::{from_qtensor, forward}``
* ``QuantSpec``             -- crates/llm/candle-llm/src/primitives/projection.rs:16-52
* ``QuantizedLinear``       -- crates/llm/candle-llm/src/primitives/quant.rs:17-43
* ``Projection``            -- crates/llm/candle-llm/src/primitives/projection.rs:56-95

Tensors are torch tensors on the GPU; torch only provides device memory and the
current stream. Every computation runs in the HIP kernels of ``libqmm.so``; if
that library is missing this module raises instead of falling back.
"""
from __future__ import annotations

import ctypes
import enum
import os
import threading
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libqmm.so")


class QmmError(RuntimeError):
    """An error reported by the C ABI (status code + message)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"qmm error {status}: {message}")
        self.status = status


# status codes of the C ABI (include/qmm.h)
QMM_OK, QMM_ERR_INVALID, QMM_ERR_HIP, QMM_ERR_NO_KERNEL, QMM_ERR_UNSUPPORTED, QMM_ERR_OOM = range(6)

_lib = None
_lib_lock = threading.Lock()

EXPORTS = (
    "qmm_last_error", "qmm_init", "qmm_block_size", "qmm_type_size", "qmm_vec_dot_type",
    "qmm_qtensor_from_ggml", "qmm_qtensor_quantize", "qmm_qtensor_dequantize",
    "qmm_qtensor_to_ggml", "qmm_qtensor_info", "qmm_qtensor_ggml_bytes", "qmm_qtensor_free",
    "qmm_quantize_rows", "qmm_matmul_workspace_size", "qmm_matmul", "qmm_matmul_q",
    "qmm_matmul_multi", "qmm_block_dots", "qmm_moe_route", "qmm_moe_gemv", "qmm_moe_gemm_workspace_size", "qmm_moe_gemm",
    "qmm_moe_ffn_workspace_size",
    "qmm_moe_ffn", "qmm_matmul_ex", "qmm_matmul_ex_workspace_size", "qmm_ffn", "qmm_ffn_workspace_size",
    "qmm_qkv_rope_kv_append_n", "qmm_qkv_rope_kv_append_n_workspace_size", "qmm_rms_norm", "qmm_embed_rows",
    "qmm_rope_kv_append", "qmm_decode_attention", "qmm_silu_mul_quantize", "qmm_greedy_advance",
    "qmm_matmul_q_ex", "qmm_decode_attention_workspace_size", "qmm_decode_rope_attention",
    "qmm_greedy_workspace_size", "qmm_matmul_multi_q", "qmm_silu_mul_matmul",
    "qmm_gguf_open", "qmm_gguf_open_memory", "qmm_gguf_close", "qmm_gguf_version", "qmm_gguf_alignment",
    "qmm_gguf_tensor_count", "qmm_gguf_metadata_count", "qmm_gguf_find_tensor", "qmm_gguf_meta_find",
    "qmm_gguf_tensor_info", "qmm_gguf_type_size", "qmm_gguf_tensor_data", "qmm_gguf_meta_info",
    "qmm_gguf_meta_u64", "qmm_gguf_meta_i64", "qmm_gguf_meta_f64", "qmm_gguf_meta_string",
    "qmm_gguf_load_qtensor", "qmm_qtensor_dequantize_to", "qmm_embed_rows_n", "qmm_rope_kv_append_n",
    "qmm_prefill_attention", "qmm_prefill_attention_o", "qmm_prefill_attention_o_workspace_size",
    "qmm_silu_mul", "qmm_matmul_q_workspace_size", "qmm_matmul_noalloc",
    "qmm_stream_read", "qmm_reload_tuning", "qmm_moe_route_ex", "qmm_moe_ffn_ex_workspace_size", "qmm_moe_ffn_ex",
    "qmm_decode_rope_attention_warm", "qmm_matmul_grouped",
)


def lib() -> ctypes.CDLL:
    """Load libqmm.so (built in-tree by ``__graft_entry__.build()``)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
        pp = ctypes.POINTER(ctypes.c_void_p)
        sig = {
            "qmm_last_error": ([], ctypes.c_char_p),
            "qmm_init": ([i32], i32),
            "qmm_reload_tuning": ([], None),
            "qmm_block_size": ([i32], i32),
            "qmm_type_size": ([i32], i32),
            "qmm_vec_dot_type": ([i32], i32),
            "qmm_qtensor_from_ggml": ([i32, i64, i64, vp, i32, vp, pp], i32),
            "qmm_qtensor_quantize": ([i32, i64, i64, vp, vp, pp], i32),
            "qmm_qtensor_dequantize": ([vp, vp, vp], i32),
            "qmm_qtensor_to_ggml": ([vp, vp, i32, vp], i32),
            "qmm_qtensor_info": ([vp, ctypes.POINTER(i32), ctypes.POINTER(i64), ctypes.POINTER(i64)], i32),
            "qmm_qtensor_ggml_bytes": ([vp], sz),
            "qmm_qtensor_free": ([vp], None),
            "qmm_quantize_rows": ([i32, vp, i64, i64, i64, vp, vp], i32),
            "qmm_matmul_workspace_size": ([vp, i64], sz),
            "qmm_matmul": ([vp, vp, i64, i64, vp, i64, vp, sz, vp], i32),
            "qmm_matmul_q": ([vp, vp, i64, vp, i64, vp, sz, vp], i32),
            "qmm_matmul_q_workspace_size": ([vp, i64], sz),
            "qmm_matmul_noalloc": ([vp, vp, i64, i64, vp, i64, vp], i32),
            "qmm_matmul_multi": ([ctypes.POINTER(vp), i32, vp, i64, i64, ctypes.POINTER(vp),
                                  ctypes.POINTER(i64), vp, sz, vp], i32),
            "qmm_block_dots": ([vp, vp, i64, vp, i64, vp, vp, sz, vp], i32),
            "qmm_moe_route": ([vp, i64, i32, i32, i32, vp, vp, vp, vp, vp, vp], i32),
            "qmm_moe_gemv": ([ctypes.POINTER(vp), i32, i32, vp, i64, vp, vp, ctypes.POINTER(vp), vp], i32),
            "qmm_moe_gemm_workspace_size": ([vp, i64], ctypes.c_size_t),
            "qmm_moe_gemm": ([ctypes.POINTER(vp), i32, i32, vp, i64, i64, i64, vp, vp, ctypes.POINTER(vp), vp,
                              ctypes.c_size_t, vp], i32),
            "qmm_moe_ffn_workspace_size": ([vp, vp, i64, i32, i32], sz),
            "qmm_moe_ffn": ([vp, i64, i64, vp, i32, i32, vp, vp, vp, vp, i64, vp, sz, vp], i32),
            "qmm_moe_route_ex": ([vp, i64, i32, i32, i32, ctypes.c_float, vp, vp, vp, vp, vp, vp], i32),
            "qmm_moe_ffn_ex_workspace_size": ([vp, vp, i64, i32, i32, vp, vp, vp], sz),
            "qmm_moe_ffn_ex": ([vp, i64, i64, vp, i32, i32, i32, ctypes.c_float, vp, vp, vp, vp, vp, vp, vp, vp, i64,
                                vp, sz, vp], i32),
            "qmm_matmul_ex": ([ctypes.POINTER(vp), i32, vp, i64, i64, vp, ctypes.c_float, i32, ctypes.POINTER(vp),
                               ctypes.POINTER(i64), vp, sz, vp], i32),
            "qmm_matmul_ex_workspace_size": ([vp, i64, i32], sz),
            "qmm_ffn": ([vp, vp, vp, vp, i64, i64, vp, ctypes.c_float, i32, vp, i64, vp, sz, vp], i32),
            "qmm_ffn_workspace_size": ([vp, vp, vp, i64, i32], sz),
            "qmm_qkv_rope_kv_append_n": ([vp, vp, vp, vp, i64, i64, vp, ctypes.c_float, vp, vp, i64, vp, i64, vp, vp,
                                          i32, i32, i32, i32, vp, sz, vp], i32),
            "qmm_qkv_rope_kv_append_n_workspace_size": ([vp, vp, vp, i64, i32], sz),
            "qmm_rms_norm": ([vp, i64, i64, i64, vp, ctypes.c_float, vp, i64, vp], i32),
            "qmm_embed_rows": ([vp, i64, i64, vp, vp, vp, i64, vp], i32),
            "qmm_rope_kv_append": ([vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp], i32),
            "qmm_decode_attention": ([vp, vp, vp, vp, vp, i32, i32, i32, i32, ctypes.c_float, vp, sz, vp], i32),
            "qmm_decode_rope_attention": ([vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, ctypes.c_float,
                                           vp, sz, vp], i32),
            "qmm_matmul_grouped": ([vp, vp, i32, vp, vp, vp], i32),
            "qmm_decode_rope_attention_warm": ([vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32,
                                                ctypes.c_float, vp, sz, vp, vp, i32, vp, vp], i32),
            "qmm_decode_attention_workspace_size": ([i32, i32, i32, i32], sz),
            "qmm_greedy_workspace_size": ([i64], sz),
            "qmm_silu_mul_quantize": ([vp, vp, i64, i64, i64, vp, vp], i32),
            "qmm_greedy_advance": ([vp, i64, vp, i64, vp, i32, vp, sz, vp], i32),
            "qmm_matmul_q_ex": ([vp, vp, i64, vp, i64, i32, vp, sz, vp], i32),
            "qmm_silu_mul_matmul": ([vp, vp, vp, vp, i32, vp], i32),
            "qmm_matmul_multi_q": ([ctypes.POINTER(vp), i32, vp, i64, ctypes.POINTER(vp), ctypes.POINTER(i64), vp,
                                    sz, vp], i32),
            "qmm_gguf_open": ([ctypes.c_char_p, pp], i32),
            "qmm_gguf_open_memory": ([ctypes.c_char_p, sz, pp], i32),
            "qmm_gguf_close": ([vp], None),
            "qmm_gguf_version": ([vp], i32),
            "qmm_gguf_alignment": ([vp], ctypes.c_uint64),
            "qmm_gguf_tensor_count": ([vp], i64),
            "qmm_gguf_metadata_count": ([vp], i64),
            "qmm_gguf_find_tensor": ([vp, ctypes.c_char_p], i64),
            "qmm_gguf_meta_find": ([vp, ctypes.c_char_p], i64),
            "qmm_gguf_tensor_info": ([vp, i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(i32),
                                      ctypes.POINTER(i64), ctypes.POINTER(i32), ctypes.POINTER(ctypes.c_uint64)], i32),
            "qmm_gguf_type_size": ([i32, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)], i32),
            "qmm_gguf_tensor_data": ([vp, i64, pp, ctypes.POINTER(sz)], i32),
            "qmm_gguf_meta_info": ([vp, i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(i32), ctypes.POINTER(i32),
                                    ctypes.POINTER(ctypes.c_uint64)], i32),
            "qmm_gguf_meta_u64": ([vp, i64, i64, ctypes.POINTER(ctypes.c_uint64)], i32),
            "qmm_gguf_meta_i64": ([vp, i64, i64, ctypes.POINTER(i64)], i32),
            "qmm_gguf_meta_f64": ([vp, i64, i64, ctypes.POINTER(ctypes.c_double)], i32),
            "qmm_gguf_meta_string": ([vp, i64, i64, pp, ctypes.POINTER(ctypes.c_uint64)], i32),
            "qmm_gguf_load_qtensor": ([vp, i64, i32, vp, pp], i32),
            "qmm_qtensor_dequantize_to": ([vp, vp, i32, vp], i32),
            "qmm_embed_rows_n": ([vp, i64, i64, vp, i64, i64, vp, i64, vp], i32),
            "qmm_rope_kv_append_n": ([vp, vp, vp, i64, i64, i64, vp, vp, i64, i64, vp, vp, i32, i32, i32, i32, vp],
                                     i32),
            "qmm_prefill_attention": ([vp, i64, vp, vp, i64, i64, vp, i64, i32, i32, i32, i32, ctypes.c_float, vp],
                                      i32),
            "qmm_prefill_attention_o": ([vp, i64, vp, vp, i64, i64, i32, i32, i32, i32, ctypes.c_float, vp, vp, i64, vp,
                                         sz, vp], i32),
            "qmm_prefill_attention_o_workspace_size": ([vp, i64], sz),
            "qmm_silu_mul": ([vp, vp, vp, i64, vp], i32),
            "qmm_stream_read": ([vp, ctypes.c_size_t, vp, i32, i32, vp], i32),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def last_error() -> str:
    """The calling thread's last error message from the library."""
    return lib().qmm_last_error().decode(errors="replace")


def _check(status: int) -> None:
    if status != 0:
        raise QmmError(status, last_error())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class GgmlDType(enum.IntEnum):
    """GGML block types of the quantized path (GGUF numbering)."""

    Q8_0 = 8
    Q4K = 12
    Q6K = 14
    Q8K = 15

    def block_size(self) -> int:
        return lib().qmm_block_size(int(self))

    def type_size(self) -> int:
        return lib().qmm_type_size(int(self))

    def vec_dot_type(self) -> "GgmlDType":
        v = lib().qmm_vec_dot_type(int(self))
        if v < 0:
            raise QmmError(1, f"{self.name} has no vec-dot type")
        return GgmlDType(v)


def _device_of(t: torch.Tensor) -> torch.device:
    if t.device.type != "cuda":
        raise QmmError(1, f"tensor must be on a GPU, got {t.device}")
    return t.device


def quantize_rows(vdtype: GgmlDType, x: torch.Tensor) -> torch.Tensor:
    """VecDotType::from_float on the GPU: f32 [m, k] -> uint8 [m, row_bytes] GGML blocks."""
    dev = _device_of(x)
    if x.dtype != torch.float32 or x.dim() != 2:
        raise QmmError(1, "quantize_rows expects a 2-D float32 tensor")
    if x.stride(1) != 1:
        x = x.contiguous()
    vdtype = GgmlDType(vdtype)
    m, k = x.shape
    if k % vdtype.block_size():
        raise QmmError(1, f"k = {k} is not a multiple of {vdtype.name}'s block size {vdtype.block_size()}")
    out = torch.empty((m, k // vdtype.block_size() * vdtype.type_size()), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _check(lib().qmm_quantize_rows(int(vdtype), x.data_ptr(), m, k, x.stride(0), out.data_ptr(),
                                       _stream(dev)))
    return out


class QTensor:
    """A GGML block-quantized [n, k] weight resident on one GPU."""

    def __init__(self, handle: ctypes.c_void_p, device: torch.device):
        self._h = handle
        self.device = device
        dt, n, k = ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64()
        _check(lib().qmm_qtensor_info(handle, ctypes.byref(dt), ctypes.byref(n), ctypes.byref(k)))
        self._dtype = GgmlDType(dt.value)
        self.shape: Tuple[int, int] = (n.value, k.value)

    # -- constructors ---------------------------------------------------
    @classmethod
    def quantize(cls, tensor: torch.Tensor, dtype: GgmlDType) -> "QTensor":
        """QTensor::quantize of a dense [n, k] weight, computed on the tensor's GPU."""
        dtype = GgmlDType(dtype)
        if dtype == GgmlDType.Q8K:
            raise QmmError(1, "Q8K is an activation-only type")
        dev = _device_of(tensor)
        if tensor.dim() != 2:
            raise QmmError(1, f"QTensor::quantize expects a 2-D weight, got shape {tuple(tensor.shape)}")
        n, k = tensor.shape
        if k % dtype.block_size():
            raise QmmError(1, f"quantize: the last dim {k} is not a multiple of {dtype.name}'s block size "
                              f"{dtype.block_size()}")
        w = tensor.to(torch.float32).contiguous()
        h = ctypes.c_void_p()
        with torch.cuda.device(dev):
            _check(lib().qmm_qtensor_quantize(int(dtype), n, k, w.data_ptr(), _stream(dev), ctypes.byref(h)))
        return cls(h, dev)

    @classmethod
    def quantize_onto(cls, tensor: torch.Tensor, dtype: GgmlDType, device: torch.device) -> "QTensor":
        """QTensor::quantize_onto (candle-gen/src/quant/mod.rs:693-728): a host, contiguous, zero-offset
        f32 source quantized straight into a QTensor on `device` (here: copied up, then quantized there).
        Any other source is an error, as in the reference."""
        if tensor.device.type != "cpu":
            raise QmmError(1, f"quantize_onto expects a CPU source tensor, got {tensor.device}")
        if not tensor.is_contiguous() or tensor.storage_offset() != 0:
            raise QmmError(1, "quantize_onto expects a contiguous source with zero offset")
        dev = torch.device(device)
        if dev.type != "cuda":
            raise QmmError(1, f"quantize_onto targets a GPU device, got {dev}")
        return cls.quantize(tensor.to(dev), dtype)

    @classmethod
    def from_ggml(cls, data, dtype: GgmlDType, shape: Sequence[int],
                  device: Optional[torch.device] = None) -> "QTensor":
        """QTensor::new(QStorage::from_data(GGML bytes), shape).

        ``data`` is bytes / a uint8 numpy array (host) or a uint8 torch tensor (host or GPU)."""
        dtype = GgmlDType(dtype)
        n, k = int(shape[0]), int(shape[1])
        on_dev = 0
        keep = None
        if isinstance(data, torch.Tensor):
            t = data.contiguous().view(torch.uint8)
            if t.device.type == "cuda":
                device = t.device
                on_dev = 1
            keep = t
            ptr = t.data_ptr()
            nbytes = t.numel()
        else:
            arr = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray))
                                       else data, dtype=np.uint8)
            keep = arr
            ptr = arr.ctypes.data
            nbytes = arr.size
        if dtype == GgmlDType.Q8K:
            raise QmmError(1, "Q8K is an activation-only type")
        if k % dtype.block_size():
            raise QmmError(1, f"k = {k} is not a multiple of {dtype.name}'s block size {dtype.block_size()}")
        expect = n * (k // dtype.block_size()) * dtype.type_size()
        if nbytes != expect:
            raise QmmError(1, f"{dtype.name} [{n}, {k}] needs {expect} bytes, got {nbytes}")
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        h = ctypes.c_void_p()
        with torch.cuda.device(device):
            _check(lib().qmm_qtensor_from_ggml(int(dtype), n, k, ptr, on_dev, _stream(device), ctypes.byref(h)))
        del keep
        return cls(h, device)

    # -- accessors ------------------------------------------------------
    def dtype(self) -> GgmlDType:
        return self._dtype

    def storage_size_in_bytes(self) -> int:
        return int(lib().qmm_qtensor_ggml_bytes(self._h))

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """QTensor::dequantize -> [n, k] on the tensor's GPU: f32, or f16 / bf16 rounded once from it
        (QTensor::dequantize_f16; the dequant-dense strategy's to_dtype)."""
        tag = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 30}.get(dtype)
        if tag is None:
            raise QmmError(1, f"dequantize to {dtype}: float32, float16 or bfloat16")
        out = torch.empty(self.shape, dtype=dtype, device=self.device)
        with torch.cuda.device(self.device):
            _check(lib().qmm_qtensor_dequantize_to(self._h, out.data_ptr(), tag, _stream(self.device)))
        return out

    def dequantize_f16(self) -> torch.Tensor:
        return self.dequantize(torch.float16)

    def to_ggml(self) -> np.ndarray:
        """GGML block bytes of the tensor (host, uint8)."""
        out = np.empty(self.storage_size_in_bytes(), dtype=np.uint8)
        with torch.cuda.device(self.device):
            _check(lib().qmm_qtensor_to_ggml(self._h, out.ctypes.data, 0, _stream(self.device)))
        return out

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and _lib is not None:
            _lib.qmm_qtensor_free(h)
            self._h = None


class QMatMul:
    """QMatMul over a QTensor: ``forward(x) = x @ dequant(W)^T`` with x quantized to the vec-dot type."""

    def __init__(self, qtensor: QTensor):
        self.qtensor = qtensor

    @classmethod
    def from_qtensor(cls, qtensor: QTensor) -> "QMatMul":
        return cls(qtensor)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        n, k = self.qtensor.shape
        if x.dtype != torch.float32:
            raise QmmError(1, f"QMatMul::forward expects float32 input, got {x.dtype}")
        if x.shape[-1] != k:
            raise QmmError(1, f"shape mismatch: input last dim {x.shape[-1]} vs weight in-dim {k}")
        if x.device != self.qtensor.device:
            raise QmmError(1, f"input on {x.device}, weight on {self.qtensor.device}")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, k)
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        m = x2.shape[0]
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
        if m == 0:
            return y.reshape(*lead, n)
        L = lib()
        ws_bytes = int(L.qmm_matmul_workspace_size(self.qtensor.handle, m))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
        with torch.cuda.device(x.device):
            _check(L.qmm_matmul(self.qtensor.handle, x2.data_ptr(), m, x2.stride(0), y.data_ptr(), n,
                                ws.data_ptr(), ws_bytes, _stream(x.device)))
        return y.reshape(*lead, n)

    def forward_via_f16(self, x: torch.Tensor) -> torch.Tensor:
        """QMatMul::forward_via_f16: the weight dequantized to a dense f16 tile, x cast to f16, a dense
        matmul (a plain library GEMM), the result cast back to x's dtype
        (candle-gen-lens/src/text_encoder.rs:518-529)."""
        n, k = self.qtensor.shape
        if x.shape[-1] != k:
            raise QmmError(1, f"shape mismatch: input last dim {x.shape[-1]} vs weight in-dim {k}")
        w = self.qtensor.dequantize(torch.float16)
        return torch.matmul(x.to(torch.float16), w.t()).to(x.dtype)

    __call__ = forward


class MatmulStrategy(enum.Enum):
    """How a quantized QLinear computes x @ W^T (candle-gen/src/quant/mod.rs:202-227)."""
    DEQUANT_DENSE = "dequant_dense"  # weight dequantized to x's dtype, dense matmul (outlier-safe)
    INT8_FAST = "int8_fast"          # QMatMul::forward: activation quantized to Q8_K / Q8_0


class QLinear:
    """Quantized linear of the media models (candle-gen/src/quant/mod.rs:515-568): x @ W^T (+ b) over a
    QTensor with either strategy. DEQUANT_DENSE keeps the activation full precision (the weight is
    dequantized per call, the QTensor stays resident); INT8_FAST flattens the leading dims, runs the
    f32 activation through QMatMul::forward and casts back to x's dtype."""

    def __init__(self, weight: QTensor, bias: Optional[torch.Tensor] = None,
                 strategy: MatmulStrategy = MatmulStrategy.DEQUANT_DENSE):
        self.weight, self.bias, self.strategy = weight, bias, strategy
        self._mm = QMatMul(weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.strategy == MatmulStrategy.DEQUANT_DENSE:
            w = self.weight.dequantize(torch.float32).to(x.dtype)
            b = self.bias.to(x.dtype) if self.bias is not None else None
            return torch.nn.functional.linear(x, w, b)
        y = self._mm.forward(x.to(torch.float32).contiguous())
        if self.bias is not None:
            y = y + self.bias
        return y.to(x.dtype)

    __call__ = forward


def matmul_multi(qts: Sequence[QTensor], x: torch.Tensor) -> Tuple[torch.Tensor, ...]:
    """Several QMatMul::forward on one input (same dtype and k) in one launch."""
    if not 1 <= len(qts) <= 8:
        raise QmmError(1, "matmul_multi takes 1..8 weights")
    k = qts[0].shape[1]
    if x.dtype != torch.float32 or x.shape[-1] != k:
        raise QmmError(1, "matmul_multi expects float32 input with last dim k")
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    m = x2.shape[0]
    ys = [torch.empty((m, q.shape[0]), dtype=torch.float32, device=x.device) for q in qts]
    L = lib()
    ws_bytes = max(int(L.qmm_matmul_workspace_size(q.handle, m)) for q in qts)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    hs = (ctypes.c_void_p * len(qts))(*[q.handle.value for q in qts])
    yp = (ctypes.c_void_p * len(qts))(*[y.data_ptr() for y in ys])
    ld = (ctypes.c_int64 * len(qts))(*[q.shape[0] for q in qts])
    with torch.cuda.device(x.device):
        _check(L.qmm_matmul_multi(hs, len(qts), x2.data_ptr(), m, x2.stride(0), yp, ld, ws.data_ptr(),
                                  ws_bytes, _stream(x.device)))
    return tuple(y.reshape(*x.shape[:-1], y.shape[1]) for y in ys)


def matmul_grouped(pairs: Sequence[Tuple[QTensor, int]], xs: Sequence[torch.Tensor],
                   outs: Optional[Sequence[torch.Tensor]] = None) -> Tuple[torch.Tensor, ...]:
    """QMatMul::forward of each (weight, group) pair on the single f32 row xs[group], all in one launch
    (qmm_matmul_grouped: up to 8 weights per group, two groups, one k-quant dtype); same bits as one
    QMatMul::forward per weight."""
    if not 1 <= len(pairs) <= 16 or not 1 <= len(xs) <= 2:
        raise QmmError(1, "matmul_grouped takes 1..16 weights over one or two rows")
    rows = []
    for x in xs:
        if x.dtype != torch.float32 or x.numel() != x.shape[-1]:
            raise QmmError(1, "matmul_grouped expects one float32 row per group")
        rows.append(x.reshape(-1).contiguous())
    dev = rows[0].device
    ys = list(outs) if outs is not None else [torch.empty(q.shape[0], dtype=torch.float32, device=dev)
                                              for q, _ in pairs]
    L = lib()
    hs = (ctypes.c_void_p * len(pairs))(*[q.handle.value for q, _ in pairs])
    gp = (ctypes.c_int * len(pairs))(*[int(g) for _, g in pairs])
    xp = (ctypes.c_void_p * 2)(*[r.data_ptr() for r in rows] + [None] * (2 - len(rows)))
    yp = (ctypes.c_void_p * len(pairs))(*[y.data_ptr() for y in ys])
    with torch.cuda.device(dev):
        _check(L.qmm_matmul_grouped(hs, gp, len(pairs), xp, yp, _stream(dev)))
    return tuple(ys)


def q_workspace(qts: Sequence[QTensor], m: int) -> Tuple[Optional[torch.Tensor], int]:
    """A device workspace for the pre-quantized entry points (None when m <= 8)."""
    L = lib()
    nbytes = max(int(L.qmm_matmul_q_workspace_size(q.handle, m)) for q in qts)
    if nbytes == 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=qts[0].device), nbytes


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def matmul_q(qt: QTensor, xq: torch.Tensor, m: int, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y[m, n] from pre-quantized activations (uint8 GGML vec-dot blocks on the GPU)."""
    n = qt.shape[0]
    y = out if out is not None else torch.empty((m, n), dtype=torch.float32, device=qt.device)
    ws, nbytes = q_workspace([qt], m)
    with torch.cuda.device(qt.device):
        _check(lib().qmm_matmul_q(qt.handle, xq.data_ptr(), m, y.data_ptr(), y.stride(0), _ptr(ws), nbytes,
                                  _stream(qt.device)))
    return y


def block_dots(qt: QTensor, xq: torch.Tensor, m: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Exact int32 block dots [m, n, nb(, 2)] and the f32 outputs of the same GEMV launch."""
    n, k = qt.shape
    nb = k // qt.dtype().block_size()
    per = 2 if qt.dtype() == GgmlDType.Q4K else 1
    dots = torch.zeros((m, n, nb, per), dtype=torch.int32, device=qt.device)
    y = torch.empty((m, n), dtype=torch.float32, device=qt.device)
    ws, nbytes = q_workspace([qt], m)
    with torch.cuda.device(qt.device):
        _check(lib().qmm_block_dots(qt.handle, xq.data_ptr(), m, y.data_ptr(), n, dots.data_ptr(), _ptr(ws), nbytes,
                                    _stream(qt.device)))
    return (dots if per == 2 else dots[..., 0]), y


def moe_route(logits: torch.Tensor, topk: int, renormalize: bool = True, routed_scaling_factor: float = 1.0):
    """Device routing: returns (counts, offsets, pair_token, pair_weight, token_pairs). Weights are the
    selected probabilities renormalised over the selection, or (renormalize False) times
    routed_scaling_factor (MoeMlp::forward, models/llama.rs:1436-1447)."""
    t, e = logits.shape
    dev = logits.device
    lg = logits.to(torch.float32).contiguous()
    counts = torch.empty(e, dtype=torch.int32, device=dev)
    offsets = torch.empty(e + 1, dtype=torch.int32, device=dev)
    ptok = torch.empty(t * topk, dtype=torch.int32, device=dev)
    pw = torch.empty(t * topk, dtype=torch.float32, device=dev)
    tp = torch.empty(t * topk, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        _check(lib().qmm_moe_route_ex(lg.data_ptr(), t, e, topk, int(renormalize), routed_scaling_factor,
                                      counts.data_ptr(), offsets.data_ptr(), ptok.data_ptr(), pw.data_ptr(),
                                      tp.data_ptr(), _stream(dev)))
    return counts, offsets, ptok, pw, tp


def moe_ffn(x: torch.Tensor, logits: torch.Tensor, gate: QTensor, up: QTensor, down: QTensor, topk: int,
            norm_topk_prob: bool = True, routed_scaling_factor: float = 1.0, shared=None,
            shared_gate: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Mixture-of-experts FFN (MoeMlp::forward, models/llama.rs:1416-1487) on stacked expert weights:
    top-k routing (renormalised, or scaled by routed_scaling_factor), each expert's gated MLP on its
    tokens, the weighted outputs summed in expert order; then `shared` = (gate, up, down) QTensors of the
    always-on shared expert, added after the routed sum, scaled per token by sigmoid(x . shared_gate)
    when shared_gate (f32 [hidden]) is given."""
    t, hdim = x.shape
    e = logits.shape[1]
    dev = x.device
    xx = x.to(torch.float32).contiguous()
    lg = logits.to(torch.float32).contiguous()
    out = torch.empty((t, hdim), dtype=torch.float32, device=dev)
    L = lib()
    sg, su, sd = (s.handle for s in shared) if shared is not None else (None, None, None)
    if shared is None and shared_gate is not None:
        raise QmmError(QMM_ERR_INVALID, "a shared-expert gate without a shared expert")
    gw = shared_gate.to(torch.float32).contiguous() if shared_gate is not None else None
    with torch.cuda.device(dev):
        wsb = int(L.qmm_moe_ffn_ex_workspace_size(gate.handle, down.handle, t, e, topk, sg, su, sd))
        if wsb == 0:
            raise QmmError(QMM_ERR_INVALID, "moe_ffn: " + last_error())
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        _check(L.qmm_moe_ffn_ex(xx.data_ptr(), t, hdim, lg.data_ptr(), e, topk, int(norm_topk_prob),
                                routed_scaling_factor, gate.handle, up.handle, down.handle, sg, su, sd,
                                gw.data_ptr() if gw is not None else None, out.data_ptr(), hdim, ws.data_ptr(), wsb,
                                _stream(dev)))
    return out


# ---------------------------------------------------------------------------
# engine-level wrappers (crates/llm/candle-llm/src/primitives/{projection,quant}.rs)
# ---------------------------------------------------------------------------

class QuantSpec:
    """Group-wise quantization spec: 4 bits -> Q4_K, 8 bits -> Q8_0 (projection.rs:16-52)."""

    def __init__(self, dtype: GgmlDType):
        self.dtype = GgmlDType(dtype)

    @classmethod
    def q4(cls) -> "QuantSpec":
        return cls(GgmlDType.Q4K)

    @classmethod
    def q8(cls) -> "QuantSpec":
        return cls(GgmlDType.Q8_0)

    @classmethod
    def from_bits(cls, bits: int) -> Optional["QuantSpec"]:
        if bits == 4:
            return cls.q4()
        if bits == 8:
            return cls.q8()
        return None

    def bits(self) -> int:
        return 8 if self.dtype == GgmlDType.Q8_0 else 4

    def __eq__(self, other) -> bool:
        return isinstance(other, QuantSpec) and other.dtype == self.dtype

    def __repr__(self) -> str:
        return f"QuantSpec({self.dtype.name})"


class QuantizedLinear:
    """A linear projection with a GGML block-quantized weight (quant.rs:17-43)."""

    def __init__(self, inner: QMatMul, bias: Optional[torch.Tensor]):
        self.inner = inner
        self.bias = bias

    @classmethod
    def quantize(cls, weight: torch.Tensor, dtype: GgmlDType, bias: Optional[torch.Tensor] = None) -> "QuantizedLinear":
        qt = QTensor.quantize(weight.to(torch.float32), dtype)
        return cls(QMatMul.from_qtensor(qt), bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = self.inner.forward(x.to(torch.float32)).to(x.dtype)
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        return y

    __call__ = forward


class Projection:
    """A projection weight that is dense or quantized (projection.rs:56-95)."""

    def __init__(self, dense_weight: Optional[torch.Tensor] = None, dense_bias: Optional[torch.Tensor] = None,
                 quantized: Optional[QuantizedLinear] = None):
        self._w = dense_weight
        self._b = dense_bias
        self._q = quantized

    @classmethod
    def load(cls, weight: torch.Tensor, quant: Optional[QuantSpec]) -> "Projection":
        return cls.load_with_bias(weight, None, quant)

    @classmethod
    def load_with_bias(cls, weight: torch.Tensor, bias: Optional[torch.Tensor],
                       quant: Optional[QuantSpec]) -> "Projection":
        if quant is None:
            return cls(dense_weight=weight, dense_bias=bias)
        return cls(quantized=QuantizedLinear.quantize(weight, quant.dtype, bias))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._q is not None:
            return self._q.forward(x)
        return torch.nn.functional.linear(x, self._w, self._b)

    __call__ = forward

    def is_quantized(self) -> bool:
        return self._q is not None
