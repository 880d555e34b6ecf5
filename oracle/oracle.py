"""ctypes wrapper around the C oracle (``oracle/ggml_oracle.c``).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this module; the product
package never does.  Arrays are numpy; block buffers are GGML bytes (uint8).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libggml_oracle.so")

F32, F16, Q8_0, Q4K, Q6K, Q8K = 0, 1, 8, 12, 14, 15
_ELEMS = {Q8_0: 32, Q4K: 256, Q6K: 256, Q8K: 256}
_BYTES = {Q8_0: 34, Q4K: 144, Q6K: 210, Q8K: 292}
VEC_DOT_TYPE = {Q8_0: Q8_0, Q4K: Q8K, Q6K: Q8K}
# vec_dot bodies: candle's generic ones (the reference's default build) or its AVX2 + FMA ones
GENERIC, AVX2 = 0, 1

_lib = None


def build() -> None:
    """Compile the oracle with its Makefile (gcc, no reference sources)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_quantize.argtypes = [i32, vp, i64, vp]
        L.orc_dequantize.argtypes = [i32, vp, i64, vp]
        L.orc_vec_dot.argtypes = [i32, i64, vp, vp]
        L.orc_vec_dot.restype = ctypes.c_float
        L.orc_block_dots.argtypes = [i32, i64, vp, vp, vp]
        L.orc_matmul.argtypes = [i32, i64, i64, i64, vp, vp, vp, i32]
        L.orc_matmul_prequant.argtypes = [i32, i64, i64, i64, vp, vp, vp, i32]
        L.orc_matmul_impl.argtypes = [i32, i64, i64, i64, vp, vp, vp, i32, i32]
        L.orc_matmul_prequant_impl.argtypes = [i32, i64, i64, i64, vp, vp, vp, i32, i32]
        L.orc_vec_dot_avx2.argtypes = [i32, i64, vp, vp]
        L.orc_vec_dot_avx2.restype = ctypes.c_float
        L.orc_make_qkx1_quants.argtypes = [i32, i32, vp, i32, vp, vp]
        L.orc_make_qkx1_quants.restype = None
        L.orc_make_qx_quants.argtypes = [i32, i32, vp, vp, i32]
        L.orc_make_qx_quants.restype = ctypes.c_float
        L.orc_make_qx_quants_first.argtypes = [i32, i32, vp, vp, vp]
        L.orc_make_qx_quants_first.restype = ctypes.c_float
        for f in ("orc_block_elems", "orc_block_bytes", "orc_vec_dot_type"):
            getattr(L, f).argtypes = [i32]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def block_elems(dt: int) -> int:
    return _ELEMS[dt]


def block_bytes(dt: int) -> int:
    return _BYTES[dt]


def row_bytes(dt: int, k: int) -> int:
    """GGML bytes of a row of k elements; k must be a whole number of blocks (the C routines
    process every element they are given, so a partial block would run past the buffer)."""
    if k <= 0 or k % _ELEMS[dt]:
        raise ValueError(f"row length {k} is not a whole number of {_ELEMS[dt]}-element blocks (dtype {dt})")
    return k // _ELEMS[dt] * _BYTES[dt]


def f32_to_f16_bits(x: float) -> int:
    return lib().orc_f32_to_f16(float(x))


def f16_bits_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(int(h))


def make_qkx1_quants(x: np.ndarray, nmax: int = 15, ntry: int = 5):
    """The Q4_K sub-block fit (quantized/utils.rs make_qkx1_quants): (scale, -min) of x."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    sc, mn = np.zeros(1, np.float32), np.zeros(1, np.float32)
    lib().orc_make_qkx1_quants(nmax, ntry, _ptr(x), x.size, _ptr(sc), _ptr(mn))
    return float(sc[0]), float(mn[0])


def make_qx_quants(x: np.ndarray, nmax: int = 32, rmse_type: int = 1):
    """The Q6_K sub-block fit (quantized/utils.rs make_qx_quants): (scale, l) with l in [-nmax, nmax).
    rmse_type 0 (bare rounding) and 1 (x^2-weighted refinement, the one BlockQ6K uses) are restated."""
    if rmse_type not in (0, 1):
        raise ValueError(f"make_qx_quants: rmse_type {rmse_type} is not restated (0 and 1 are)")
    x = np.ascontiguousarray(x, dtype=np.float32)
    L = np.zeros(x.size, np.int8)
    s = lib().orc_make_qx_quants(x.size, nmax, _ptr(x), _ptr(L), rmse_type)
    return float(s), L.astype(np.int32) - nmax


def make_qx_quants_first(x: np.ndarray, nmax: int = 32):
    """make_qx_quants (rmse_type 1) stopped after its first refinement loop: (scale, l, accepted passes)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    L = np.zeros(x.size, np.int8)
    passes = np.zeros(1, np.int32)
    s = lib().orc_make_qx_quants_first(x.size, nmax, _ptr(x), _ptr(L), _ptr(passes))
    return float(s), L.astype(np.int32) - nmax, int(passes[0])


def quantize(dt: int, x: np.ndarray) -> np.ndarray:
    """from_float of a row-major f32 array; returns GGML bytes, shape [rows, row_bytes]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    rows = x.size // k
    out = np.zeros((rows, row_bytes(dt, k)), dtype=np.uint8)
    rc = lib().orc_quantize(dt, _ptr(x), x.size, _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle quantize failed for dtype {dt}, shape {x.shape}")
    return out


def dequantize(dt: int, blocks: np.ndarray, n_elems: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_elems, dtype=np.float32)
    rc = lib().orc_dequantize(dt, _ptr(blocks), n_elems, _ptr(out))
    if rc != 0:
        raise ValueError("oracle dequantize failed")
    return out


def vec_dot(dt: int, k: int, w_row: np.ndarray, x_row: np.ndarray) -> float:
    return lib().orc_vec_dot(dt, k, _ptr(np.ascontiguousarray(w_row)), _ptr(np.ascontiguousarray(x_row)))


def block_dots(dt: int, w: np.ndarray, xq: np.ndarray, k: int) -> np.ndarray:
    """Integer block dots for every (token m, weight row n).

    Returns int32 [m, n, nb] (Q8_0, Q6_K) or [m, n, nb, 2] (Q4_K: isum_d, isum_m)."""
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, row_bytes(dt, k))
    vt = VEC_DOT_TYPE[dt]
    xq = np.ascontiguousarray(xq, dtype=np.uint8).reshape(-1, row_bytes(vt, k))
    nb = k // _ELEMS[dt]
    per = 2 if dt == Q4K else 1
    out = np.zeros((xq.shape[0], w.shape[0], nb * per), dtype=np.int32)
    L = lib()
    for m in range(xq.shape[0]):
        for n in range(w.shape[0]):
            row = out[m, n]
            rc = L.orc_block_dots(dt, k, _ptr(w[n]), _ptr(xq[m]), row.ctypes.data)
            if rc != 0:
                raise ValueError("oracle block_dots failed")
    if dt == Q4K:
        return out.reshape(xq.shape[0], w.shape[0], nb, 2)
    return out


def simd_supported() -> bool:
    return bool(lib().orc_simd_supported())


def vec_dot_avx2(dt: int, k: int, w_row: np.ndarray, x_row: np.ndarray) -> float:
    return lib().orc_vec_dot_avx2(dt, k, _ptr(np.ascontiguousarray(w_row)), _ptr(np.ascontiguousarray(x_row)))


def matmul(dt: int, x: np.ndarray, w: np.ndarray, k: int, nthreads: int = 0, impl: int = GENERIC) -> np.ndarray:
    """Candle k_quants::matmul: y[m, n] = vec_dot(W[n], quant(x[m])) with the chosen vec_dot bodies."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, row_bytes(dt, k))
    y = np.zeros((x.shape[0], w.shape[0]), dtype=np.float32)
    rc = lib().orc_matmul_impl(dt, x.shape[0], k, w.shape[0], _ptr(x), _ptr(w), _ptr(y), nthreads, impl)
    if rc != 0:
        raise ValueError("oracle matmul failed")
    return y


def matmul_prequant(dt: int, xq: np.ndarray, w: np.ndarray, k: int, nthreads: int = 0,
                    impl: int = GENERIC) -> np.ndarray:
    vt = VEC_DOT_TYPE[dt]
    xq = np.ascontiguousarray(xq, dtype=np.uint8).reshape(-1, row_bytes(vt, k))
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, row_bytes(dt, k))
    y = np.zeros((xq.shape[0], w.shape[0]), dtype=np.float32)
    rc = lib().orc_matmul_prequant_impl(dt, xq.shape[0], k, w.shape[0], _ptr(xq), _ptr(w), _ptr(y), nthreads,
                                        impl)
    if rc != 0:
        raise ValueError("oracle matmul failed")
    return y
