"""MI355X-native quantized matmul (Candle QTensor/QMatMul over GGML Q8_0/Q4_K/Q6_K).

The compute lives in ``inference_amd/_lib/libqmm.so`` (C ABI: ``include/qmm.h``),
built from ``inference_amd/csrc`` for gfx950. ``inference_amd.qmm`` mirrors the
reference engine's QTensor / QMatMul / QuantizedLinear surface over it.
"""
from .qmm import (  # noqa: F401
    GgmlDType,
    MatmulStrategy,
    QLinear,
    Projection,
    QMatMul,
    QmmError,
    QTensor,
    QuantizedLinear,
    QuantSpec,
    block_dots,
    matmul_grouped,
    matmul_multi,
    moe_ffn,
    moe_route,
    matmul_q,
    quantize_rows,
)
