"""Dense dequantization and the dequant-dense matmul strategy on the GPU.

* qmm_qtensor_dequantize_to: f32 bit-exact with the oracle dequantizer
  (mlx-llm/src/gguf/dequant.rs formulas), f16 / bf16 equal to that f32 value
  rounded to nearest even (numpy's f16 cast; bf16 rounding written out here);
* QMatMul.forward_via_f16 (candle-gen-lens/src/text_encoder.rs:518-529): an
  f16 dense matmul of the dequantized weight, within f16 accuracy of the f32
  dense product;
* QLinear (candle-gen/src/quant/mod.rs:515-568): DEQUANT_DENSE is the dense
  product of the dequantized weight (+ bias); INT8_FAST is QMatMul.forward
  bit for bit; and the reference's outlier regression
  (q4_packed_forward_survives_outlier_activations, quant/mod.rs:1539-1602):
  +30000 outliers on zero-weight channels leave the dequant-dense path on
  the f32 result (cosine > 0.99) while the int8 activation path collapses.
"""
import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, MatmulStrategy, QLinear, QMatMul, QTensor
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ORC = {GgmlDType.Q8_0: orc.Q8_0, GgmlDType.Q4K: orc.Q4K, GgmlDType.Q6K: orc.Q6K}


def bf16_rne(a):
    b = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def cosine(a, b):
    """Cosine similarity; 0 when either side is all zeros (the collapsed int8 path)."""
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    return float(a @ b / (na * nb)) if na > 0 and nb > 0 else 0.0


@pytest.mark.parametrize("dt", [GgmlDType.Q8_0, GgmlDType.Q4K, GgmlDType.Q6K])
def test_dequantize_dtypes_bit_exact(dt):
    rng = np.random.default_rng(int(dt))
    n, k = 96, 512
    w = (rng.standard_normal((n, k)) * rng.uniform(0.01, 3.0, (n, 1))).astype(np.float32)
    wq = orc.quantize(ORC[dt], w)
    qt = QTensor.from_ggml(wq, dt, (n, k), device=DEV)
    ref = orc.dequantize(ORC[dt], wq, n * k).reshape(n, k).astype(np.float32)
    np.testing.assert_array_equal(qt.dequantize().cpu().numpy(), ref)
    np.testing.assert_array_equal(qt.dequantize(torch.float16).cpu().numpy(), ref.astype(np.float16))
    got = qt.dequantize(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(got, bf16_rne(ref))
    with pytest.raises(Exception):
        qt.dequantize(torch.int32)


@pytest.mark.parametrize("dt", [GgmlDType.Q8_0, GgmlDType.Q4K, GgmlDType.Q6K])
def test_forward_via_f16(dt):
    rng = np.random.default_rng(10 + int(dt))
    n, k, m = 300, 1024, 17
    wq = orc.quantize(ORC[dt], (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    qt = QTensor.from_ggml(wq, dt, (n, k), device=DEV)
    x = rng.standard_normal((2, m, k)).astype(np.float32)
    y = QMatMul.from_qtensor(qt).forward_via_f16(torch.from_numpy(x).to(DEV))
    assert y.dtype == torch.float32 and y.shape == (2, m, n)
    wd = orc.dequantize(ORC[dt], wq, n * k).reshape(n, k).astype(np.float64)
    ref = x.astype(np.float64) @ wd.T
    err = np.abs(y.cpu().numpy() - ref).max() / np.sqrt((ref ** 2).mean())
    assert err <= 5e-3  # f16 operands: ~2^-11 relative per input, accumulated in f32


@pytest.mark.parametrize("dt", [GgmlDType.Q8_0, GgmlDType.Q4K, GgmlDType.Q6K])
def test_qlinear_strategies(dt):
    rng = np.random.default_rng(20 + int(dt))
    n, k = 200, 512
    wq = orc.quantize(ORC[dt], (rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    qt = QTensor.from_ggml(wq, dt, (n, k), device=DEV)
    b = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(DEV)
    x = torch.from_numpy(rng.standard_normal((3, 5, k)).astype(np.float32)).to(DEV)
    wd = orc.dequantize(ORC[dt], wq, n * k).reshape(n, k).astype(np.float64)
    ref = x.cpu().numpy().astype(np.float64) @ wd.T + b.cpu().numpy()
    dense = QLinear(qt, b, MatmulStrategy.DEQUANT_DENSE).forward(x)
    assert dense.shape == (3, 5, n)
    assert np.abs(dense.cpu().numpy() - ref).max() / np.sqrt((ref ** 2).mean()) <= 1e-4
    fast = QLinear(qt, b, MatmulStrategy.INT8_FAST).forward(x)
    assert torch.equal(fast, QMatMul.from_qtensor(qt).forward(x) + b)
    # bf16 activations: the dense strategy computes in bf16 and returns bf16
    xb = x.to(torch.bfloat16)
    yb = QLinear(qt, b, MatmulStrategy.DEQUANT_DENSE).forward(xb)
    assert yb.dtype == torch.bfloat16
    assert cosine(yb.float().cpu().numpy(), ref) > 0.999


@pytest.mark.parametrize("dt", [GgmlDType.Q8_0, GgmlDType.Q6K])
def test_dequant_dense_survives_outlier_activations(dt):
    """The reference's regression: per 32-block, channel 0 has zero weight and a +30000 activation."""
    rng = np.random.default_rng(30)
    in_dim, out_dim, m, blk = 256, 256, 64, 32
    w = (rng.standard_normal((out_dim, in_dim)) * 0.1).astype(np.float32)
    w[:, ::blk] = 0.0
    x = rng.standard_normal((m, in_dim)).astype(np.float32)
    x[:, ::blk] = 30000.0
    ref = x.astype(np.float64) @ w.T.astype(np.float64)
    wq = orc.quantize(ORC[dt], w)
    qt = QTensor.from_ggml(wq, dt, (out_dim, in_dim), device=DEV)
    xd = torch.from_numpy(x).to(DEV)
    dq = cosine(QLinear(qt, None, MatmulStrategy.DEQUANT_DENSE).forward(xd).cpu().numpy(), ref)
    q8 = cosine(QLinear(qt, None, MatmulStrategy.INT8_FAST).forward(xd).cpu().numpy(), ref)
    assert dq > 0.99, dq
    assert dq > q8 + 0.05, (dq, q8)


def test_quantize_onto_equals_device_quantize():
    """QTensor::quantize_onto from a host weight gives the same blocks as QTensor::quantize on the device."""
    w = torch.from_numpy(np.random.default_rng(31).standard_normal((300, 512)).astype(np.float32) * 0.02)
    for dt in (GgmlDType.Q4K, GgmlDType.Q6K, GgmlDType.Q8_0):
        a = QTensor.quantize_onto(w, dt, DEV)
        b = QTensor.quantize(w.to(DEV), dt)
        assert a.device == DEV and np.array_equal(a.to_ggml(), b.to_ggml())
