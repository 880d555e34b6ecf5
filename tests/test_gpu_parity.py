"""GPU parity of the HIP path against the CPU oracle (run on an MI355X).

Bars (from the task's parity contract):
  * byte / integer work bit-exact: activation quantizers (Q8_K, Q8_0), weight
    quantizers (Q4_K, Q6_K, Q8_0), GGML import/export, dequantization, and
    every per-(row, super-block) integer block dot;
  * f32 outputs: max|y_gpu - y_cpu| / rms(y_cpu) <= 1e-3 (TOL below).
Sizes: small shapes where the oracle's per-block dump is cheap, and the
BASELINE configuration shapes for the f32 outputs.
"""
import ctypes

import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, QMatMul, QTensor, QuantizedLinear, QmmError, block_dots, quantize_rows
from inference_amd import matmul_q
from inference_amd.synth import normal
from oracle import oracle as orc
import quant_ties

pytestmark = pytest.mark.gpu

TOL = 1e-3  # max|dy| / rms(y_ref), the north-star tolerance for f32 outputs
DEV = torch.device("cuda", 0)
ORC = {GgmlDType.Q8_0: orc.Q8_0, GgmlDType.Q4K: orc.Q4K, GgmlDType.Q6K: orc.Q6K, GgmlDType.Q8K: orc.Q8K}
WEIGHT_TYPES = [GgmlDType.Q4K, GgmlDType.Q6K, GgmlDType.Q8_0]


def rel_err(y, y_ref):
    y_ref = np.asarray(y_ref, dtype=np.float64)
    rms = np.sqrt(np.mean(y_ref ** 2))
    return float(np.abs(np.asarray(y, dtype=np.float64) - y_ref).max() / rms)


def special_activation_rows(k):
    """Rows exercising the Q8_K / Q8_0 edge cases: zero blocks, ties, sign of the max, clamping."""
    rows = []
    z = np.zeros(k, np.float32)
    rows.append(z.copy())  # all-zero -> d = 0, q = 0, bsums = 0
    t = np.zeros(k, np.float32)
    t[0] = -128.0  # Q8_K: iscale = 1 exactly -> x.5 values are exact ties (round away from zero)
    t[1:16] = np.array([2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.5, -3.5, 126.5, -126.5, 7.5, 11.5, -0.5, 0.5, 64.5],
                       np.float32)
    rows.append(t)
    c = np.zeros(k, np.float32)
    c[::2] = -1.0
    c[1::2] = 1.0  # first max is -1 -> iscale = +128, +1 clamps to +127
    rows.append(c)
    c2 = -c  # first max is +1 -> iscale = -128
    rows.append(c2)
    s = np.zeros(k, np.float32)
    s[k // 2 + 3] = 3.0  # single non-zero in a later block
    rows.append(s)
    q = np.zeros(k, np.float32)
    q[:32] = np.arange(-16, 16, dtype=np.float32) * (127.0 / 16.0)  # Q8_0 ties around d
    if k >= 64:
        q[32:64] = 127.0 * np.linspace(-1, 1, 32, dtype=np.float32)
    rows.append(q)
    return np.stack(rows)


@pytest.mark.parametrize("m,k", [(1, 256), (1, 4096), (3, 4096), (8, 14336), (2, 512)])
def test_q8k_activation_quantizer_bit_exact(m, k):
    x = np.concatenate([normal(10 + m, (m, k)), special_activation_rows(k)])
    xq = quantize_rows(GgmlDType.Q8K, torch.from_numpy(x).to(DEV)).cpu().numpy()
    ref = orc.quantize(orc.Q8K, x)
    assert xq.shape == ref.shape
    assert np.array_equal(xq, ref)


@pytest.mark.parametrize("m,k", [(1, 32), (1, 4096), (5, 4096), (2, 14336)])
def test_q8_0_activation_quantizer_bit_exact(m, k):
    x = np.concatenate([normal(20 + m, (m, k)), special_activation_rows(k)])
    xq = quantize_rows(GgmlDType.Q8_0, torch.from_numpy(x).to(DEV)).cpu().numpy()
    ref = orc.quantize(orc.Q8_0, x)
    assert np.array_equal(xq, ref)


def test_activation_quantizer_honours_row_stride():
    x = normal(30, (4, 8192))
    xt = torch.from_numpy(x).to(DEV)[:, 1024:1024 + 4096]  # row stride 8192, offset view
    xq = quantize_rows(GgmlDType.Q8K, xt).cpu().numpy()
    assert np.array_equal(xq, orc.quantize(orc.Q8K, np.ascontiguousarray(x[:, 1024:1024 + 4096])))


def special_weight_rows(k):
    rows = [np.zeros(k, np.float32), np.full(k, 0.5, np.float32), np.full(k, -0.25, np.float32)]
    one_hot = np.zeros(k, np.float32)
    one_hot[5] = 1.0
    rows.append(one_hot)
    rows.append(normal(41, (k,), 1e-6))  # f16 scales in the subnormal range
    rows.append(normal(42, (k,), 100.0))
    rows.append(np.abs(normal(43, (k,), 0.02)))  # non-negative rows: min clamps to 0
    rows.append(-np.abs(normal(44, (k,), 0.02)))
    ramp = np.linspace(-1, 1, k, dtype=np.float32)
    rows.append(ramp)
    return np.stack(rows)


@pytest.mark.parametrize("dt", WEIGHT_TYPES)
def test_weight_quantizer_bit_exact(dt):
    # the tie rows put every rounding step of the quantizers exactly on k + 0.5 (tests/quant_ties.py;
    # the oracle's codes there are pinned to round half away from zero by test_oracle_quant_pins.py)
    k = 4096
    w = np.concatenate([normal(40, (48, k), 0.02), special_weight_rows(k), quant_ties.weight_tie_rows(k)])
    qt = QTensor.quantize(torch.from_numpy(w).to(DEV), dt)
    assert qt.shape == w.shape and qt.dtype() == dt
    got = qt.to_ggml()
    ref = orc.quantize(ORC[dt], w).reshape(-1)
    assert got.size == ref.size == qt.storage_size_in_bytes()
    mism = np.flatnonzero(got != ref)
    assert mism.size == 0, f"{mism.size} bytes differ, first at {mism[:8]}"


@pytest.mark.parametrize("dt", WEIGHT_TYPES)
def test_ggml_import_export_and_dequantize_bit_exact(dt):
    n, k = 40, 1024
    w = np.concatenate([normal(50, (n, k), 0.02), special_weight_rows(k)])
    ref_bytes = orc.quantize(ORC[dt], w)
    for src in (ref_bytes, torch.from_numpy(ref_bytes).to(DEV)):  # host and device GGML bytes
        qt = QTensor.from_ggml(src, dt, w.shape, device=DEV)
        assert np.array_equal(qt.to_ggml(), ref_bytes.reshape(-1))
        deq = qt.dequantize().cpu().numpy()
        ref = orc.dequantize(ORC[dt], ref_bytes, w.size).reshape(w.shape)
        assert np.array_equal(deq.view(np.uint32), ref.view(np.uint32))


BLOCK_DOT_CASES = [
    (GgmlDType.Q4K, 64, 256), (GgmlDType.Q4K, 37, 2048), (GgmlDType.Q4K, 96, 4096), (GgmlDType.Q4K, 24, 14336),
    (GgmlDType.Q6K, 64, 256), (GgmlDType.Q6K, 37, 2048), (GgmlDType.Q6K, 96, 4096), (GgmlDType.Q6K, 24, 14336),
    (GgmlDType.Q8_0, 64, 32), (GgmlDType.Q8_0, 37, 2048), (GgmlDType.Q8_0, 96, 4096), (GgmlDType.Q8_0, 8, 14336),
]


@pytest.mark.parametrize("dt,n,k", BLOCK_DOT_CASES)
@pytest.mark.parametrize("m", [1, 3, 8])
def test_block_dots_bit_exact_and_outputs(dt, n, k, m):
    w = np.concatenate([normal(60, (n, k), 0.02), special_weight_rows(k)[:3]])
    wq = orc.quantize(ORC[dt], w)
    x = normal(61 + m, (m, k))
    x[0, :k // 2] *= 50.0  # uneven activation scales across blocks
    qt = QTensor.from_ggml(wq, dt, w.shape, device=DEV)
    vt = dt.vec_dot_type()
    xq = quantize_rows(vt, torch.from_numpy(x).to(DEV))
    dots, y = block_dots(qt, xq, m)
    ref = orc.block_dots(ORC[dt], wq, xq.cpu().numpy(), k)
    assert np.array_equal(dots.cpu().numpy(), ref)
    y_ref = orc.matmul_prequant(ORC[dt], xq.cpu().numpy(), wq, k)
    assert rel_err(y.cpu().numpy(), y_ref) <= TOL
    # the plain GEMV launch (no dump) gives the same outputs
    y2 = matmul_q(qt, xq, m).cpu().numpy()
    assert rel_err(y2, y_ref) <= TOL


GENERIC_CFGS = ["4,1,1", "4,2,1", "4,1,2", "8,1,1", "8,1,2"]
M1_ONLY_CFGS = ["8,2,1", "16,1,1", "16,1,2"]


@pytest.mark.parametrize("cfg", GENERIC_CFGS + M1_ONLY_CFGS)
@pytest.mark.parametrize("dt", WEIGHT_TYPES)
def test_every_launch_shape_is_correct(dt, cfg, monkeypatch):
    """All compiled (waves/workgroup, rows/wave, loads/row) variants, on ragged row counts."""
    monkeypatch.setenv("QMM_GEMV_CFG", cfg)
    for n, k in ((1, 256), (13, 2048), (70, 4096), (9, 14336)):
        w = normal(70 + n, (n, k), 0.02)
        wq = orc.quantize(ORC[dt], w)
        qt = QTensor.from_ggml(wq, dt, w.shape, device=DEV)
        for m in ((1, 2, 8) if cfg in GENERIC_CFGS else (1,)):
            x = normal(71, (m, k))
            xq = quantize_rows(dt.vec_dot_type(), torch.from_numpy(x).to(DEV))
            dots, y = block_dots(qt, xq, m)
            assert np.array_equal(dots.cpu().numpy(), orc.block_dots(ORC[dt], wq, xq.cpu().numpy(), k))
            assert rel_err(y.cpu().numpy(), orc.matmul_prequant(ORC[dt], xq.cpu().numpy(), wq, k)) <= TOL


@pytest.mark.parametrize("dt", WEIGHT_TYPES)
def test_small_grid_walks_many_rows(dt, monkeypatch):
    """A grid sized for one wave per CU makes every wave loop over ~10 rows."""
    monkeypatch.setenv("QMM_GEMV_WAVES_PER_CU", "1")
    n, k = 3000, 2048
    w = normal(80, (n, k), 0.02)
    wq = orc.quantize(ORC[dt], w)
    qt = QTensor.from_ggml(wq, dt, w.shape, device=DEV)
    x = normal(81, (2, k))
    y = QMatMul.from_qtensor(qt).forward(torch.from_numpy(x).to(DEV)).cpu().numpy()
    assert rel_err(y, orc.matmul(ORC[dt], x, wq, k)) <= TOL


@pytest.mark.parametrize("dt,k", [(GgmlDType.Q8_0, 4160), (GgmlDType.Q8_0, 5120), (GgmlDType.Q4K, 4352),
                                  (GgmlDType.Q6K, 4352)])
def test_one_row_many_rows_ragged_slices(dt, k, monkeypatch):
    """One activation row (the one-row kernels) with every wave looping over ~12 rows of several
    slices, the last one ragged: Q8_0 (one block per lane, 64 per slice) rows of 130 / 160 blocks
    are three slices, the second issued with the first and each next row's first two before the
    reduction; Q4_K / Q6_K rows of 17 blocks (16 per slice) are two."""
    monkeypatch.setenv("QMM_GEMV_WAVES_PER_CU", "1")
    n = 3000
    w = normal(82, (n, k), 0.02)
    wq = orc.quantize(ORC[dt], w)
    qt = QTensor.from_ggml(wq, dt, w.shape, device=DEV)
    x = normal(83, (1, k))
    x[0, : k // 3] *= 20.0
    y = QMatMul.from_qtensor(qt).forward(torch.from_numpy(x).to(DEV)).cpu().numpy()
    assert rel_err(y, orc.matmul(ORC[dt], x, wq, k)) <= TOL
    xq = quantize_rows(dt.vec_dot_type(), torch.from_numpy(x).to(DEV))
    y2 = matmul_q(qt, xq, 1).cpu().numpy()
    assert rel_err(y2, orc.matmul_prequant(ORC[dt], xq.cpu().numpy(), wq, k)) <= TOL


CONFIG_SHAPES = [
    (GgmlDType.Q8_0, 4096, 4096, 0, 1),      # config 1 (seeds 0 / 1)
    (GgmlDType.Q4K, 4096, 4096, 2, 3),       # config 2: q_proj
    (GgmlDType.Q4K, 1024, 4096, 2, 3),       # k/v_proj
    (GgmlDType.Q4K, 14336, 4096, 2, 3),      # gate/up
    (GgmlDType.Q4K, 4096, 14336, 2, 3),      # down
    (GgmlDType.Q6K, 1024, 4096, 4, 3),       # config 3: attn_v
    (GgmlDType.Q6K, 4096, 14336, 4, 3),      # ffn_down
]


@pytest.mark.parametrize("dt,n,k,wseed,xseed", CONFIG_SHAPES)
def test_config_shapes_match_cpu_path(dt, n, k, wseed, xseed):
    w = normal(wseed, (n, k), 0.02)
    wq = orc.quantize(ORC[dt], w)
    qt = QTensor.from_ggml(wq, dt, (n, k), device=DEV)
    x = normal(xseed, (1, k))
    y = QMatMul.from_qtensor(qt).forward(torch.from_numpy(x).to(DEV)).cpu().numpy()
    y_ref = orc.matmul(ORC[dt], x, wq, k)
    assert rel_err(y, y_ref) <= TOL
    # sampled exact block dots at full size (rows spread over the matrix)
    rows = np.linspace(0, n - 1, 8).astype(int)
    xq = quantize_rows(dt.vec_dot_type(), torch.from_numpy(x).to(DEV))
    dots, _ = block_dots(qt, xq, 1)
    ref = orc.block_dots(ORC[dt], wq[rows], xq.cpu().numpy(), k)
    assert np.array_equal(dots.cpu().numpy()[:, rows], ref)


def test_batched_rows_beyond_eight_are_chunked():
    n, k = 200, 2048
    w = normal(90, (n, k), 0.02)
    wq = orc.quantize(orc.Q6K, w)
    qt = QTensor.from_ggml(wq, GgmlDType.Q6K, w.shape, device=DEV)
    x = normal(91, (2, 13, k))  # [b, s, k] -> 26 rows
    y = QMatMul.from_qtensor(qt).forward(torch.from_numpy(x).to(DEV))
    assert tuple(y.shape) == (2, 13, n)
    assert rel_err(y.cpu().numpy().reshape(26, n), orc.matmul(orc.Q6K, x.reshape(26, k), wq, k)) <= TOL


def test_reference_quantized_linear_q8_approximates_dense():
    """crates/llm/candle-llm/src/primitives/quant.rs:52-80 on the GPU path."""
    out, inn = 4, 256
    i = np.arange(out * inn)
    w = ((i * 7 % 13).astype(np.float32) / 13.0 - 0.5).reshape(out, inn)
    x = (np.arange(inn, dtype=np.float32) / inn - 0.5).reshape(1, inn)
    dense = x @ w.T
    q = QuantizedLinear.quantize(torch.from_numpy(w).to(DEV), GgmlDType.Q8_0, None)
    got = q.forward(torch.from_numpy(x).to(DEV)).cpu().numpy()
    assert np.all(np.abs(dense - got) < 0.05)


def test_reference_q4k_cosine_vs_dense():
    """candle-gen/src/quant/mod.rs:1141-1172: Q4_K 64x256, x 4x256, cos > 0.99 vs dense."""
    w = normal(100, (64, 256), 0.1)
    x = normal(101, (4, 256))
    q = QuantizedLinear.quantize(torch.from_numpy(w).to(DEV), GgmlDType.Q4K, None)
    got = q.forward(torch.from_numpy(x).to(DEV)).cpu().numpy().ravel()
    dense = (x @ w.T).ravel()
    cos = float(np.dot(got, dense) / np.linalg.norm(got) / np.linalg.norm(dense))
    assert cos > 0.99


def test_bias_and_dtype_cast_in_quantized_linear():
    w = normal(110, (32, 512), 0.05)
    b = normal(111, (32,))
    x = normal(112, (3, 512))
    q = QuantizedLinear.quantize(torch.from_numpy(w).to(DEV), GgmlDType.Q4K, torch.from_numpy(b).to(DEV))
    y16 = q.forward(torch.from_numpy(x).to(DEV).to(torch.bfloat16))
    assert y16.dtype == torch.bfloat16
    y = q.forward(torch.from_numpy(x).to(DEV)).cpu().numpy()
    wq = orc.quantize(orc.Q4K, w)
    assert rel_err(y - b, orc.matmul(orc.Q4K, x, wq, 512)) <= TOL


def test_errors_are_raised_not_swallowed():
    qt = QTensor.quantize(torch.from_numpy(normal(120, (8, 512), 0.02)).to(DEV), GgmlDType.Q4K)
    mm = QMatMul.from_qtensor(qt)
    with pytest.raises(QmmError):
        mm.forward(torch.zeros(1, 512, device=DEV, dtype=torch.float16))  # f32 required
    with pytest.raises(QmmError):
        mm.forward(torch.zeros(1, 256, device=DEV))  # K mismatch
    with pytest.raises(QmmError):
        QTensor.quantize(torch.zeros(4, 200, device=DEV), GgmlDType.Q4K)  # not a block multiple
    with pytest.raises(QmmError):
        QTensor.from_ggml(np.zeros(100, np.uint8), GgmlDType.Q4K, (1, 256), device=DEV)  # wrong byte count


def test_repeated_calls_are_deterministic():
    qt = QTensor.quantize(torch.from_numpy(normal(130, (4096, 4096), 0.02)).to(DEV), GgmlDType.Q4K)
    x = torch.from_numpy(normal(131, (1, 4096))).to(DEV)
    mm = QMatMul.from_qtensor(qt)
    y0 = mm.forward(x)
    for _ in range(5):
        assert torch.equal(mm.forward(x), y0)


FUSED_CFGS = ["8,1,1", "8,1,2", "16,1,1", "16,1,2"]


@pytest.mark.parametrize("cfg", FUSED_CFGS)
@pytest.mark.parametrize("dt", WEIGHT_TYPES)
def test_fused_prologue_quantization_is_bit_identical(dt, cfg, monkeypatch):
    """QMatMul.forward with m <= 2 quantizes x inside the GEMV; its outputs must equal,
    bit for bit, the staged GEMV fed with the (CPU-identical) quantize_rows bytes."""
    for n, k in ((37, 2048), (70, 4096), (9, 14336)):
        w = normal(140 + n, (n, k), 0.02)
        qt = QTensor.from_ggml(orc.quantize(ORC[dt], w), dt, w.shape, device=DEV)
        for m in (1, 2):
            x = np.concatenate([normal(141, (m, k)), special_activation_rows(k)])[-m:] if m == 2 else normal(142, (1, k))
            xt = torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
            monkeypatch.setenv("QMM_GEMV_CFG", cfg)
            y_fused = QMatMul.from_qtensor(qt).forward(xt)
            monkeypatch.delenv("QMM_GEMV_CFG")  # staged reference with its default launch shape
            y_staged = matmul_q(qt, quantize_rows(dt.vec_dot_type(), xt), m)
            assert torch.equal(y_fused, y_staged), f"n={n} k={k} m={m}"


@pytest.mark.parametrize("dt", WEIGHT_TYPES)
@pytest.mark.parametrize("m", [1, 2, 5])
def test_matmul_multi_equals_separate_forwards(dt, m):
    from inference_amd import matmul_multi
    k = 4096
    qts = [QTensor.quantize(torch.from_numpy(normal(150 + i, (n, k), 0.02)).to(DEV), dt)
           for i, n in enumerate((4096, 1024, 1000, 17))]
    x = torch.from_numpy(normal(160, (m, k))).to(DEV)
    ys = matmul_multi(qts, x)
    for q, y in zip(qts, ys):
        assert torch.equal(y, QMatMul.from_qtensor(q).forward(x))


@pytest.mark.parametrize("dt", WEIGHT_TYPES)
@pytest.mark.parametrize("m", [1, 2, 3])
@pytest.mark.parametrize("count", [5, 8])
def test_matmul_multi_eight_jobs(dt, m, count):
    """More than four weights in one call (the eight-job kernels at m = 1, two launches otherwise):
    bit-identical to separate forwards, fused prologue and pre-quantized activation alike."""
    from inference_amd import matmul_multi, qmm
    k = 1024
    rows = (4096, 1024, 1024, 700, 33, 512, 256, 1)[:count]
    qts = [QTensor.quantize(torch.from_numpy(normal(240 + i, (n, k), 0.02)).to(DEV), dt)
           for i, n in enumerate(rows)]
    x = torch.from_numpy(normal(250 + m, (m, k))).to(DEV)
    ys = matmul_multi(qts, x)
    xq = quantize_rows(dt.vec_dot_type(), x)
    yq = [torch.empty((m, n), dtype=torch.float32, device=DEV) for n in rows]
    ws, ws_bytes = qmm.q_workspace(qts, m)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    qmm._check(qmm.lib().qmm_matmul_multi_q((vp * count)(*[q.handle.value for q in qts]), count, xq.data_ptr(), m,
                                            (vp * count)(*[y.data_ptr() for y in yq]), (i64 * count)(*rows),
                                            qmm._ptr(ws), ws_bytes, qmm._stream(DEV)))
    for q, y, y2 in zip(qts, ys, yq):
        ref = QMatMul.from_qtensor(q).forward(x)
        assert torch.equal(y, ref)
        assert torch.equal(y2, ref)


# ---------------------------------------------------------------------------
# prefill GEMM (m > 8): int8 MFMA path
# ---------------------------------------------------------------------------

GEMM_CASES = [(GgmlDType.Q4K, 100, 512), (GgmlDType.Q4K, 300, 1024), (GgmlDType.Q6K, 100, 512),
              (GgmlDType.Q6K, 130, 1024), (GgmlDType.Q8_0, 130, 512), (GgmlDType.Q8_0, 64, 1024)]


@pytest.mark.parametrize("dt,n,k", GEMM_CASES)
@pytest.mark.parametrize("m", [9, 64, 100, 257])
def test_gemm_block_dots_bit_exact(dt, n, k, m):
    w = np.concatenate([normal(170, (n, k), 0.02), special_weight_rows(k)[:4]])
    wq = orc.quantize(ORC[dt], w)
    qt = QTensor.from_ggml(wq, dt, w.shape, device=DEV)
    x = normal(171 + m, (m, k))
    x[1, : k // 2] *= 40.0
    x[2] = 0.0  # an all-zero activation row
    xq = quantize_rows(dt.vec_dot_type(), torch.from_numpy(x).to(DEV))
    dots, y = block_dots(qt, xq, m)
    ref = orc.block_dots(ORC[dt], wq, xq.cpu().numpy(), k)
    assert np.array_equal(dots.cpu().numpy(), ref)
    y_ref = orc.matmul_prequant(ORC[dt], xq.cpu().numpy(), wq, k)
    assert rel_err(y.cpu().numpy(), y_ref) <= TOL
    # f32 entry point (quantizes into the GEMM plane layout in one kernel)
    y2 = QMatMul.from_qtensor(qt).forward(torch.from_numpy(x).to(DEV)).cpu().numpy()
    assert rel_err(y2, orc.matmul(ORC[dt], x, wq, k)) <= TOL


@pytest.mark.parametrize("gen", [{}, {"QMM_MMQ": "2"}, {"QMM_MMQ": "4"}, {"QMM_MMQ": "4", "QMM_MMQ4_BN": "128"}])
@pytest.mark.parametrize("n,k,m", [(300, 1024, 9), (130, 512, 257), (64, 256, 130)])
def test_gemm_q4k_generations_bit_exact(monkeypatch, gen, n, k, m):
    """Every Q4_K GEMM generation (the default mmqs: split-scale int8 d term, bf16 mins term; mmq2: per-sub-block
    VALU scaling; mmq4: split-scale MFMA operands, 128x64 and 128x128 tiles) gives the oracle's integer block
    dots and f32 outputs within TOL."""
    for key, val in gen.items():
        monkeypatch.setenv(key, val)
    w = np.concatenate([normal(180 + n, (n, k), 0.02), special_weight_rows(k)[:4]])
    wq = orc.quantize(orc.Q4K, w)
    qt = QTensor.from_ggml(wq, GgmlDType.Q4K, w.shape, device=DEV)
    x = normal(181 + m, (m, k))
    x[1, : k // 2] *= 40.0
    x[2] = 0.0
    xq = quantize_rows(GgmlDType.Q8K, torch.from_numpy(x).to(DEV))
    dots, y = block_dots(qt, xq, m)
    assert np.array_equal(dots.cpu().numpy(), orc.block_dots(orc.Q4K, wq, xq.cpu().numpy(), k))
    assert rel_err(y.cpu().numpy(), orc.matmul_prequant(orc.Q4K, xq.cpu().numpy(), wq, k)) <= TOL
    y2 = QMatMul.from_qtensor(qt).forward(torch.from_numpy(x).to(DEV)).cpu().numpy()
    assert rel_err(y2, orc.matmul(orc.Q4K, x, wq, k)) <= TOL


@pytest.mark.parametrize("gen", [{}, {"QMM_MMQ6": "1"}])
@pytest.mark.parametrize("n,k,m", [(300, 1024, 9), (130, 512, 257), (64, 256, 130), (257, 2048, 128)])
def test_gemm_q6k_generations_bit_exact(monkeypatch, gen, n, k, m):
    """Both Q6_K GEMM generations (the default mmqs6: each int8 sub-block scale as three digits in [-3, 4]
    multiplied into the int8 MFMA operands; mmq<Q6_K>: masked MFMAs and a multiply-add per sub-block) give
    the oracle's integer block dots and f32 outputs within TOL. The weight holds the saturating block (int8
    scales -128 and 127, the ends of the digit range) and the tie block (odd scales), tiled along k."""
    for key, val in gen.items():
        monkeypatch.setenv(key, val)
    w = np.concatenate([normal(190 + n, (n, k), 0.02), special_weight_rows(k)[:4],
                        np.tile(quant_ties.q6k_saturating_block()[0], (2, k // 256)),
                        np.tile(quant_ties.q6k_block()[0], (2, k // 256))]).astype(np.float32)
    wq = orc.quantize(orc.Q6K, w)
    qt = QTensor.from_ggml(wq, GgmlDType.Q6K, w.shape, device=DEV)
    x = normal(191 + m, (m, k))
    x[1, : k // 2] *= 40.0
    x[2] = 0.0
    xq = quantize_rows(GgmlDType.Q8K, torch.from_numpy(x).to(DEV))
    dots, y = block_dots(qt, xq, m)
    assert np.array_equal(dots.cpu().numpy(), orc.block_dots(orc.Q6K, wq, xq.cpu().numpy(), k))
    assert rel_err(y.cpu().numpy(), orc.matmul_prequant(orc.Q6K, xq.cpu().numpy(), wq, k)) <= TOL
    y2 = QMatMul.from_qtensor(qt).forward(torch.from_numpy(x).to(DEV)).cpu().numpy()
    assert rel_err(y2, orc.matmul(orc.Q6K, x, wq, k)) <= TOL


@pytest.mark.parametrize("n,k,m", [(300, 1024, 9), (130, 512, 257), (64, 256, 130), (257, 2048, 128)])
def test_gemm_q8_0_generations_bit_exact(monkeypatch, n, k, m):
    """Both Q8_0 GEMM generations (the default mmqs8: activation rows and weight codes straight into LDS,
    128 x 128 tiles of eight waves; mmq<Q8_0>: 64 x 128 tiles staged through registers) give the oracle's
    integer block dots, and the same f32 outputs bit for bit (the same multiply-add per block in the same
    order), within TOL of the oracle; also through the f32 entry point."""
    w = np.concatenate([normal(200 + n, (n, k), 0.02), special_weight_rows(k)[:4]]).astype(np.float32)
    wq = orc.quantize(orc.Q8_0, w)
    qt = QTensor.from_ggml(wq, GgmlDType.Q8_0, w.shape, device=DEV)
    x = normal(201 + m, (m, k))
    x[1, : k // 2] *= 40.0
    x[2] = 0.0
    xq = quantize_rows(GgmlDType.Q8_0, torch.from_numpy(x).to(DEV))
    ref_dots = orc.block_dots(orc.Q8_0, wq, xq.cpu().numpy(), k)
    outs = []
    for gen in ({}, {"QMM_MMQ8": "1"}):
        monkeypatch.delenv("QMM_MMQ8", raising=False)
        for key, val in gen.items():
            monkeypatch.setenv(key, val)
        dots, y = block_dots(qt, xq, m)
        assert np.array_equal(dots.cpu().numpy(), ref_dots), gen
        y2 = QMatMul.from_qtensor(qt).forward(torch.from_numpy(x).to(DEV))
        assert rel_err(y2.cpu().numpy(), orc.matmul(orc.Q8_0, x, wq, k)) <= TOL
        outs.append((y, y2))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert rel_err(outs[0][0].cpu().numpy(), orc.matmul_prequant(orc.Q8_0, xq.cpu().numpy(), wq, k)) <= TOL


@pytest.mark.parametrize("dt,n,k,wseed", [(GgmlDType.Q4K, 14336, 4096, 6), (GgmlDType.Q4K, 4096, 14336, 6),
                                          (GgmlDType.Q6K, 4096, 14336, 6), (GgmlDType.Q8_0, 14336, 4096, 6),
                                          (GgmlDType.Q8_0, 4096, 14336, 6)])
def test_prefill_config_shapes_match_cpu_path(dt, n, k, wseed):
    """Config 4: x 512 x k (seed 5) through QMatMul.forward; the CPU path is
    evaluated on 48 of the 512 rows (spread over the batch). The Q8_0 legs run the
    bench's Q8_0 GEMM shapes (the engine's Q8 projections)."""
    w = normal(wseed, (n, k), 0.02)
    wq = orc.quantize(ORC[dt], w)
    qt = QTensor.from_ggml(wq, dt, (n, k), device=DEV)
    x = normal(5, (512, k))
    y = QMatMul.from_qtensor(qt).forward(torch.from_numpy(x).to(DEV)).cpu().numpy()
    rows = np.linspace(0, 511, 48).astype(int)
    y_ref = orc.matmul(ORC[dt], x[rows], wq, k)
    assert rel_err(y[rows], y_ref) <= TOL


# ---------------------------------------------------------------------------
# mixture of experts (config 5)
# ---------------------------------------------------------------------------

def _stacked_experts(E, H, F, seed, dt_gu=GgmlDType.Q4K, dt_down=GgmlDType.Q6K):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    mats = {}
    for name, rows, cols, dt in (("gate", F, H, dt_gu), ("up", F, H, dt_gu), ("down", H, F, dt_down)):
        w = torch.randn((E * rows, cols), generator=g, device=DEV) * 0.02
        qt = QTensor.quantize(w, dt)
        del w
        raw = qt.to_ggml()
        per = raw.size // E
        mats[name] = (qt, [raw[e * per:(e + 1) * per] for e in range(E)])
    return mats


def test_moe_route_matches_oracle():
    from inference_amd import moe_route
    from oracle import moe
    # decode sizes, prefill sizes, the limits (T*k = 8192, E = 256, k = 8) and ragged token counts
    for T, E, k in ((8, 8, 2), (37, 16, 4), (1, 4, 1), (512, 8, 2), (4096, 8, 2), (1000, 256, 8), (130, 64, 3)):
        logits = normal(200 + T, (T, E))
        counts, offsets, ptok, pw, tp = [a.cpu().numpy() for a in moe_route(torch.from_numpy(logits).to(DEV), k)]
        experts, weights = moe.route(logits, k)
        assert counts.sum() == T * k and offsets[-1] == T * k
        for e in range(E):
            toks = [t for t in range(T) if e in experts[t]]
            assert list(ptok[offsets[e]:offsets[e] + counts[e]]) == toks
            for i, t in enumerate(toks):
                assert abs(pw[offsets[e] + i] - weights[t][experts[t].index(e)]) < 1e-6
        for t in range(T):
            es = [int(np.searchsorted(offsets, p, side="right") - 1) for p in tp[t * k:(t + 1) * k]]
            assert es == sorted(experts[t]) and all(ptok[p] == t for p in tp[t * k:(t + 1) * k])


@pytest.mark.parametrize("E,H,F,T,k", [(8, 512, 1024, 8, 2), (4, 256, 512, 3, 2), (8, 512, 768, 16, 2)])
def test_moe_ffn_matches_oracle_small(E, H, F, T, k):
    from inference_amd import moe_ffn
    from oracle import moe
    mats = _stacked_experts(E, H, F, 210 + E + T)
    x = normal(220, (T, H))
    logits = normal(221, (T, E))
    y = moe_ffn(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), mats["gate"][0], mats["up"][0],
                mats["down"][0], k).cpu().numpy()
    y_ref = moe.moe_ffn(x, logits, mats["gate"][1], mats["up"][1], mats["down"][1], orc.Q4K, orc.Q6K, k)
    assert rel_err(y, y_ref) <= TOL


def test_moe_ffn_config5_matches_oracle():
    """Config 5: 8 experts, Q4_K gate/up 14336x4096, Q6_K down 4096x14336, 8 tokens, top-2."""
    from inference_amd import moe_ffn
    from oracle import moe
    E, H, F, T, k = 8, 4096, 14336, 8, 2
    mats = _stacked_experts(E, H, F, 7)
    x = normal(7, (T, H))
    logits = normal(8, (T, E))
    y = moe_ffn(torch.from_numpy(x).to(DEV), torch.from_numpy(logits).to(DEV), mats["gate"][0], mats["up"][0],
                mats["down"][0], k).cpu().numpy()
    y_ref = moe.moe_ffn(x, logits, mats["gate"][1], mats["up"][1], mats["down"][1], orc.Q4K, orc.Q6K, k)
    assert rel_err(y, y_ref) <= TOL


def test_moe_gemv_equals_per_expert_forward():
    """The expert-grouped GEMV gives, bit for bit, each expert's own QMatMul on its gathered rows."""
    from inference_amd import moe_route, qmm
    E, H, F, T, k = 8, 1024, 2048, 8, 2
    mats = _stacked_experts(E, H, F, 230)
    x = torch.from_numpy(normal(231, (T, H))).to(DEV)
    counts, offsets, ptok, pw, tp = moe_route(torch.from_numpy(normal(232, (T, E))).to(DEV), k)
    P = T * k
    xg = x[ptok.long()]
    xq = quantize_rows(GgmlDType.Q8K, xg)
    yg = torch.empty((P, F), device=DEV)
    yu = torch.empty((P, F), device=DEV)
    import ctypes
    hs = (ctypes.c_void_p * 2)(mats["gate"][0].handle.value, mats["up"][0].handle.value)
    ys = (ctypes.c_void_p * 2)(yg.data_ptr(), yu.data_ptr())
    qmm._check(qmm.lib().qmm_moe_gemv(hs, 2, E, xq.data_ptr(), P, counts.data_ptr(), offsets.data_ptr(), ys,
                                      qmm._stream(DEV)))
    c, o = counts.cpu().numpy(), offsets.cpu().numpy()
    gate_full = mats["gate"][0].dequantize()  # only for slicing per-expert tensors below
    for e in range(E):
        if c[e] == 0:
            continue
        qe = QTensor.from_ggml(mats["gate"][1][e], GgmlDType.Q4K, (F, H), device=DEV)
        ref = matmul_q(qe, xq[o[e]:o[e] + c[e]].contiguous(), int(c[e]))
        assert torch.equal(yg[o[e]:o[e] + c[e]], ref)
    del gate_full
