"""The prefetch-ring one-row GEMV kernels (gemv1p) against gemv1 and the CPU oracle.

gemv1p keeps the per-block arithmetic, the summation order and the output
path of gemv1, so its outputs must be bit-identical to gemv1's for every
format, launch kind (staged Q8_K / fused quantization with and without the
RMSNorm prologue / mixed Q4_K+Q6_K jobs / eight-job tables / accumulate) and
prefetch depth; against the oracle the f32 bar is max|dy| / rms <= 1e-3.
QMM_GEMV1P selects the kernel family per launch (0: gemv1, P: gemv1p with P
slices in flight).
"""
import ctypes

import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, QTensor, qmm
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 1e-3
ORC = {GgmlDType.Q4K: orc.Q4K, GgmlDType.Q6K: orc.Q6K}
vp, i64 = ctypes.c_void_p, ctypes.c_int64


def L():
    return qmm.lib()


def S():
    return qmm._stream(DEV)


def t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / np.sqrt((want ** 2).mean()))


def run_ex(qts, x, k, norm_w, accumulate, y0=None):
    """qmm_matmul_ex over qts (fused quantization); returns the outputs."""
    rows = [qt_rows(q) for q in qts]
    wsb = max(int(L().qmm_matmul_ex_workspace_size(q.handle, 1, int(norm_w is not None))) for q in qts)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    ys = [(y0[i].clone() if y0 is not None else torch.full((1, n), float("nan"), device=DEV))
          for i, n in enumerate(rows)]
    qmm._check(L().qmm_matmul_ex((vp * len(qts))(*[q.handle.value for q in qts]), len(qts), x.data_ptr(), 1, k,
                                 norm_w.data_ptr() if norm_w is not None else None, ctypes.c_float(1e-5),
                                 int(accumulate), (vp * len(qts))(*[y.data_ptr() for y in ys]),
                                 (i64 * len(qts))(*rows), ws.data_ptr(), wsb, S()))
    torch.cuda.synchronize()
    return ys


def run_multi_q(qts, xq):
    rows = [qt_rows(q) for q in qts]
    ys = [torch.full((1, n), float("nan"), device=DEV) for n in rows]
    qmm._check(L().qmm_matmul_multi_q((vp * len(qts))(*[q.handle.value for q in qts]), len(qts), xq.data_ptr(), 1,
                                      (vp * len(qts))(*[y.data_ptr() for y in ys]), (i64 * len(qts))(*rows), None, 0,
                                      S()))
    torch.cuda.synchronize()
    return ys


def qt_rows(q):
    dt, n, k = ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64()
    qmm._check(L().qmm_qtensor_info(q.handle, ctypes.byref(dt), ctypes.byref(n), ctypes.byref(k)))
    return int(n.value)


def under(monkeypatch, p, fn):
    monkeypatch.setenv("QMM_GEMV1P", str(p))
    try:
        return fn()
    finally:
        monkeypatch.delenv("QMM_GEMV1P")


SHAPES = [(1000, 4096), (4099, 4096), (333, 2304), (700, 14336), (257, 16384)]


@pytest.mark.parametrize("dt", [GgmlDType.Q4K, GgmlDType.Q6K])
@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("mode", ["staged", "fused", "norm", "accumulate"])
def test_ring_equals_gemv1_and_oracle(monkeypatch, dt, n, k, mode):
    rng = np.random.default_rng(n + k + int(dt))
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((1, k)).astype(np.float32)
    wq = orc.quantize(ORC[dt], w)
    qt = QTensor.from_ggml(wq, dt, (n, k), device=DEV)
    xd = t(x)
    nw = rng.uniform(0.5, 1.5, k).astype(np.float32) if mode == "norm" else None
    nwd = t(nw) if nw is not None else None
    y0 = [t(rng.standard_normal((1, n)).astype(np.float32))] if mode == "accumulate" else None
    if mode == "staged":
        xq = t(orc.quantize(orc.Q8K, x), torch.uint8)
        call = lambda: run_multi_q([qt], xq)[0]  # noqa: E731
    else:
        call = lambda: run_ex([qt], xd, k, nwd, mode == "accumulate", y0)[0]  # noqa: E731
    ref = under(monkeypatch, 0, call)
    for p in (1, 2):
        got = under(monkeypatch, p, call)
        assert torch.equal(got, ref), f"P={p}: differs from gemv1"
    # oracle: the same quantized activation, the reference block dots
    xin = x
    if nw is not None:
        from oracle import llama as ol
        xin = ol.rms_norm(x, nw, 1e-5)
    want = orc.matmul(ORC[dt], xin, wq, k)
    if y0 is not None:
        want = want + y0[0].cpu().numpy()
    assert rel_err(ref.cpu().numpy(), want) <= TOL


@pytest.mark.parametrize("k", [4096, 14336])
@pytest.mark.parametrize("mode", ["staged", "fused", "norm"])
@pytest.mark.parametrize("njobs", [3, 6])
def test_ring_mixed_and_eight_job_tables(monkeypatch, k, mode, njobs):
    """Mixed Q4_K / Q6_K jobs in one launch (q/k/v-like) and eight-job tables."""
    rng = np.random.default_rng(7 * k + njobs)
    dts = [GgmlDType.Q4K, GgmlDType.Q4K, GgmlDType.Q6K, GgmlDType.Q4K, GgmlDType.Q6K, GgmlDType.Q4K][:njobs]
    rows = [4096, 1024, 1024, 2000, 515, 64][:njobs]
    qts = [QTensor.quantize(t((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), dt)
           for n, dt in zip(rows, dts)]
    x = rng.standard_normal((1, k)).astype(np.float32)
    xd = t(x)
    nwd = t(rng.uniform(0.5, 1.5, k).astype(np.float32)) if mode == "norm" else None
    if mode == "staged":
        xq = t(orc.quantize(orc.Q8K, x), torch.uint8)
        call = lambda: run_multi_q(qts, xq)  # noqa: E731
    else:
        call = lambda: run_ex(qts, xd, k, nwd, False)  # noqa: E731
    ref = under(monkeypatch, 0, call)
    for p in (1, 2):
        got = under(monkeypatch, p, call)
        for j, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), f"P={p} job {j}: differs from gemv1"


def test_default_policy_uses_ring_for_q6k_long_rows():
    """The default dispatch (no QMM_GEMV1P) gives the same bits as gemv1 on the down shape."""
    rng = np.random.default_rng(5)
    n, k = 4096, 14336
    qt = QTensor.quantize(t((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), GgmlDType.Q6K)
    xq = t(orc.quantize(orc.Q8K, rng.standard_normal((1, k)).astype(np.float32)), torch.uint8)
    got = run_multi_q([qt], xq)[0]
    import os
    os.environ["QMM_GEMV1P"] = "0"
    try:
        ref = run_multi_q([qt], xq)[0]
    finally:
        del os.environ["QMM_GEMV1P"]
    assert torch.equal(got, ref)


def _moe_gemv(qts, E, xq, P, counts, offsets, F):
    ys = [torch.full((P, F), float("nan"), device=DEV) for _ in qts]
    qmm._check(L().qmm_moe_gemv((vp * len(qts))(*[q.handle.value for q in qts]), len(qts), E, xq.data_ptr(), P,
                                counts.data_ptr(), offsets.data_ptr(), (vp * len(qts))(*[y.data_ptr() for y in ys]),
                                S()))
    torch.cuda.synchronize()
    return ys


@pytest.mark.parametrize("dt,K", [(GgmlDType.Q4K, 4096), (GgmlDType.Q6K, 5120), (GgmlDType.Q4K, 5120)])
@pytest.mark.parametrize("skew", [False, True, "single"])
def test_moe_ring_gemv_equals_generic(monkeypatch, dt, K, skew):
    """The expert ring GEMV (QMM_MOE_GEMV=P) against the generic M = 8 expert GEMV: bit-identical, including
    experts with more than eight tokens (skew: every token routes to experts 0 and 1) and one active expert
    taking the whole grid (single: top-1 routing, every token to expert 3)."""
    from inference_amd import moe_route
    E, F, T = 4, 768, 10
    k = 1 if skew == "single" else 2
    rng = np.random.default_rng(K + (2 if skew == "single" else int(skew)))
    qts = [QTensor.quantize(t((rng.standard_normal((E * F, K)) * 0.02).astype(np.float32)), dt) for _ in range(2)]
    logits = rng.standard_normal((T, E)).astype(np.float32)
    if skew == "single":
        logits[:, 3] += 10.0
    elif skew:
        logits[:, :2] += 10.0
    counts, offsets, ptok, pw, tp = moe_route(t(logits), k)
    P = T * k
    xg = t(rng.standard_normal((T, K)).astype(np.float32))[ptok.long()]
    xq = t(orc.quantize(orc.Q8K, xg.cpu().numpy()), torch.uint8)
    monkeypatch.setenv("QMM_MOE_GEMV", "0")
    ref = _moe_gemv(qts, E, xq, P, counts, offsets, F)
    for p in ("1", "2"):
        monkeypatch.setenv("QMM_MOE_GEMV", p)
        got = _moe_gemv(qts, E, xq, P, counts, offsets, F)
        for a, b in zip(got, ref):
            assert torch.equal(a, b), f"P={p}"
    if skew == "single":
        assert int(counts[3]) == T and int(counts.sum()) == T
    elif skew:
        assert int(counts[0]) > 8


def _matmul_q(qt, xq, m, n, y0=None):
    y = y0.clone() if y0 is not None else torch.full((m, n), float("nan"), device=DEV)
    qmm._check(L().qmm_matmul_q_ex(qt.handle, xq.data_ptr(), m, y.data_ptr(), n, int(y0 is not None), None, 0,
                                   S()))
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("dt", [GgmlDType.Q4K, GgmlDType.Q6K])
@pytest.mark.parametrize("n,k", [(1000, 4096), (4099, 4096), (333, 5120), (700, 14336)])
@pytest.mark.parametrize("m", [2, 5, 8])
@pytest.mark.parametrize("acc", [False, True])
def test_multirow_kernel_equals_general_gemv(monkeypatch, dt, n, k, m, acc):
    """Two to eight staged rows of one k-quant weight take the token-interleaved multi-row kernel
    (by default on weights of >= 2048 rows, from seven rows on smaller ones; QMM_GEMV_ROWS=2 forces it):
    bit-identical to the general multi-row GEMV (QMM_GEMV_ROWS=0), with and without accumulation,
    including a K with a partial slice (5120) and row counts that are not multiples of 16; within 1e-3
    of the oracle."""
    rng = np.random.default_rng(n * 7 + k + m + int(dt) + 100 * int(acc))
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    wq = orc.quantize(ORC[dt], w)
    qt = QTensor.from_ggml(wq, dt, (n, k), device=DEV)
    xq = t(orc.quantize(orc.Q8K, x), torch.uint8)
    y0 = t(rng.standard_normal((m, n)).astype(np.float32)) if acc else None
    monkeypatch.setenv("QMM_GEMV_ROWS", "2")
    got = _matmul_q(qt, xq, m, n, y0)
    monkeypatch.setenv("QMM_GEMV_ROWS", "0")
    ref = _matmul_q(qt, xq, m, n, y0)
    assert torch.equal(got, ref), "differs from the general multi-row GEMV"
    want = orc.matmul(ORC[dt], x, wq, k)
    if acc:
        want = want + y0.cpu().numpy()
    assert rel_err(got.cpu().numpy(), want) <= TOL
