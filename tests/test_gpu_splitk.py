"""Split-K prefill GEMMs: narrow weights at small m spread their K steps over blockIdx.z.

A GEMM whose output tiles cover fewer than half the CUs (e.g. m = 127 against
N = 1024 or 4096) splits its 256-element K steps into S ranges; each range's
f32 partial goes to the workspace and a second kernel sums the partials in
split order. The integer block dots are the unsplit kernel's (bit-exact); the
f32 outputs are re-associated sums, so the bar is the north star's
max|dy| / rms <= 1e-3 against the oracle, and ~1e-6 against the unsplit run.
QMM_SPLITK=<S> forces S splits (1 = off).
"""
import ctypes

import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, QMatMul, QTensor, qmm
from inference_amd.synth import normal
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 1e-3
ORC = {GgmlDType.Q4K: orc.Q4K, GgmlDType.Q6K: orc.Q6K, GgmlDType.Q8_0: orc.Q8_0}
vp, i64 = ctypes.c_void_p, ctypes.c_int64


def rel_err(y, y_ref):
    y_ref = np.asarray(y_ref, dtype=np.float64)
    return float(np.abs(np.asarray(y, dtype=np.float64) - y_ref).max() / np.sqrt(np.mean(y_ref ** 2)))


def weight(dt, n, k, seed):
    w = normal(seed, (n, k), 0.02)
    return QTensor.from_ggml(orc.quantize(ORC[dt], w), dt, (n, k), device=DEV)


@pytest.mark.parametrize("dt,n,k,m", [
    (GgmlDType.Q4K, 1024, 4096, 127),   # mmq4, 16 tiles
    (GgmlDType.Q4K, 4096, 14336, 127),  # mmq4, 64 tiles, 56 K steps
    (GgmlDType.Q4K, 1000, 2304, 33),    # ragged N, 9 K steps
    (GgmlDType.Q6K, 1024, 4096, 127),   # mmq<Q6_K>, 16 tiles
    (GgmlDType.Q6K, 4096, 14336, 127),
    (GgmlDType.Q8_0, 512, 4096, 100),
])
def test_split_k_outputs(monkeypatch, dt, n, k, m):
    qt = weight(dt, n, k, 900 + n + m)
    x = torch.from_numpy(normal(901 + m, (m, k))).to(DEV)
    want = orc.matmul(ORC[dt], x.cpu().numpy(), qt.to_ggml(), k)
    mm = QMatMul(qt)
    monkeypatch.setenv("QMM_SPLITK", "1")
    ref = mm.forward(x)
    assert rel_err(ref.cpu().numpy(), want) <= TOL
    for sp in ("3", "16", None):  # forced uneven splits, the most splits, the default plan
        if sp is None:
            monkeypatch.delenv("QMM_SPLITK")
        else:
            monkeypatch.setenv("QMM_SPLITK", sp)
        got = mm.forward(x)
        assert rel_err(got.cpu().numpy(), want) <= TOL, f"splits {sp}"
        assert rel_err(got.cpu().numpy(), ref.cpu().numpy()) <= 1e-5, f"splits {sp}"


@pytest.mark.parametrize("dt", [GgmlDType.Q4K, GgmlDType.Q6K])
def test_split_k_block_dots_bit_exact(monkeypatch, dt):
    """The dump kernels under split-K write every (row, column, block) dot once, from the split that owns it."""
    n, k, m = 256, 2048, 20
    qt = weight(dt, n, k, 910)
    x = normal(911, (m, k))
    xq = orc.quantize(orc.Q8K, x)
    want = orc.block_dots(ORC[dt], qt.to_ggml(), xq, k)
    y_ref = orc.matmul_prequant(ORC[dt], xq, qt.to_ggml(), k)
    for sp in ("1", "3", "8"):
        monkeypatch.setenv("QMM_SPLITK", sp)
        dots, y = qmm.block_dots(qt, torch.from_numpy(xq).to(DEV), m)
        assert np.array_equal(dots.cpu().numpy(), want), f"splits {sp}"
        assert rel_err(y.cpu().numpy(), y_ref) <= TOL


@pytest.mark.parametrize("norm", [False, True])
def test_split_k_in_matmul_ex_accumulate(monkeypatch, norm):
    """matmul_ex at m > 8 with RMSNorm rows and the residual add: the partials sit after the normalised rows
    in the workspace, and the sum kernel adds onto y."""
    n, k, m = 1024, 4096, 64
    qts = [weight(GgmlDType.Q4K, n, k, 920), weight(GgmlDType.Q4K, 512, k, 921)]
    x = normal(922, (m, k))
    nw = np.linspace(0.5, 1.5, k).astype(np.float32)
    y0 = [normal(923 + j, (m, q.shape[0])) for j, q in enumerate(qts)]
    L = qmm.lib()

    def run():
        wsb = max(int(L.qmm_matmul_ex_workspace_size(q.handle, m, int(norm))) for q in qts)
        ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
        ys = [torch.from_numpy(a).to(DEV) for a in y0]
        nwd = torch.from_numpy(nw).to(DEV)
        xd = torch.from_numpy(x).to(DEV)
        qmm._check(L.qmm_matmul_ex((vp * 2)(*[q.handle.value for q in qts]), 2, xd.data_ptr(), m, k,
                                   nwd.data_ptr() if norm else None, ctypes.c_float(1e-5), 1,
                                   (vp * 2)(*[y.data_ptr() for y in ys]), (i64 * 2)(*[q.shape[0] for q in qts]),
                                   ws.data_ptr(), wsb, qmm._stream(DEV)))
        torch.cuda.synchronize()
        return [y.cpu().numpy() for y in ys]
    monkeypatch.setenv("QMM_SPLITK", "1")
    ref = run()
    monkeypatch.delenv("QMM_SPLITK")
    got = run()
    from oracle import llama as ol
    xin = ol.rms_norm(x, nw, 1e-5) if norm else x
    for j, q in enumerate(qts):
        want = y0[j] + orc.matmul(orc.Q4K, xin, q.to_ggml(), k)
        assert rel_err(got[j], want) <= TOL
        assert rel_err(got[j], ref[j]) <= 1e-5
