"""qmm_matmul_grouped: several QMatMul::forward calls at m = 1 on two independent rows in one launch.

Every output must equal, bit for bit, qmm_matmul on that weight and row (the same Q8_K activation bytes and
the same per-row arithmetic as the one-row GEMV), and the f32 outputs must be within 1e-3 * rms of the
oracle's k_quants::matmul. Cases: the config-2 set (q/k/v/gate/up on one row, down on another), one group
only, eight weights in a group, Q6_K weights, rows that leave some waves idle, and argument errors.
"""
import ctypes

import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, QmmError, QTensor, matmul_grouped, qmm
from inference_amd.synth import normal
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ORC = {GgmlDType.Q4K: orc.Q4K, GgmlDType.Q6K: orc.Q6K}


def rel_err(y, y_ref):
    y_ref = np.asarray(y_ref, dtype=np.float64)
    return float(np.abs(np.asarray(y, dtype=np.float64) - y_ref).max() / np.sqrt(np.mean(y_ref ** 2)))


def weights(shapes, dt, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return [QTensor.quantize(torch.randn((n, k), generator=g, device=DEV) * 0.02, dt) for n, k in shapes]


def single(qt, x):
    n, k = qt.shape
    y = torch.empty((1, n), dtype=torch.float32, device=DEV)
    L = qmm.lib()
    wsb = int(L.qmm_matmul_workspace_size(qt.handle, 1))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    qmm._check(L.qmm_matmul(qt.handle, x.data_ptr(), 1, k, y.data_ptr(), n, ws.data_ptr(), wsb, qmm._stream(DEV)))
    return y.reshape(-1)


CASES = [
    # (dtype, shapes of group 0, shapes of group 1)
    (GgmlDType.Q4K, [(4096, 4096), (1024, 4096), (1024, 4096), (14336, 4096), (14336, 4096)], [(4096, 14336)]),
    (GgmlDType.Q4K, [(768, 2048), (256, 2048)], []),
    (GgmlDType.Q4K, [], [(1000, 1024), (24, 1024)]),
    (GgmlDType.Q4K, [(64 + 7 * i, 512) for i in range(8)], [(33, 8192)] * 8),
    (GgmlDType.Q6K, [(4096, 4096), (1024, 4096)], [(4096, 14336)]),
    (GgmlDType.Q6K, [(5, 256)], [(3, 16384)]),
]


@pytest.mark.parametrize("dt,g0,g1", CASES)
def test_grouped_equals_single_launches_and_oracle(dt, g0, g1):
    qts = weights(g0 + g1, dt, 900 + len(g0) * 7 + len(g1))
    pairs = [(q, 0) for q in qts[:len(g0)]] + [(q, 1) for q in qts[len(g0):]]
    k0 = g0[0][1] if g0 else 256
    k1 = g1[0][1] if g1 else 256
    xs_np = [normal(910 + k0, (1, k0)), normal(911 + k1, (1, k1))]
    xs = [torch.from_numpy(x).to(DEV) for x in xs_np]
    outs = [torch.full((q.shape[0],), float("nan"), device=DEV) for q, _ in pairs]
    matmul_grouped(pairs, xs, outs)
    torch.cuda.synchronize()
    for i, (q, gi) in enumerate(pairs):
        got = outs[i].cpu().numpy()
        want = single(q, xs[gi]).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (i, q.shape)
        ref = orc.matmul(ORC[dt], xs_np[gi], q.to_ggml(), q.shape[1])
        assert rel_err(got, ref) <= 1e-3, (i, q.shape)


def test_grouped_rejects_bad_arguments():
    a, b = weights([(256, 1024), (256, 2048)], GgmlDType.Q4K, 920)
    c = weights([(256, 1024)], GgmlDType.Q6K, 921)[0]
    d = weights([(256, 1024)], GgmlDType.Q8_0, 922)[0]
    x = [torch.zeros((1, 1024), device=DEV), torch.zeros((1, 2048), device=DEV)]
    with pytest.raises(QmmError):
        matmul_grouped([(a, 0), (b, 0)], x)  # one group, two k
    with pytest.raises(QmmError):
        matmul_grouped([(a, 0), (c, 1)], x)  # two dtypes
    with pytest.raises(QmmError):
        matmul_grouped([(d, 0)], x)  # Q8_0
    with pytest.raises(QmmError):
        matmul_grouped([(a, 0)] * 9, x)  # nine weights in one group
    L = qmm.lib()
    hs = (ctypes.c_void_p * 1)(a.handle.value)
    y = torch.empty(256, device=DEV)
    assert L.qmm_matmul_grouped(hs, (ctypes.c_int * 1)(2), 1, (ctypes.c_void_p * 2)(x[0].data_ptr(), None),
                                (ctypes.c_void_p * 1)(y.data_ptr()), qmm._stream(DEV)) != 0  # group 2
