"""qmm_matmul_noalloc: qmm_matmul with the library's per-device scratch array.

Its outputs must equal qmm_matmul's with a caller workspace bit for bit (the
same kernels and the same workspace layout), for two calls in a row where the
second is smaller (the array keeps the first call's contents), over the GEMV
(fused and staged) and GEMM paths and every weight format; a call that needs
more than the array is refused before any launch; and the call works inside a
stream capture (no allocation), every replay equal to the eager result.
"""
import ctypes

import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, QTensor, qmm
from inference_amd.synth import normal

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def L():
    return qmm.lib()


def S():
    return qmm._stream(DEV)


def with_ws(qt, x, m):
    n = qt.shape[0]
    y = torch.full((m, n), float("nan"), device=DEV)
    nb = int(L().qmm_matmul_workspace_size(qt.handle, m))
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=DEV)
    qmm._check(L().qmm_matmul(qt.handle, x.data_ptr(), m, x.stride(0), y.data_ptr(), n, ws.data_ptr(), nb, S()))
    return y


def noalloc(qt, x, m, y=None):
    n = qt.shape[0]
    y = torch.full((m, n), float("nan"), device=DEV) if y is None else y
    qmm._check(L().qmm_matmul_noalloc(qt.handle, x.data_ptr(), m, x.stride(0), y.data_ptr(), n, S()))
    return y


@pytest.fixture(scope="module", autouse=True)
def init():
    qmm._check(L().qmm_init(0))  # set-up: resolves the scratch array's address on device 0


@pytest.mark.parametrize("dt,n,k", [(GgmlDType.Q4K, 4096, 4096), (GgmlDType.Q6K, 1024, 4096),
                                    (GgmlDType.Q8_0, 1024, 2048)])
def test_noalloc_equals_caller_workspace(dt, n, k):
    qt = QTensor.quantize(torch.from_numpy(normal(900 + int(dt), (n, k), 0.02)).to(DEV), dt)
    # each pair: a call, then a smaller one that finds the first call's contents
    for m_big, m_small in ((512, 127), (64, 9), (8, 3), (2, 1)):
        xb = torch.from_numpy(normal(910 + m_big, (m_big, k))).to(DEV)
        xs = torch.from_numpy(normal(920 + m_small, (m_small, k))).to(DEV)
        yb = noalloc(qt, xb, m_big)
        ys = noalloc(qt, xs, m_small)
        torch.cuda.synchronize()
        assert torch.equal(yb, with_ws(qt, xb, m_big)), (dt, m_big)
        assert torch.equal(ys, with_ws(qt, xs, m_small)), (dt, m_small)


def test_noalloc_refuses_calls_beyond_its_scratch():
    k = 4096
    qt = QTensor.quantize(torch.from_numpy(normal(930, (256, k), 0.02)).to(DEV), GgmlDType.Q4K)
    m = 16384  # GEMM planes alone: 16384 * 4096 int8 = 64 MiB, plus scales and sums
    assert int(L().qmm_matmul_workspace_size(qt.handle, m)) > (64 << 20)
    x = torch.zeros(1, device=DEV)  # never read: the size check comes first
    y = torch.zeros(1, device=DEV)
    rc = L().qmm_matmul_noalloc(qt.handle, x.data_ptr(), m, k, y.data_ptr(), 256, S())
    assert rc == qmm.QMM_ERR_INVALID and "QMM_NOALLOC_SCRATCH_BYTES" in qmm.last_error()


@pytest.mark.parametrize("m", [1, 64])
def test_noalloc_under_stream_capture(m):
    k, n = 4096, 1024
    qt = QTensor.quantize(torch.from_numpy(normal(940 + m, (n, k), 0.02)).to(DEV), GgmlDType.Q4K)
    x = torch.from_numpy(normal(950 + m, (m, k))).to(DEV)
    y = torch.empty((m, n), device=DEV)
    want = with_ws(qt, x, m)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        noalloc(qt, x, m, y)  # warm-up outside the capture (kernel lookups)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            qmm._check(L().qmm_matmul_noalloc(qt.handle, x.data_ptr(), m, k, y.data_ptr(), n,
                                              ctypes.c_void_p(s.cuda_stream)))
    torch.cuda.synchronize()
    for rep in range(4):
        y.fill_(float("nan"))
        with_ws(qt, x[:1].contiguous(), 1)  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), rep
