"""Stream-K schedule of the Q4_K prefill GEMM (qmm_mmqs_q4k_sk, opt-in with QMM_STREAMK=1), the tile-count
remedy of the reference's MMQ launcher (mmq_gguf/mmq_instance_q4_k.cu:47-75, the fixup at
mmq_gguf.cuh:3442-3517).

A grid whose tile count is not a whole number of rounds over the CUs runs its whole rounds as data-parallel
tiles and the rest as equal (tile, K step) ranges per CU; the last workgroup to finish a split tile adds the
segments' partials in K order. Checked here:
* f32 outputs within 1e-3 * rms of the oracle's k_quants::matmul on a sample of rows, at shapes that give
  data-parallel rounds plus a stream-K remainder (512 x 14336 x 4096: 448 tiles), all stream-K (512 x 4096 x
  14336: 128 tiles of 56 K steps; 257 x 4096 x 4096), ragged edge tiles, and the remainder-plus-a-round rule
  (1000 x 9000 x 1024);
* the stream-K result equals the default plan's (QMM_STREAMK unset) within 1e-5 * rms: only the f32
  association of the K split differs;
* it is deterministic (two calls, and every replay of a captured graph, equal bit for bit), and accumulate
  adds to y.
"""
import ctypes

import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, QTensor, qmm
from inference_amd.synth import normal
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
vp, i64 = ctypes.c_void_p, ctypes.c_int64

SHAPES = [(512, 14336, 4096), (512, 4096, 14336), (257, 4096, 4096), (300, 2000, 8192), (1000, 9000, 1024)]


def rel_err(y, y_ref):
    y_ref = np.asarray(y_ref, dtype=np.float64)
    return float(np.abs(np.asarray(y, dtype=np.float64) - y_ref).max() / np.sqrt(np.mean(y_ref ** 2)))


def weight(n, k, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return QTensor.quantize(torch.randn((n, k), generator=g, device=DEV) * 0.02, GgmlDType.Q4K)


def matmul(qt, x, y=None, accumulate=0):
    m, k = x.shape
    n = qt.shape[0]
    y = torch.empty((m, n), device=DEV) if y is None else y
    wsb = int(qmm.lib().qmm_matmul_ex_workspace_size(qt.handle, m, 0))
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    qmm._check(qmm.lib().qmm_matmul_ex((vp * 1)(qt.handle.value), 1, x.data_ptr(), m, k, None, ctypes.c_float(0),
                                       accumulate, (vp * 1)(y.data_ptr()), (i64 * 1)(n), ws.data_ptr(), wsb,
                                       qmm._stream(DEV)))
    return y


@pytest.fixture
def streamk(monkeypatch):
    monkeypatch.setenv("QMM_STREAMK", "1")
    return monkeypatch


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_streamk_matches_oracle_and_plain_grid(m, n, k, streamk):
    qt = weight(n, k, 40 + m)
    xh = normal(41 + n, (m, k))
    x = torch.from_numpy(xh).to(DEV)
    with_sk = int(qmm.lib().qmm_matmul_workspace_size(qt.handle, m))
    y = matmul(qt, x)
    y2 = matmul(qt, x)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    rows = np.unique(np.linspace(0, m - 1, 16).astype(int))
    ref = orc.matmul(orc.Q4K, np.ascontiguousarray(xh[rows]), qt.to_ggml(), k)
    assert rel_err(y.cpu().numpy()[rows], ref) <= 1e-3
    streamk.delenv("QMM_STREAMK")
    assert int(qmm.lib().qmm_matmul_workspace_size(qt.handle, m)) != with_sk  # the plan did change
    yp = matmul(qt, x)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), yp.cpu().numpy()) <= 1e-5


def test_streamk_accumulates(streamk):
    m, n, k = 512, 4096, 14336
    qt = weight(n, k, 77)
    x = torch.from_numpy(normal(78, (m, k))).to(DEV)
    y0 = torch.from_numpy(normal(79, (m, n))).to(DEV)
    y = matmul(qt, x, y0.clone(), accumulate=1)
    plain = matmul(qt, x)
    torch.cuda.synchronize()
    assert rel_err((y - y0).cpu().numpy(), plain.cpu().numpy()) <= 1e-5


def test_streamk_graph_replays_equal_eager(streamk):
    """The counters are cleared by a kernel inside the call, so every replay of a captured call starts from
    zeros: between the replays the workspace is filled with 0xff bytes and an eager GEMM of another shape runs."""
    m, n, k = 512, 14336, 4096
    qt = weight(n, k, 88)
    other = weight(4096, 14336, 89)
    x = torch.from_numpy(normal(90, (m, k))).to(DEV)
    xo = torch.from_numpy(normal(91, (m, 14336))).to(DEV)
    want = matmul(qt, x)
    y = torch.empty((m, n), device=DEV)
    wsb = int(qmm.lib().qmm_matmul_ex_workspace_size(qt.handle, m, 0))
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()

    def call(stream):
        qmm._check(qmm.lib().qmm_matmul_ex((vp * 1)(qt.handle.value), 1, x.data_ptr(), m, k, None,
                                           ctypes.c_float(0), 0, (vp * 1)(y.data_ptr()), (i64 * 1)(n),
                                           ws.data_ptr(), wsb, stream))
    with torch.cuda.stream(s):
        call(ctypes.c_void_p(s.cuda_stream))
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            call(ctypes.c_void_p(s.cuda_stream))
    torch.cuda.synchronize()
    for _ in range(4):
        y.fill_(float("nan"))
        ws.fill_(255)
        matmul(other, xo)  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)


def test_streamk_inside_ffn_and_qkv(streamk):
    """The fused prefill entry points take the same plan: with stream-K on, qmm_ffn (gate / up through the
    stream-K scratch, down through qmm_matmul's path) and qmm_qkv_rope_kv_append_n (q stream-K, k / v split)
    still equal the launches they replace bit for bit."""
    import test_gpu_ffn as f
    f.test_ffn_equals_the_launches_it_replaces(512)
    f.test_qkv_rope_equals_the_launches_it_replaces(200, 0)
