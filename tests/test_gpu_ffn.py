"""qmm_ffn (the gated feed-forward block of m rows) against the launches it replaces and the CPU oracle.

At m > 8 the entry point sums the gate / up GEMMs' split-K partials inside its SiLU launch, in the
order qmm_splitk_sum uses, so its output must equal qmm_matmul_ex (gate, up) -> qmm_silu_mul ->
qmm_matmul_ex (down, accumulate) bit for bit; at m <= 8 it runs the GEMV calls themselves. The
oracle check holds the f32 result to max|d| <= 1e-3 * rms.
"""
import ctypes

import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, QTensor, qmm
from oracle import llama as ol
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 1e-3
vp, i64 = ctypes.c_void_p, ctypes.c_int64


def L():
    return qmm.lib()


def S():
    return qmm._stream(DEV)


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, torch.float32)


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / np.sqrt((want ** 2).mean()))


def make(H, F, seed, gdt=GgmlDType.Q4K, ddt=GgmlDType.Q6K):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = {name: torch.randn(shape, generator=g, device=DEV) * 0.02
         for name, shape in (("gate", (F, H)), ("up", (F, H)), ("down", (H, F)))}
    return (QTensor.quantize(w["gate"], gdt), QTensor.quantize(w["up"], gdt), QTensor.quantize(w["down"], ddt))


def ffn(gate, up, down, x, m, nw, y, accumulate=1):
    H = gate.shape[1]
    wsb = int(L().qmm_ffn_workspace_size(gate.handle, up.handle, down.handle, m, 1 if nw is not None else 0))
    assert wsb > 0
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    qmm._check(L().qmm_ffn(gate.handle, up.handle, down.handle, x.data_ptr(), m, H,
                           nw.data_ptr() if nw is not None else None, ctypes.c_float(1e-5), accumulate, y.data_ptr(),
                           H, ws.data_ptr(), ws.numel(), S()))


def chain(gate, up, down, x, m, nw, y):
    """The three calls qmm_ffn replaces (the batched prefill's traced path)."""
    F, H = gate.shape
    g = torch.empty((m, F), device=DEV)
    u = torch.empty((m, F), device=DEV)
    h = torch.empty((m, F), device=DEV)
    wsb = max(int(L().qmm_matmul_ex_workspace_size(q.handle, m, 1)) for q in (gate, up, down))
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    eps = ctypes.c_float(1e-5)
    qmm._check(L().qmm_matmul_ex((vp * 2)(gate.handle.value, up.handle.value), 2, x.data_ptr(), m, H,
                                 nw.data_ptr() if nw is not None else None, eps, 0,
                                 (vp * 2)(g.data_ptr(), u.data_ptr()), (i64 * 2)(F, F), ws.data_ptr(), ws.numel(),
                                 S()))
    qmm._check(L().qmm_silu_mul(g.data_ptr(), u.data_ptr(), h.data_ptr(), m * F, S()))
    qmm._check(L().qmm_matmul_ex((vp * 1)(down.handle.value), 1, h.data_ptr(), m, F, None, eps, 1,
                                 (vp * 1)(y.data_ptr()), (i64 * 1)(H), ws.data_ptr(), ws.numel(), S()))


@pytest.mark.parametrize("m", [127, 64, 9, 8, 3, 1])
def test_ffn_equals_the_launches_it_replaces(m):
    """The 8B FFN shape (gate / up 14336x4096 Q4_K, down 4096x14336 Q6_K) on the GEMM path (127 rows: the
    batched prefill's, gate / up split over K; 64, 9) and the GEMV path (8, 3, 1)."""
    H, F = 4096, 14336
    gate, up, down = make(H, F, 5)
    rng = np.random.default_rng(m)
    x = t(rng.standard_normal((m, H)).astype(np.float32))
    nw = t(rng.uniform(0.5, 1.5, H).astype(np.float32))
    res = t(rng.standard_normal((m, H)).astype(np.float32))
    y1, y2 = res.clone(), res.clone()
    ffn(gate, up, down, x, m, nw, y1)
    chain(gate, up, down, x, m, nw, y2)
    assert torch.equal(y1, y2)
    # in place on the residual stream (y = x), as the prefill calls it
    x3 = x.clone()
    ffn(gate, up, down, x3, m, nw, x3)
    y4 = x.clone()
    chain(gate, up, down, x, m, nw, y4)
    assert torch.equal(x3, y4)


@pytest.mark.parametrize("m,norm", [(40, True), (12, False), (5, True)])
def test_ffn_matches_oracle(m, norm):
    H, F = 512, 1536
    gate, up, down = make(H, F, 7, gdt=GgmlDType.Q6K, ddt=GgmlDType.Q4K)
    rng = np.random.default_rng(100 + m)
    x = rng.standard_normal((m, H)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, H).astype(np.float32)
    y = torch.zeros((m, H), device=DEV)
    ffn(gate, up, down, t(x), m, t(nw) if norm else None, y, accumulate=0)
    n = ol.rms_norm(x, nw, 1e-5) if norm else x
    gb, ub, db = gate.to_ggml(), up.to_ggml(), down.to_ggml()
    hmid = (ol.silu(orc.matmul(orc.Q6K, n, gb, H)) * orc.matmul(orc.Q6K, n, ub, H)).astype(np.float32)
    want = orc.matmul(orc.Q4K, hmid, db, F)
    assert rel_err(y.cpu().numpy(), want) <= TOL


def test_ffn_rejects_bad_shapes_and_formats():
    gate, up, down = make(512, 1024, 9)
    wrong = QTensor.quantize(torch.zeros((512, 512), device=DEV), GgmlDType.Q4K)
    q80 = QTensor.quantize(torch.zeros((1024, 512), device=DEV), GgmlDType.Q8_0)
    assert int(L().qmm_ffn_workspace_size(gate.handle, up.handle, wrong.handle, 16, 1)) == 0
    assert int(L().qmm_ffn_workspace_size(q80.handle, q80.handle, down.handle, 16, 1)) == 0
    x = torch.zeros((16, 512), device=DEV)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    with pytest.raises(qmm.QmmError):
        qmm._check(L().qmm_ffn(gate.handle, up.handle, wrong.handle, x.data_ptr(), 16, 512, None,
                               ctypes.c_float(1e-5), 0, x.data_ptr(), 512, ws.data_ptr(), ws.numel(), S()))
    need = int(L().qmm_ffn_workspace_size(gate.handle, up.handle, down.handle, 16, 0))
    with pytest.raises(qmm.QmmError, match="workspace"):
        qmm._check(L().qmm_ffn(gate.handle, up.handle, down.handle, x.data_ptr(), 16, 512, None,
                               ctypes.c_float(1e-5), 0, x.data_ptr(), 512, ws.data_ptr(), need - 1, S()))
