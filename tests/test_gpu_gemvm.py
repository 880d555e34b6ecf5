"""The multi-token GEMV on the int8 matrix cores (qmm_gemv_rowsm_q4k for 2..8 staged rows of a dense Q4_K
weight, qmm_moe_gemvm_q4k for the MoE expert GEMV): the reference's mmvq at batch 2..8
(mmvq_gguf.cu:725-807) and its MoE expert GEMV.

One v_mfma_i32_16x16x64_i8 takes 16 token rows against 16 weight rows; the sub-block scales are split
into the weight operand (sc = 8 sh + sl) and the mins term is two more MFMAs over the activation sums, so
every block's integers are the one-row kernels' and only the f32 order of the block sum differs (blocks in
order per output instead of the lane tree). Checked here:
* against the CPU oracle (k_quants::matmul) within 1e-3 of the output rms, and against the
  token-interleaved VALU kernels (QMM_GEMVM=0) within 1e-5, at 2, 5, 6 and 8 rows, with and without
  accumulation, row counts that are not a multiple of 16 and a K of 20 super-blocks;
* the default policy takes it at 6..8 rows of a weight of >= 8192 rows (equal, bit for bit, to the forced
  run) and not below (equal to the VALU kernel);
* the MoE expert GEMV: experts with more than 16 tokens (several passes), a single expert holding every
  token, idle experts, and the default policy at six or more pairs per expert; qmm_moe_ffn end to end
  against oracle/moe.py at 48 tokens.
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
vp = ctypes.c_void_p


def L():
    return qmm.lib()


def t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / np.sqrt((want ** 2).mean()))


def matmul_q(qt, xq, m, n, y0=None):
    y = y0.clone() if y0 is not None else torch.full((m, n), float("nan"), device=DEV)
    qmm._check(L().qmm_matmul_q_ex(qt.handle, xq.data_ptr(), m, y.data_ptr(), n, int(y0 is not None), None, 0,
                                   qmm._stream(DEV)))
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("n,k", [(14336, 4096), (8200, 4096), (1000, 5120)])
@pytest.mark.parametrize("m", [2, 5, 6, 8])
@pytest.mark.parametrize("acc", [False, True])
def test_rows_mfma_matches_oracle_and_valu_kernel(monkeypatch, n, k, m, acc):
    rng = np.random.default_rng(n + k + 10 * m + int(acc))
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    wq = orc.quantize(orc.Q4K, w)
    qt = QTensor.from_ggml(wq, GgmlDType.Q4K, (n, k), device=DEV)
    xq = t(orc.quantize(orc.Q8K, x), torch.uint8)
    y0 = t(rng.standard_normal((m, n)).astype(np.float32)) if acc else None
    monkeypatch.setenv("QMM_GEMVM", "1")
    got = matmul_q(qt, xq, m, n, y0)
    got2 = matmul_q(qt, xq, m, n, y0)
    assert torch.equal(got, got2)  # deterministic
    monkeypatch.setenv("QMM_GEMVM", "0")
    valu = matmul_q(qt, xq, m, n, y0)
    assert rel_err(got.cpu().numpy(), valu.cpu().numpy()) <= 1e-5
    want = orc.matmul(orc.Q4K, x, wq, k)
    if acc:
        want = want + y0.cpu().numpy()
    assert rel_err(got.cpu().numpy(), want) <= TOL
    assert not torch.isnan(got).any()


@pytest.mark.parametrize("m", [4, 6, 8])
def test_rows_default_policy(monkeypatch, m):
    rng = np.random.default_rng(77 + m)
    n, k = 14336, 4096
    qt = QTensor.quantize(t(rng.standard_normal((n, k)) * 0.02), GgmlDType.Q4K)
    xq = t(orc.quantize(orc.Q8K, rng.standard_normal((m, k)).astype(np.float32)), torch.uint8)
    monkeypatch.delenv("QMM_GEMVM", raising=False)
    default = matmul_q(qt, xq, m, n)
    monkeypatch.setenv("QMM_GEMVM", "1" if m >= 6 else "0")
    assert torch.equal(default, matmul_q(qt, xq, m, n))


def _moe_gemv(qts, E, xq, P, counts, offsets, F):
    ys = [torch.full((P, F), float("nan"), device=DEV) for _ in qts]
    qmm._check(L().qmm_moe_gemv((vp * len(qts))(*[q.handle.value for q in qts]), len(qts), E, xq.data_ptr(), P,
                                counts.data_ptr(), offsets.data_ptr(), (vp * len(qts))(*[y.data_ptr() for y in ys]),
                                qmm._stream(DEV)))
    torch.cuda.synchronize()
    return ys


@pytest.mark.parametrize("K", [4096, 5120])
@pytest.mark.parametrize("skew", [False, True, "single"])
def test_moe_mfma_gemv(monkeypatch, K, skew):
    """gate | up expert GEMV over 40 tokens: the matrix-core kernel against the ring kernel (1e-5) and each
    expert's oracle matmul (1e-3); skew routes every token to experts 0 and 1 (40 tokens each: three
    passes of 16), single (top-1) sends all of them to expert 3."""
    from inference_amd import moe_route
    E, F, T = 6, 776, 40
    k = 1 if skew == "single" else 2
    rng = np.random.default_rng(K + 3 * (2 if skew == "single" else int(skew)))
    ws = [(rng.standard_normal((E * F, K)) * 0.02).astype(np.float32) for _ in range(2)]
    raws = [orc.quantize(orc.Q4K, w).reshape(-1) for w in ws]
    qts = [QTensor.from_ggml(r, GgmlDType.Q4K, (E * F, K), device=DEV) for r in raws]
    logits = rng.standard_normal((T, E)).astype(np.float32)
    if skew == "single":
        logits[:, 3] += 10.0
    elif skew:
        logits[:, :2] += 10.0
    counts, offsets, ptok, pw, tp = moe_route(t(logits), k)
    P = T * k
    xg_np = rng.standard_normal((T, K)).astype(np.float32)[ptok.cpu().numpy()]
    xq_np = orc.quantize(orc.Q8K, xg_np)
    xq = t(xq_np, torch.uint8)
    monkeypatch.setenv("QMM_GEMVM", "1")
    got = _moe_gemv(qts, E, xq, P, counts, offsets, F)
    monkeypatch.setenv("QMM_GEMVM", "0")
    ref = _moe_gemv(qts, E, xq, P, counts, offsets, F)
    c, o = counts.cpu().numpy(), offsets.cpu().numpy()
    per = raws[0].size // E
    for j in range(2):
        assert not torch.isnan(got[j]).any()
        assert rel_err(got[j].cpu().numpy(), ref[j].cpu().numpy()) <= 1e-5
        for e in range(E):
            if c[e] == 0:
                continue
            want = orc.matmul(orc.Q4K, xg_np[o[e]:o[e] + c[e]], raws[j][e * per:(e + 1) * per], K)
            assert rel_err(got[j][o[e]:o[e] + c[e]].cpu().numpy(), want) <= TOL, (j, e)
    if skew == "single":
        assert int(c[3]) == T
    elif skew:
        assert int(c[0]) == T and int(c[1]) == T


def test_moe_ffn_many_tokens_matches_oracle(monkeypatch):
    """48 tokens, top-2 over 8 experts (12 pairs per expert: the default policy's matrix-core expert GEMV
    for gate / up, the ring kernel for the Q6_K down): qmm_moe_ffn against oracle/moe.py, and within 1e-3
    of the run with QMM_GEMVM=0 (the f32 order of gate / up can move a SiLU*mul requantization step)."""
    from inference_amd import moe_ffn
    from oracle import moe
    E, H, F, T, k = 8, 1024, 1536, 48, 2
    rng = np.random.default_rng(4848)
    raws = {}
    qts = {}
    for name, rows, cols, dt, od in (("gate", F, H, GgmlDType.Q4K, orc.Q4K), ("up", F, H, GgmlDType.Q4K, orc.Q4K),
                                     ("down", H, F, GgmlDType.Q6K, orc.Q6K)):
        r = orc.quantize(od, (rng.standard_normal((E * rows, cols)) * 0.02).astype(np.float32)).reshape(-1)
        qts[name] = QTensor.from_ggml(r, dt, (E * rows, cols), device=DEV)
        per = r.size // E
        raws[name] = [r[e * per:(e + 1) * per] for e in range(E)]
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    monkeypatch.delenv("QMM_GEMVM", raising=False)
    y = moe_ffn(t(x), t(logits), qts["gate"], qts["up"], qts["down"], k).cpu().numpy()
    monkeypatch.setenv("QMM_GEMVM", "0")
    y0 = moe_ffn(t(x), t(logits), qts["gate"], qts["up"], qts["down"], k).cpu().numpy()
    y_ref = moe.moe_ffn(x, logits, raws["gate"], raws["up"], raws["down"], orc.Q4K, orc.Q6K, k)
    for got in (y, y0):
        cos = float((got * y_ref).sum() / np.sqrt((got * got).sum() * (y_ref * y_ref).sum()))
        assert cos >= 0.99999 and rel_err(got, y_ref) <= 1e-2, (cos, rel_err(got, y_ref))
