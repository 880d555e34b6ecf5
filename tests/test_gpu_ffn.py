"""The prefill's fused entry points against the launches they replace (and qmm_ffn against the CPU oracle):
qmm_ffn, the gated feed-forward block of m rows, and qmm_qkv_rope_kv_append_n, q / k / v with RoPE and the
KV append.

At m > 8 the entry point sums the gate / up GEMMs' split-K partials inside its SiLU launch, in the
order qmm_splitk_sum uses (or, where gate and up would each be split, runs both as one unsplit launch, as
qmm_matmul_ex does for the same pair), so its output must equal qmm_matmul_ex (gate, up) -> qmm_silu_mul ->
qmm_matmul_ex (down, accumulate) bit for bit; at m <= 8 it runs the GEMV calls themselves. The
oracle check holds the f32 result to max|d| <= 1e-3 * rms.
"""
import ctypes

import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, QTensor, qmm
from inference_amd.llama_decode import LlamaConfig, rope_tables
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


def device_rms_norm(x, nw):
    """The device's RMSNorm rows (qmm_rms_norm, which the GEMMs' fused norm prologue equals bit for bit), so
    that the oracle quantizes the very f32 values the device did: a last-bit difference of the norm that
    lands on a Q8_K rounding tie would otherwise move one activation code (up to ~2e-3 of the rms)."""
    m, k = x.shape
    xd, nwd, out = t(x), t(nw), torch.empty((m, k), device=DEV)
    qmm._check(L().qmm_rms_norm(xd.data_ptr(), m, k, k, nwd.data_ptr(), ctypes.c_float(1e-5), out.data_ptr(), k,
                                S()))
    torch.cuda.synchronize()
    return out.cpu().numpy()


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


@pytest.mark.parametrize("m", [127, 64, 24])
def test_gate_up_pair_equals_unsplit_launches(monkeypatch, m):
    """Gate and up at 8B shape and m rows (each alone split over K) run as one launch over both weights
    (grid z = weight), unsplit: bit-identical to one unsplit launch per weight (QMM_SPLITK=1,
    QMM_FFN_SEPARATE=1), here with the residual add and output strides wider than the rows, and within
    1e-3 * rms of the oracle. Also the split launches (QMM_FFN_SEPARATE=1) hold the same bar."""
    H, F = 4096, 14336
    gate, up, _ = make(H, F, 7)
    rng = np.random.default_rng(300 + m)
    x = rng.standard_normal((m, H)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, H).astype(np.float32)
    r0 = rng.standard_normal((m, F)).astype(np.float32)
    r1 = rng.standard_normal((m, F)).astype(np.float32)
    ld0, ld1 = F + 64, F + 320

    def run():
        y0 = torch.full((m, ld0), float("nan"), device=DEV)
        y1 = torch.full((m, ld1), float("nan"), device=DEV)
        y0[:, :F], y1[:, :F] = t(r0), t(r1)
        wsb = max(int(L().qmm_matmul_ex_workspace_size(q.handle, m, 1)) for q in (gate, up))
        ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
        xd, nwd = t(x), t(nw)
        qmm._check(L().qmm_matmul_ex((vp * 2)(gate.handle.value, up.handle.value), 2, xd.data_ptr(), m, H,
                                     nwd.data_ptr(), ctypes.c_float(1e-5), 1, (vp * 2)(y0.data_ptr(), y1.data_ptr()),
                                     (i64 * 2)(ld0, ld1), ws.data_ptr(), wsb, S()))
        torch.cuda.synchronize()
        assert torch.isnan(y0[:, F:]).all() and torch.isnan(y1[:, F:]).all()  # the stride gaps untouched
        return y0[:, :F].cpu().numpy(), y1[:, :F].cpu().numpy()

    got = run()
    monkeypatch.setenv("QMM_FFN_SEPARATE", "1")
    split = run()
    monkeypatch.setenv("QMM_SPLITK", "1")
    unsplit = run()
    for a, b in zip(got, unsplit):
        assert np.array_equal(a, b)
    xin = device_rms_norm(x, nw)
    for q, r, a, b in zip((gate, up), (r0, r1), got, split):
        want = r + orc.matmul(orc.Q4K, xin, q.to_ggml(), H)
        assert rel_err(a, want) <= TOL and rel_err(b, want) <= TOL


@pytest.mark.parametrize("m", [257, 127, 64, 24, 9])
@pytest.mark.parametrize("kinds", ["q4k_q4k_q6k", "q4k_q4k"])
def test_multi_weight_launch_matches_separate_launches(monkeypatch, m, kinds):
    """q / k / v of the 8B shape (4096, 1024, 1024 rows of 4096; v Q6_K) through qmm_matmul_ex at m rows: one
    launch over all weights with jointly chosen split counts (qmm_mmqs_multi), then a split sum per weight,
    with the residual add. Against one launch per weight (QMM_QKV_SEPARATE=1: each with its own split count)
    within 1e-5 * rms (the split sums' f32 order), and against the oracle within 1e-3 * rms. 257 rows take
    three row tiles per weight, 9 the smallest GEMM."""
    H = 4096
    dts = [GgmlDType.Q4K, GgmlDType.Q4K, GgmlDType.Q6K][:len(kinds.split("_"))]
    rows = [4096, 1024, 1024][:len(dts)]
    g = torch.Generator(device=DEV).manual_seed(400 + m)
    qts = [QTensor.quantize(torch.randn((n, H), generator=g, device=DEV) * 0.02, dt) for n, dt in zip(rows, dts)]
    rng = np.random.default_rng(410 + m)
    x = rng.standard_normal((m, H)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, H).astype(np.float32)
    r0 = [rng.standard_normal((m, n)).astype(np.float32) for n in rows]

    def run():
        ys = [t(r) for r in r0]
        wsb = max(int(L().qmm_matmul_ex_workspace_size(q.handle, m, 1)) for q in qts)
        ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
        xd, nwd = t(x), t(nw)
        qmm._check(L().qmm_matmul_ex((vp * len(qts))(*[q.handle.value for q in qts]), len(qts), xd.data_ptr(), m, H,
                                     nwd.data_ptr(), ctypes.c_float(1e-5), 1,
                                     (vp * len(qts))(*[y.data_ptr() for y in ys]), (i64 * len(qts))(*rows),
                                     ws.data_ptr(), wsb, S()))
        torch.cuda.synchronize()
        return [y.cpu().numpy() for y in ys]

    got = run()
    monkeypatch.setenv("QMM_QKV_SEPARATE", "1")
    sep = run()
    xin = device_rms_norm(x, nw)
    for q, dt, r, a, b in zip(qts, dts, r0, got, sep):
        want = r + orc.matmul(orc.Q4K if dt == GgmlDType.Q4K else orc.Q6K, xin, q.to_ggml(), H)
        assert rel_err(a, b) <= 1e-5
        assert rel_err(a, want) <= TOL and rel_err(b, want) <= TOL


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


@pytest.mark.parametrize("m,first", [(127, 0), (64, 5), (9, 0), (8, 0), (3, 7)])
def test_qkv_rope_equals_the_launches_it_replaces(m, first):
    """The 8B attention projections (q 4096x4096 and k 1024x4096 Q4_K, v 1024x4096 Q6_K; 32 / 8 heads of
    128) on the GEMM path (127, 64, 9 rows: q, k and v split over K) and the GEMV path (8, 3): rotated q
    and both caches equal qmm_matmul_ex followed by qmm_rope_kv_append_n bit for bit."""
    H, heads, kvh, hd, max_seq = 4096, 32, 8, 128, 256
    g = torch.Generator(device=DEV).manual_seed(11)
    wq = QTensor.quantize(torch.randn((heads * hd, H), generator=g, device=DEV) * 0.02, GgmlDType.Q4K)
    wk = QTensor.quantize(torch.randn((kvh * hd, H), generator=g, device=DEV) * 0.02, GgmlDType.Q4K)
    wv = QTensor.quantize(torch.randn((kvh * hd, H), generator=g, device=DEV) * 0.02, GgmlDType.Q6K)
    cos, sin = (t(a) for a in rope_tables(LlamaConfig.llama3_8b(), max_seq))
    rng = np.random.default_rng(200 + m)
    x = t(rng.standard_normal((m, H)).astype(np.float32))
    nw = t(rng.uniform(0.5, 1.5, H).astype(np.float32))
    eps = ctypes.c_float(1e-5)
    nq, nkv = heads * hd, kvh * hd
    caches = [torch.full((kvh, max_seq, hd), 7.0, device=DEV) for _ in range(4)]
    q1 = torch.zeros((m, nq), device=DEV)
    wsb = int(L().qmm_qkv_rope_kv_append_n_workspace_size(wq.handle, wk.handle, wv.handle, m, 1))
    assert wsb > 0
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    qmm._check(L().qmm_qkv_rope_kv_append_n(wq.handle, wk.handle, wv.handle, x.data_ptr(), m, H, nw.data_ptr(), eps,
                                            cos.data_ptr(), sin.data_ptr(), first, q1.data_ptr(), nq,
                                            caches[0].data_ptr(), caches[1].data_ptr(), heads, kvh, hd, max_seq,
                                            ws.data_ptr(), ws.numel(), S()))
    q2 = torch.zeros((m, nq), device=DEV)
    k2 = torch.zeros((m, nkv), device=DEV)
    v2 = torch.zeros((m, nkv), device=DEV)
    wsb2 = max(int(L().qmm_matmul_ex_workspace_size(w.handle, m, 1)) for w in (wq, wk, wv))
    ws2 = torch.empty(wsb2, dtype=torch.uint8, device=DEV)
    qmm._check(L().qmm_matmul_ex((vp * 3)(wq.handle.value, wk.handle.value, wv.handle.value), 3, x.data_ptr(), m, H,
                                 nw.data_ptr(), eps, 0, (vp * 3)(q2.data_ptr(), k2.data_ptr(), v2.data_ptr()),
                                 (i64 * 3)(nq, nkv, nkv), ws2.data_ptr(), ws2.numel(), S()))
    qmm._check(L().qmm_rope_kv_append_n(q2.data_ptr(), k2.data_ptr(), v2.data_ptr(), nq, nkv, nkv, cos.data_ptr(),
                                        sin.data_ptr(), first, m, caches[2].data_ptr(), caches[3].data_ptr(), heads,
                                        kvh, hd, max_seq, S()))
    assert torch.equal(q1, q2)
    assert torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])
    # the positions outside [first, first + m) are untouched
    assert bool((caches[0][:, :first] == 7.0).all()) and bool((caches[0][:, first + m:] == 7.0).all())


def test_qkv_rope_rejects_bad_arguments():
    g = torch.Generator(device=DEV).manual_seed(12)
    wq = QTensor.quantize(torch.randn((256, 512), generator=g, device=DEV) * 0.02, GgmlDType.Q4K)
    wk = QTensor.quantize(torch.randn((128, 512), generator=g, device=DEV) * 0.02, GgmlDType.Q4K)
    x = torch.zeros((16, 512), device=DEV)
    cs = torch.zeros((32, 64), device=DEV)
    kc = torch.zeros((2, 32, 64), device=DEV)
    ws = torch.empty(1 << 22, dtype=torch.uint8, device=DEV)

    def call(heads, kvh, first, m=16, wv=wk):
        return L().qmm_qkv_rope_kv_append_n(wq.handle, wk.handle, wv.handle, x.data_ptr(), m, 512, None,
                                            ctypes.c_float(1e-5), cs.data_ptr(), cs.data_ptr(), first, x.data_ptr(),
                                            512, kc.data_ptr(), kc.data_ptr(), heads, kvh, 64, 32, ws.data_ptr(),
                                            ws.numel(), S())
    assert call(3, 2, 0) != 0     # heads % kv_heads
    assert call(4, 1, 0) != 0     # wk rows != kv_heads * head_dim
    assert call(4, 2, 20) != 0    # positions past max_seq
    wv8 = QTensor.quantize(torch.zeros((128, 512), device=DEV), GgmlDType.Q8_0)
    assert call(4, 2, 0, wv=wv8) != 0  # Q8_0 weight
    # the workspace query refuses what the weights alone rule out, as qmm_ffn_workspace_size does
    size = L().qmm_qkv_rope_kv_append_n_workspace_size
    assert size(wq.handle, wk.handle, wk.handle, 16, 1) > 0
    assert size(wq.handle, wk.handle, wv8.handle, 16, 1) == 0  # Q8_0 weight
    assert size(wq.handle, wk.handle, wq.handle, 16, 1) == 0   # k and v of different row counts
    assert size(wq.handle, wk.handle, wk.handle, 0, 1) == 0    # no rows

@pytest.mark.parametrize("m,heads,kv_heads,hd,dt", [(127, 32, 8, 128, GgmlDType.Q4K), (127, 32, 8, 128, GgmlDType.Q6K),
                                                    (24, 32, 8, 128, GgmlDType.Q4K), (9, 32, 8, 128, GgmlDType.Q4K),
                                                    (5, 32, 8, 128, GgmlDType.Q4K), (40, 8, 8, 128, GgmlDType.Q4K),
                                                    (33, 16, 4, 64, GgmlDType.Q6K)])
def test_prefill_attention_o_equals_the_two_calls(monkeypatch, m, heads, kv_heads, hd, dt):
    """qmm_prefill_attention_o (causal attention of m prompt rows, then o and the residual add) against
    qmm_prefill_attention followed by qmm_matmul_ex(o, accumulate), bit for bit: with the attention launch
    writing the o GEMM's Q8_K planes (m > 8, G * head_dim a multiple of 256: 32 / 8 heads of 128, 16 / 4 of
    64), and through the two calls themselves (m = 5: the GEMV; 8 / 8 heads: 128 outputs per kv head;
    QMM_ATTN_O_SEPARATE=1)."""
    H, max_seq, first = heads * hd, 160, 3
    g = torch.Generator(device=DEV).manual_seed(500 + m)
    wo = QTensor.quantize(torch.randn((4096, H), generator=g, device=DEV) * 0.02, dt)
    q = torch.randn((m, H), generator=g, device=DEV)
    kc = torch.randn((kv_heads, max_seq, hd), generator=g, device=DEV)
    vc = torch.randn((kv_heads, max_seq, hd), generator=g, device=DEV)
    x0 = torch.randn((m, 4096), generator=g, device=DEV)
    scale = ctypes.c_float(1.0 / np.sqrt(hd))

    def fused():
        x = x0.clone()
        wsb = int(L().qmm_prefill_attention_o_workspace_size(wo.handle, m))
        ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
        qmm._check(L().qmm_prefill_attention_o(q.data_ptr(), H, kc.data_ptr(), vc.data_ptr(), first, m, heads,
                                               kv_heads, hd, max_seq, scale, wo.handle, x.data_ptr(), 4096,
                                               ws.data_ptr(), wsb, S()))
        return x

    att = torch.empty((m, H), device=DEV)
    qmm._check(L().qmm_prefill_attention(q.data_ptr(), H, kc.data_ptr(), vc.data_ptr(), first, m, att.data_ptr(), H,
                                         heads, kv_heads, hd, max_seq, scale, S()))
    want = x0.clone()
    wsb = int(L().qmm_matmul_ex_workspace_size(wo.handle, m, 0))
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    qmm._check(L().qmm_matmul_ex((vp * 1)(wo.handle.value), 1, att.data_ptr(), m, H, None, ctypes.c_float(0), 1,
                                 (vp * 1)(want.data_ptr()), (i64 * 1)(4096), ws.data_ptr(), wsb, S()))
    assert torch.equal(fused(), want)
    monkeypatch.setenv("QMM_ATTN_O_SEPARATE", "1")
    assert torch.equal(fused(), want)


def test_prefill_attention_o_rejects_bad_arguments():
    g = torch.Generator(device=DEV).manual_seed(9)
    wo = QTensor.quantize(torch.randn((512, 1024), generator=g, device=DEV) * 0.02, GgmlDType.Q4K)
    t1 = torch.zeros(4096, device=DEV)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    with pytest.raises(qmm.QmmError):  # o weight's k (1024) != heads * head_dim (2048)
        qmm._check(L().qmm_prefill_attention_o(t1.data_ptr(), 2048, t1.data_ptr(), t1.data_ptr(), 0, 2, 16, 4, 128,
                                               64, ctypes.c_float(1.0), wo.handle, t1.data_ptr(), 512,
                                               ws.data_ptr(), ws.numel(), S()))
    with pytest.raises(qmm.QmmError):  # workspace too small
        qmm._check(L().qmm_prefill_attention_o(t1.data_ptr(), 1024, t1.data_ptr(), t1.data_ptr(), 0, 2, 8, 4, 128,
                                               64, ctypes.c_float(1.0), wo.handle, t1.data_ptr(), 512,
                                               ws.data_ptr(), 16, S()))
