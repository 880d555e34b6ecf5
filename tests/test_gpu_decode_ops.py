"""Each decode-step launch of the C-ABI against the CPU decode oracle, one op at a time.

Non-matmul ops are f32 like the reference's decode path and are held to a
few ulp-scale tolerances stated per test; matmuls (with the RMSNorm prologue
or the accumulate epilogue) to max|d| <= 1e-3 * rms.
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


def L():
    return qmm.lib()


def S():
    return qmm._stream(DEV)


def t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / np.sqrt((want ** 2).mean()))


def test_rms_norm_kernel():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((3, 4096)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    xd, wd, out = t(x), t(w), torch.zeros((3, 4096), device=DEV)
    qmm._check(L().qmm_rms_norm(xd.data_ptr(), 3, 4096, 4096, wd.data_ptr(), ctypes.c_float(1e-5), out.data_ptr(),
                                4096, S()))
    np.testing.assert_allclose(out.cpu().numpy(), ol.rms_norm(x, w, 1e-5), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("dt", [GgmlDType.Q4K, GgmlDType.Q6K])
@pytest.mark.parametrize("m", [1, 2, 5])
def test_matmul_ex_rms_norm_prologue(dt, m):
    rng = np.random.default_rng(10 + m)
    n, k = 640, 4096
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    qt = QTensor.quantize(t(w), dt)
    x = (rng.standard_normal((m, k)) * 0.05).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, k).astype(np.float32)
    xd, nwd = t(x), t(nw)
    y = torch.zeros((m, n), device=DEV)
    wsb = int(L().qmm_matmul_ex_workspace_size(qt.handle, m, 1))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    hs = (ctypes.c_void_p * 1)(qt.handle.value)
    ys = (ctypes.c_void_p * 1)(y.data_ptr())
    lds = (ctypes.c_int64 * 1)(n)
    qmm._check(L().qmm_matmul_ex(hs, 1, xd.data_ptr(), m, k, nwd.data_ptr(), ctypes.c_float(1e-5), 0, ys, lds,
                                 ws.data_ptr(), wsb, S()))
    want = orc.matmul(int(dt), ol.rms_norm(x, nw, 1e-5), qt.to_ggml(), k)
    assert rel_err(y.cpu().numpy(), want) <= 1e-3


MIXES = [(GgmlDType.Q4K, GgmlDType.Q4K, GgmlDType.Q6K), (GgmlDType.Q6K, GgmlDType.Q4K),
         (GgmlDType.Q4K, GgmlDType.Q6K, GgmlDType.Q4K, GgmlDType.Q6K, GgmlDType.Q4K)]


@pytest.mark.parametrize("dts", MIXES)
@pytest.mark.parametrize("m", [1, 2, 5, 64])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("k", [4096, 20480])
def test_matmul_ex_mixed_q4k_q6k_equals_separate_calls(monkeypatch, dts, m, norm, k):
    """Q4_K and Q6_K weights in one qmm_matmul_ex call (one mixed launch at m = 1; per-format launches
    over one shared RMSNorm and Q8_K quantization otherwise: GGML rows at m = 5, GEMM planes at m = 64):
    bit-identical to one call per weight. k = 20480 takes the long-row prologue. At m = 64 two or three
    weights that would each be split over K run as one launch with split counts chosen together
    (qmm_mmqs_multi), so there the call equals one call per weight within 1e-5 * rms (the order of the split
    sums), and bit for bit with QMM_QKV_SEPARATE=1 (one launch per weight)."""
    joint = m > 8 and len(dts) <= 3
    if joint:
        monkeypatch.setenv("QMM_QKV_SEPARATE", "1")
    rng = np.random.default_rng(40 + m + len(dts))
    rows = [700, 256, 300, 1000, 33][:len(dts)]
    qts = [QTensor.quantize(t((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), dt)
           for n, dt in zip(rows, dts)]
    x = t((rng.standard_normal((m, k)) * 0.5).astype(np.float32))
    nw = t(rng.uniform(0.5, 1.5, k).astype(np.float32)) if norm else None
    nwp = nw.data_ptr() if norm else None
    wsb = max(int(L().qmm_matmul_ex_workspace_size(q.handle, m, int(norm))) for q in qts)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    ys = [torch.full((m, n), float("nan"), device=DEV) for n in rows]
    qmm._check(L().qmm_matmul_ex((vp * len(qts))(*[q.handle.value for q in qts]), len(qts), x.data_ptr(), m, k, nwp,
                                 ctypes.c_float(1e-5), 0, (vp * len(qts))(*[y.data_ptr() for y in ys]),
                                 (i64 * len(qts))(*rows), ws.data_ptr(), wsb, S()))
    for q, n, y in zip(qts, rows, ys):
        want = torch.full((m, n), float("nan"), device=DEV)
        qmm._check(L().qmm_matmul_ex((vp * 1)(q.handle.value), 1, x.data_ptr(), m, k, nwp, ctypes.c_float(1e-5), 0,
                                     (vp * 1)(want.data_ptr()), (i64 * 1)(n), ws.data_ptr(), wsb, S()))
        assert torch.equal(y, want)
    if joint:
        monkeypatch.delenv("QMM_QKV_SEPARATE")
        yj = [torch.full((m, n), float("nan"), device=DEV) for n in rows]
        qmm._check(L().qmm_matmul_ex((vp * len(qts))(*[q.handle.value for q in qts]), len(qts), x.data_ptr(), m, k,
                                     nwp, ctypes.c_float(1e-5), 0, (vp * len(qts))(*[y.data_ptr() for y in yj]),
                                     (i64 * len(qts))(*rows), ws.data_ptr(), wsb, S()))
        for a, b in zip(yj, ys):
            assert rel_err(a.cpu().numpy(), b.cpu().numpy()) <= 1e-5


@pytest.mark.parametrize("m", [1, 3])
def test_matmul_multi_q_mixed_q4k_q6k(m):
    """Pre-quantized Q8_K activation shared by Q4_K and Q6_K weights: bit-identical to qmm_matmul_q."""
    rng = np.random.default_rng(50 + m)
    k, rows, dts = 2048, [513, 1024, 77], [GgmlDType.Q6K, GgmlDType.Q4K, GgmlDType.Q6K]
    qts = [QTensor.quantize(t((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), dt)
           for n, dt in zip(rows, dts)]
    xq = t(orc.quantize(orc.Q8K, rng.standard_normal((m, k)).astype(np.float32)), torch.uint8)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    ys = [torch.full((m, n), float("nan"), device=DEV) for n in rows]
    qmm._check(L().qmm_matmul_multi_q((vp * 3)(*[q.handle.value for q in qts]), 3, xq.data_ptr(), m,
                                      (vp * 3)(*[y.data_ptr() for y in ys]), (i64 * 3)(*rows), None, 0, S()))
    for q, n, y in zip(qts, rows, ys):
        want = torch.full((m, n), float("nan"), device=DEV)
        qmm._check(L().qmm_matmul_q(q.handle, xq.data_ptr(), m, want.data_ptr(), n, None, 0, S()))
        assert torch.equal(y, want)


def test_mixed_formats_other_than_k_quants_are_rejected():
    rng = np.random.default_rng(60)
    k = 1024
    a = QTensor.quantize(t((rng.standard_normal((64, k)) * 0.02).astype(np.float32)), GgmlDType.Q4K)
    b = QTensor.quantize(t((rng.standard_normal((64, k)) * 0.02).astype(np.float32)), GgmlDType.Q8_0)
    x = t(rng.standard_normal((1, k)).astype(np.float32))
    y = torch.zeros((2, 64), device=DEV)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    rc = L().qmm_matmul_ex((vp * 2)(a.handle.value, b.handle.value), 2, x.data_ptr(), 1, k, None, ctypes.c_float(0), 0,
                           (vp * 2)(y.data_ptr(), y.data_ptr() + 256), (i64 * 2)(64, 64), None, 0, S())
    assert rc == 1 and "Q4_K/Q6_K" in qmm.last_error()


@pytest.mark.parametrize("m", [1, 2, 12])
def test_matmul_ex_accumulate(m):
    rng = np.random.default_rng(20 + m)
    n, k = 384, 1024
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    qt = QTensor.quantize(t(w), GgmlDType.Q4K)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    xd, y = t(x), t(y0)
    wsb = int(L().qmm_matmul_ex_workspace_size(qt.handle, m, 0))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    hs = (ctypes.c_void_p * 1)(qt.handle.value)
    ys = (ctypes.c_void_p * 1)(y.data_ptr())
    lds = (ctypes.c_int64 * 1)(n)
    qmm._check(L().qmm_matmul_ex(hs, 1, xd.data_ptr(), m, k, None, ctypes.c_float(0), 1, ys, lds, ws.data_ptr(),
                                 wsb, S()))
    prod = orc.matmul(orc.Q4K, x, qt.to_ggml(), k)
    assert rel_err(y.cpu().numpy() - y0, prod) <= 1e-3
    np.testing.assert_allclose(y.cpu().numpy(), y0 + prod, rtol=0, atol=1e-3 * float(np.sqrt((prod ** 2).mean())))


def test_matmul_q_ex_accumulate():
    rng = np.random.default_rng(30)
    n, k = 512, 2048
    qt = QTensor.quantize(t((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), GgmlDType.Q6K)
    x = rng.standard_normal((1, k)).astype(np.float32)
    xq = orc.quantize(orc.Q8K, x)
    y0 = rng.standard_normal((1, n)).astype(np.float32)
    y = t(y0)
    xqd = t(xq, torch.uint8)
    qmm._check(L().qmm_matmul_q_ex(qt.handle, xqd.data_ptr(), 1, y.data_ptr(), n, 1, None, 0, S()))
    prod = orc.matmul_prequant(orc.Q6K, xq, qt.to_ggml(), k)
    assert rel_err(y.cpu().numpy() - y0, prod) <= 1e-3


def test_embed_rows():
    rng = np.random.default_rng(40)
    table = rng.standard_normal((50, 96)).astype(np.float32)
    ids = [7, 3, 41, 0, 50, -1, 2 ** 31 - 1]
    toks = t(np.array(ids, np.int32), torch.int32)
    td = t(table)
    for p, tok in enumerate(ids):
        pos = t(np.array([p], np.int32), torch.int32)
        x = torch.zeros(96, device=DEV)
        qmm._check(L().qmm_embed_rows(td.data_ptr(), 96, 50, toks.data_ptr(), pos.data_ptr(), x.data_ptr(), 96,
                                      S()))
        if 0 <= tok < 50:
            np.testing.assert_array_equal(x.cpu().numpy(), table[tok])
        else:  # outside the vocabulary: no table read, a NaN row
            assert torch.isnan(x).all()
    # the batched gather: the same rule per row
    xs = torch.zeros((len(ids), 96), device=DEV)
    qmm._check(L().qmm_embed_rows_n(td.data_ptr(), 96, 50, toks.data_ptr(), 0, len(ids), xs.data_ptr(), 96, S()))
    got = xs.cpu().numpy()
    for i, tok in enumerate(ids):
        if 0 <= tok < 50:
            np.testing.assert_array_equal(got[i], table[tok])
        else:
            assert np.isnan(got[i]).all()


@pytest.mark.parametrize("heads,kv_heads,hd", [(32, 8, 128), (8, 2, 64), (4, 1, 128)])
@pytest.mark.parametrize("p", [0, 1, 37, 255])
def test_rope_kv_append(heads, kv_heads, hd, p):
    rng = np.random.default_rng(50 + p)
    cfg = LlamaConfig(heads=heads, kv_heads=kv_heads, head_dim=hd)
    max_seq = 256
    cos, sin = rope_tables(cfg, max_seq)
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    k = rng.standard_normal((kv_heads, hd)).astype(np.float32)
    v = rng.standard_normal((kv_heads, hd)).astype(np.float32)
    qd, kd, vd = t(q), t(k), t(v)
    kc = torch.zeros((kv_heads, max_seq, hd), device=DEV)
    vc = torch.zeros((kv_heads, max_seq, hd), device=DEV)
    pos = t(np.array([p], np.int32), torch.int32)
    cosd, sind = t(cos), t(sin)  # held: a temporary's memory could be reused before the kernel runs
    qmm._check(L().qmm_rope_kv_append(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), cosd.data_ptr(),
                                      sind.data_ptr(), pos.data_ptr(), kc.data_ptr(), vc.data_ptr(), heads,
                                      kv_heads, hd, max_seq, S()))
    inv = ol.llama3_inv_freq(hd, cfg.rope_theta, cfg.rope_factor, cfg.rope_low, cfg.rope_high, cfg.rope_orig_ctx)
    c, s = ol.cos_sin(inv, p)
    np.testing.assert_allclose(qd.cpu().numpy(), ol.apply_rope(q, c, s), rtol=0, atol=2e-6)
    np.testing.assert_allclose(kd.cpu().numpy(), ol.apply_rope(k, c, s), rtol=0, atol=2e-6)
    kcn, vcn = kc.cpu().numpy(), vc.cpu().numpy()
    np.testing.assert_array_equal(kcn[:, p], kd.cpu().numpy())
    np.testing.assert_array_equal(vcn[:, p], v)
    others = np.ones(max_seq, bool)
    others[p] = False
    assert not kcn[:, others].any() and not vcn[:, others].any()


def attn_ws(heads, kv_heads, hd, max_seq):
    n = int(L().qmm_decode_attention_workspace_size(heads, kv_heads, hd, max_seq))
    assert n > 0
    return torch.zeros(n, dtype=torch.uint8, device=DEV)


ATTN_GEOM = [(32, 8, 128), (8, 2, 64), (4, 4, 256), (32, 4, 128), (8, 1, 64)]


# Positions from one through fewer positions than the 16 chunks to many per chunk (merged by the
# last workgroup), and past 4096.
@pytest.mark.parametrize("heads,kv_heads,hd", ATTN_GEOM)
@pytest.mark.parametrize("p", [0, 1, 17, 127, 128, 255, 256, 300, 511, 512, 4095, 6000])
def test_decode_attention(heads, kv_heads, hd, p):
    rng = np.random.default_rng(60 + p)
    max_seq = 6144
    kc = rng.standard_normal((kv_heads, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((kv_heads, max_seq, hd)).astype(np.float32)
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    out = torch.zeros((heads, hd), device=DEV)
    pos = t(np.array([p], np.int32), torch.int32)
    scale = float(np.float32(hd) ** np.float32(-0.5))
    qd, kcd, vcd = t(q), t(kc), t(vc)
    ws = attn_ws(heads, kv_heads, hd, max_seq)
    g = heads // kv_heads
    want = np.stack([ol.attend_one(q[h], kc[h // g, : p + 1], vc[h // g, : p + 1], scale) for h in range(heads)])
    for _ in range(2):  # the second call reuses the workspace
        out.zero_()
        qmm._check(L().qmm_decode_attention(qd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), pos.data_ptr(),
                                            out.data_ptr(), heads, kv_heads, hd, max_seq, ctypes.c_float(scale),
                                            ws.data_ptr(), ws.numel(), S()))
        np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-4, atol=2e-5)


def _rope_attention_case(heads, kv_heads, hd, p, stale_nan):
    rng = np.random.default_rng(90 + p)
    max_seq = 1024
    cfg = LlamaConfig(heads=heads, kv_heads=kv_heads, head_dim=hd)
    cos, sin = rope_tables(cfg, max_seq)
    kc = rng.standard_normal((kv_heads, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((kv_heads, max_seq, hd)).astype(np.float32)
    if stale_nan:  # a cache never written at p and beyond (e.g. torch.empty): nothing there may be read
        kc[:, p:] = np.nan
        vc[:, p:] = np.nan
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    k = rng.standard_normal((kv_heads, hd)).astype(np.float32)
    v = rng.standard_normal((kv_heads, hd)).astype(np.float32)
    qd, kd, vd, kcd, vcd, cosd, sind = t(q), t(k), t(v), t(kc), t(vc), t(cos), t(sin)
    pos = t(np.array([p], np.int32), torch.int32)
    out = torch.zeros((heads, hd), device=DEV)
    ws = attn_ws(heads, kv_heads, hd, max_seq)
    scale = float(np.float32(hd) ** np.float32(-0.5))
    qmm._check(L().qmm_decode_rope_attention(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), cosd.data_ptr(),
                                             sind.data_ptr(), pos.data_ptr(), kcd.data_ptr(), vcd.data_ptr(),
                                             out.data_ptr(), heads, kv_heads, hd, max_seq, ctypes.c_float(scale),
                                             ws.data_ptr(), ws.numel(), S()))
    inv = ol.llama3_inv_freq(hd, cfg.rope_theta, cfg.rope_factor, cfg.rope_low, cfg.rope_high, cfg.rope_orig_ctx)
    c, s_ = ol.cos_sin(inv, p)
    kref, vref = kc.copy(), vc.copy()
    kref[:, p] = ol.apply_rope(k, c, s_)
    vref[:, p] = v
    np.testing.assert_array_equal(kcd.cpu().numpy(), kref)
    np.testing.assert_array_equal(vcd.cpu().numpy(), vref)
    np.testing.assert_array_equal(qd.cpu().numpy(), q)
    qr = ol.apply_rope(q, c, s_)
    g = heads // kv_heads
    want = np.stack([ol.attend_one(qr[h], kref[h // g, : p + 1], vref[h // g, : p + 1], scale) for h in range(heads)])
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-4, atol=2e-5)


@pytest.mark.parametrize("heads,kv_heads,hd", ATTN_GEOM)
@pytest.mark.parametrize("p", [0, 5, 130, 511, 700, 1023])
def test_decode_rope_attention(heads, kv_heads, hd, p):
    """Fused RoPE + KV append + attention == rope_kv_append then attention (oracle on the same cache);
    the appending workgroup is chunk 0's below the split threshold and the one whose chunk holds p above."""
    _rope_attention_case(heads, kv_heads, hd, p, False)


@pytest.mark.parametrize("heads,kv_heads,hd", [(32, 8, 128), (8, 1, 64)])
@pytest.mark.parametrize("p", [0, 5, 17, 130, 700])
def test_decode_rope_attention_ignores_unwritten_cache(heads, kv_heads, hd, p):
    """The cache holds NaN at p and beyond before the fused step: the step appends row p itself and its
    output equals the oracle's, so no masked slot reads the stale rows into the sums."""
    _rope_attention_case(heads, kv_heads, hd, p, True)


def test_two_streams_own_workspaces():
    """Split-path attention (16 chunks, counter merge) and a split-K prefill GEMM, each issued on two
    streams at once with a workspace per stream, eight rounds: every output equals the one-stream result
    (attention: to the oracle's tolerance; GEMM: bit for bit), so concurrent calls with their own
    workspaces do not see each other's counters or partials."""
    rng = np.random.default_rng(77)
    heads, kv_heads, hd, max_seq = 32, 8, 128, 4096
    scale = float(np.float32(hd) ** np.float32(-0.5))
    g = heads // kv_heads
    ps = (2999, 4000)
    kc = [rng.standard_normal((kv_heads, max_seq, hd)).astype(np.float32) for _ in ps]
    vc = [rng.standard_normal((kv_heads, max_seq, hd)).astype(np.float32) for _ in ps]
    q = [rng.standard_normal((heads, hd)).astype(np.float32) for _ in ps]
    want = [np.stack([ol.attend_one(q[i][h], kc[i][h // g, : p + 1], vc[i][h // g, : p + 1], scale)
                      for h in range(heads)]) for i, p in enumerate(ps)]
    dev_in = [(t(q[i]), t(kc[i]), t(vc[i]), t(np.array([p], np.int32), torch.int32)) for i, p in enumerate(ps)]
    outs = [torch.zeros((heads, hd), device=DEV) for _ in ps]
    wss = [attn_ws(heads, kv_heads, hd, max_seq) for _ in ps]
    # GEMM: m = 127 rows against a 4096 x 4096 Q4_K weight (split-K partials in the workspace)
    m, n, k = 127, 4096, 4096
    w = QTensor.quantize(t((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), GgmlDType.Q4K)
    xs = [t(rng.standard_normal((m, k)).astype(np.float32)) for _ in ps]
    wsb = int(L().qmm_matmul_workspace_size(w.handle, m))
    gws = [torch.zeros(max(wsb, 1), dtype=torch.uint8, device=DEV) for _ in ps]
    ys = [torch.zeros((m, n), device=DEV) for _ in ps]
    ref = []
    for i in range(len(ps)):
        qmm._check(L().qmm_matmul(w.handle, xs[i].data_ptr(), m, k, ys[i].data_ptr(), n, gws[i].data_ptr(), wsb, S()))
        ref.append(ys[i].clone())
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for r in range(8):
        for i, st in enumerate(streams):
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                h = ctypes.c_void_p(st.cuda_stream)
                qd, kcd, vcd, pos = dev_in[i]
                outs[i].zero_()
                ys[i].zero_()
                qmm._check(L().qmm_decode_attention(qd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), pos.data_ptr(),
                                                    outs[i].data_ptr(), heads, kv_heads, hd, max_seq,
                                                    ctypes.c_float(scale), wss[i].data_ptr(), wss[i].numel(), h))
                qmm._check(L().qmm_matmul(w.handle, xs[i].data_ptr(), m, k, ys[i].data_ptr(), n, gws[i].data_ptr(),
                                          wsb, h))
        for st in streams:
            torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        for i in range(len(ps)):
            np.testing.assert_allclose(outs[i].cpu().numpy(), want[i], rtol=1e-4, atol=2e-5, err_msg=f"round {r}")
            assert torch.equal(ys[i], ref[i]), f"round {r} stream {i}"


def test_attention_geometry_errors():
    for bad in [(32, 5, 128, 64), (32, 2, 128, 64), (8, 2, 96, 64), (8, 2, 128, (1 << 20) + 1), (8, 2, 128, 0)]:
        assert int(L().qmm_decode_attention_workspace_size(*bad)) == 0
    ws = attn_ws(8, 2, 128, 64)
    x = torch.zeros(16, device=DEV)
    rc = L().qmm_decode_attention(x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), 8, 2, 128,
                                  64, ctypes.c_float(1.0), ws.data_ptr(), 16, S())
    assert rc == 1 and "workspace" in qmm.last_error()


def test_silu_mul_quantize():
    rng = np.random.default_rng(70)
    rows, k = 2, 1536
    gt = (rng.standard_normal((rows, k)) * 2).astype(np.float32)
    ut = rng.standard_normal((rows, k)).astype(np.float32)
    hq = torch.zeros((rows, k // 256 * 292), dtype=torch.uint8, device=DEV)
    gd, ud = t(gt), t(ut)
    qmm._check(L().qmm_silu_mul_quantize(gd.data_ptr(), ud.data_ptr(), rows, k, k, hq.data_ptr(), S()))
    h = (ol.silu(gt) * ut).astype(np.float32)
    want = orc.quantize(orc.Q8K, h)
    got = hq.cpu().numpy()
    # expf may differ from numpy's exp by an ulp: a quant may move by one step at a rounding tie
    dg = orc.dequantize(orc.Q8K, got, rows * k)
    dw = orc.dequantize(orc.Q8K, want, rows * k)
    d = np.abs(h).reshape(-1, 256).max(axis=1) / 127.0
    assert np.all(np.abs(dg - dw).reshape(-1, 256) <= 1.01 * d[:, None] + 1e-12)
    assert (got != want).mean() < 0.01


@pytest.mark.parametrize("dt,n,k", [(GgmlDType.Q6K, 4096, 14336), (GgmlDType.Q4K, 1000, 3072),
                                    (GgmlDType.Q6K, 777, 1536)])
@pytest.mark.parametrize("accumulate", [0, 1])
def test_silu_mul_matmul_equals_two_calls(dt, n, k, accumulate):
    # the fused down projection (Q8_K of silu(g) * u formed in the GEMV prologue) against the
    # two-call form (qmm_silu_mul_quantize + qmm_matmul_q_ex): bit-identical outputs
    rng = np.random.default_rng(90 + n)
    qt = QTensor.quantize(t((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), dt)
    g = t((rng.standard_normal(k) * 2).astype(np.float32))
    u = t(rng.standard_normal(k).astype(np.float32))
    y0 = rng.standard_normal(n).astype(np.float32)
    ya, yb = t(y0), t(y0)
    hq = torch.zeros(k // 256 * 292, dtype=torch.uint8, device=DEV)
    qmm._check(L().qmm_silu_mul_quantize(g.data_ptr(), u.data_ptr(), 1, k, k, hq.data_ptr(), S()))
    qmm._check(L().qmm_matmul_q_ex(qt.handle, hq.data_ptr(), 1, ya.data_ptr(), n, accumulate, None, 0, S()))
    qmm._check(L().qmm_silu_mul_matmul(qt.handle, g.data_ptr(), u.data_ptr(), yb.data_ptr(), accumulate, S()))
    torch.cuda.synchronize()
    assert torch.equal(ya, yb)
    # and the oracle on the device's own activation bytes
    want = orc.matmul_prequant(int(dt), hq.cpu().numpy()[None], qt.to_ggml(), k)[0]
    got = yb.cpu().numpy() - (y0 if accumulate else 0)
    assert rel_err(got, want) <= 1e-3


def test_silu_mul_matmul_rejects_q8_0():
    qt = QTensor.quantize(torch.zeros((64, 256), device=DEV), GgmlDType.Q8_0)
    x = torch.zeros(256, device=DEV)
    y = torch.zeros(64, device=DEV)
    rc = L().qmm_silu_mul_matmul(qt.handle, x.data_ptr(), x.data_ptr(), y.data_ptr(), 0, S())
    assert rc != 0 and "k-quant" in qmm.last_error()


def test_greedy_advance():
    logits = t(np.array([0.5, 3.0, -1.0, 3.0, 2.0], np.float32))
    toks = t(np.array([4, 4, 4, 0, 0, 0], np.int32), torch.int32)
    pos = t(np.array([0], np.int32), torch.int32)
    ws = torch.zeros(int(L().qmm_greedy_workspace_size(128256)), dtype=torch.uint8, device=DEV)

    def adv(prompt_len, capacity=6, n=5):
        qmm._check(L().qmm_greedy_advance(logits.data_ptr(), n, toks.data_ptr(), capacity, pos.data_ptr(),
                                          prompt_len, ws.data_ptr(), ws.numel(), S()))
        torch.cuda.synchronize()
        return toks.cpu().tolist(), int(pos.item())

    assert adv(3) == ([4, 4, 4, 0, 0, 0], 1)  # slot 1 holds a prompt token
    assert adv(3) == ([4, 4, 4, 0, 0, 0], 2)
    assert adv(3) == ([4, 4, 4, 1, 0, 0], 3)  # ties -> lowest index
    adv(3)
    assert adv(3) == ([4, 4, 4, 1, 1, 1], 5)
    assert adv(3) == ([4, 4, 4, 1, 1, 1], 5)  # capacity reached: nothing written, pos stays
    rng = np.random.default_rng(80)
    for trial in range(6):
        big = (rng.standard_normal(128256) * 3).astype(np.float32)
        win = int(rng.integers(0, 128256))
        big[win] = big.max() + 1.0
        if trial >= 3:  # exact ties across workgroup slices: the lowest index wins
            other = int(rng.integers(0, 128256))
            big[other] = big[win]
            win = min(win, other)
        logits = t(big)
        pos.zero_()
        adv(1, n=128256)
        assert toks[1].item() == win
    assert not ws[:256].any()
    # NaN logits count as the largest value (the first NaN wins, torch.argmax's
    # rule): the written token is always an index of the logits
    for nan_at in ([], [77], [70000, 5]):
        big = np.full(128256, np.nan if not nan_at else 0.0, np.float32)
        for i in nan_at:
            big[i] = np.nan
        logits = t(big)
        pos.zero_()
        adv(1, n=128256)
        assert toks[1].item() == (min(nan_at) if nan_at else 0)
        assert int(torch.argmax(logits).item()) == toks[1].item()
    assert not ws[:256].any()
    with pytest.raises(qmm.QmmError):
        qmm._check(L().qmm_greedy_advance(logits.data_ptr(), 5, toks.data_ptr(), 6, pos.data_ptr(), 1,
                                          ws.data_ptr(), 8, S()))


@pytest.mark.parametrize("dt", [GgmlDType.Q4K, GgmlDType.Q6K])
@pytest.mark.parametrize("m,k", [(37, 4096), (127, 4096), (64, 14336)])
def test_matmul_ex_gemm_norm_planes_equal_two_launches(dt, m, k):
    """At m > 8 the RMSNorm and the Q8_K GEMM planes come from one launch (qmm_rms_norm_q8k_mmq): the
    same bits as qmm_rms_norm's rows quantized and multiplied without the norm."""
    rng = np.random.default_rng(70 + m + k)
    n = 768
    qt = QTensor.quantize(t((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), dt)
    x = t((rng.standard_normal((m, k)) * 0.3).astype(np.float32))
    nw = t(rng.uniform(0.5, 1.5, k).astype(np.float32))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    wsb = int(L().qmm_matmul_ex_workspace_size(qt.handle, m, 1))
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)

    def mm(src, norm):
        y = torch.full((m, n), float("nan"), device=DEV)
        qmm._check(L().qmm_matmul_ex((vp * 1)(qt.handle.value), 1, src.data_ptr(), m, k,
                                     nw.data_ptr() if norm else None, ctypes.c_float(1e-5), 0,
                                     (vp * 1)(y.data_ptr()), (i64 * 1)(n), ws.data_ptr(), wsb, S()))
        torch.cuda.synchronize()
        return y
    fused = mm(x, True)
    xn = torch.empty((m, k), device=DEV)
    qmm._check(L().qmm_rms_norm(x.data_ptr(), m, k, k, nw.data_ptr(), ctypes.c_float(1e-5), xn.data_ptr(), k, S()))
    assert torch.equal(fused, mm(xn, False))


def test_rope_attention_with_l2_warming_equals_plain():
    """qmm_decode_rope_attention_warm (extra workgroups load the following launches' first weight rows into
    L2) writes the same bits as qmm_decode_rope_attention: output and both caches; bad warm plans are refused."""
    heads, kv_heads, hd, max_seq, p = 32, 8, 128, 512, 300
    rng = np.random.default_rng(77)
    cfg = LlamaConfig(heads=heads, kv_heads=kv_heads, head_dim=hd)
    cos, sin = rope_tables(cfg, max_seq)
    kc = rng.standard_normal((kv_heads, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((kv_heads, max_seq, hd)).astype(np.float32)
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    k = rng.standard_normal((kv_heads, hd)).astype(np.float32)
    v = rng.standard_normal((kv_heads, hd)).astype(np.float32)
    g = torch.Generator(device=DEV).manual_seed(78)
    wo = QTensor.quantize(torch.randn((4096, 4096), generator=g, device=DEV) * 0.02, GgmlDType.Q4K)
    wg = QTensor.quantize(torch.randn((14336, 4096), generator=g, device=DEV) * 0.02, GgmlDType.Q4K)
    wu = QTensor.quantize(torch.randn((14336, 4096), generator=g, device=DEV) * 0.02, GgmlDType.Q4K)
    scale = ctypes.c_float(float(np.float32(hd) ** np.float32(-0.5)))
    outs = []
    for warm in (False, True):
        kcd, vcd = t(kc), t(vc)
        out = torch.full((heads, hd), float("nan"), device=DEV)
        ws = attn_ws(heads, kv_heads, hd, max_seq)
        args = (t(q).data_ptr(), t(k).data_ptr(), t(v).data_ptr(), t(cos).data_ptr(), t(sin).data_ptr(),
                t(np.array([p], np.int32), torch.int32).data_ptr(), kcd.data_ptr(), vcd.data_ptr(), out.data_ptr(),
                heads, kv_heads, hd, max_seq, scale, ws.data_ptr(), ws.numel())
        if warm:
            W = (ctypes.c_void_p * 3)(wo.handle.value, wg.handle.value, wu.handle.value)
            qmm._check(L().qmm_decode_rope_attention_warm(*args, W, (ctypes.c_int * 3)(0, 1, 1), 3,
                                                          (ctypes.c_int * 2)(1, 3), S()))
            # refused: more than three weights, a decreasing launch index, a Q8_0 weight
            assert L().qmm_decode_rope_attention_warm(*args, W, (ctypes.c_int * 3)(0, 1, 1), 4,
                                                      (ctypes.c_int * 2)(1, 3), S()) != 0
            assert L().qmm_decode_rope_attention_warm(*args, W, (ctypes.c_int * 3)(1, 0, 0), 3,
                                                      (ctypes.c_int * 2)(1, 3), S()) != 0
            w8 = QTensor.quantize(torch.zeros((256, 4096), device=DEV), GgmlDType.Q8_0)
            assert L().qmm_decode_rope_attention_warm(*args, (ctypes.c_void_p * 1)(w8.handle.value),
                                                      (ctypes.c_int * 1)(0), 1, (ctypes.c_int * 1)(1), S()) != 0
        else:
            qmm._check(L().qmm_decode_rope_attention(*args, S()))
        torch.cuda.synchronize()
        outs.append((out.cpu().numpy(), kcd.cpu().numpy(), vcd.cpu().numpy()))
    for a, b in zip(outs[0], outs[1]):
        np.testing.assert_array_equal(a, b)
    assert np.isfinite(outs[0][0]).all()
