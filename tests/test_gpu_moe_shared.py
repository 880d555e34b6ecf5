"""The two branches of MoeMlp::forward (crates/llm/candle-llm/src/models/llama.rs:1416-1487) beyond the
Mixtral case: routed weights scaled by routed_scaling_factor when norm_topk_prob is false (:1436-1447), and
the always-on shared expert, ungated (DeepSeek-V2) or gated per token by sigmoid(x . shared_gate) (Qwen2-MoE,
:1476-1486). Both the decode-sized expert-GEMV path and the grouped-GEMM path are run.

Checked against the oracle (oracle/moe.py):
* routing: the same experts, and weights within f32 rounding of p * routed_scaling_factor;
* the shared expert, op level: the device's output with the shared expert minus its output without (both
  device runs, the routed part bit-identical) is the shared MLP within 1e-3 * rms of the oracle's on the same
  x, times sigmoid(x . gate) within 1e-5 when gated;
* end to end: cosine >= 0.99999 and max|d| / rms <= 1e-2 against the oracle's MoeMlp::forward (the chain
  bar of the plain MoE FFN test: a last-bit difference of silu's exp that lands on a Q8_K rounding tie moves
  one code of the down projection's activation).
"""
import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, QTensor, moe_ffn, moe_route
from inference_amd.synth import normal
from oracle import moe
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def rel_err(y, y_ref):
    y_ref = np.asarray(y_ref, dtype=np.float64)
    return float(np.abs(np.asarray(y, dtype=np.float64) - y_ref).max() / np.sqrt(np.mean(y_ref ** 2)))


def stacked(E, rows, cols, dt, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    qt = QTensor.quantize(torch.randn((E * rows, cols), generator=g, device=DEV) * 0.02, dt)
    raw = qt.to_ggml()
    per = raw.size // E
    return qt, [raw[e * per:(e + 1) * per] for e in range(E)]


@pytest.mark.parametrize("T,E,k", [(8, 8, 2), (300, 8, 2), (64, 16, 6)])
@pytest.mark.parametrize("scale", [1.0, 2.5])
def test_route_unnormalised_scaled_weights(T, E, k, scale):
    lg = normal(700 + T + E, (T, E)).astype(np.float32)
    counts, offsets, ptok, pw, tp = moe_route(torch.from_numpy(lg).to(DEV), k, renormalize=False,
                                              routed_scaling_factor=scale)
    experts, weights = moe.route(lg, k, renormalize=False, routed_scaling_factor=scale)
    c, o = counts.cpu().numpy(), offsets.cpu().numpy()
    pt, w, tpn = ptok.cpu().numpy(), pw.cpu().numpy(), tp.cpu().numpy()
    for t in range(T):
        pairs = tpn[t * k:(t + 1) * k]
        got_e = sorted(int(np.searchsorted(o, p, side="right") - 1) for p in pairs)
        assert got_e == sorted(experts[t]), t
        for p in pairs:
            e = int(np.searchsorted(o, p, side="right") - 1)
            assert pt[p] == t and o[e] <= p < o[e] + c[e]
            want = float(weights[t][experts[t].index(e)])
            assert abs(float(w[p]) - want) <= 2e-6 * abs(want) + 1e-12, (t, e, float(w[p]), want)


@pytest.mark.parametrize("T", [8, 96])
@pytest.mark.parametrize("norm,scale", [(False, 2.5), (True, 1.0)])
def test_moe_ffn_shared_expert_and_scaling(T, norm, scale):
    E, H, F, Fs, k = 4, 512, 768, 512, 2
    gate, gper = stacked(E, F, H, GgmlDType.Q4K, 720 + T)
    up, uper = stacked(E, F, H, GgmlDType.Q4K, 721 + T)
    down, dper = stacked(E, H, F, GgmlDType.Q6K, 722 + T)
    sg, (sg_b,) = stacked(1, Fs, H, GgmlDType.Q4K, 723 + T)
    su, (su_b,) = stacked(1, Fs, H, GgmlDType.Q4K, 724 + T)
    sd, (sd_b,) = stacked(1, H, Fs, GgmlDType.Q6K, 725 + T)
    x = normal(726 + T, (T, H))
    lg = normal(727 + T, (T, E)).astype(np.float32)
    gvec = (normal(728 + T, (H,)) * 0.05).astype(np.float32)
    xd, ld, gd = torch.from_numpy(x).to(DEV), torch.from_numpy(lg).to(DEV), torch.from_numpy(gvec).to(DEV)

    base = moe_ffn(xd, ld, gate, up, down, k, norm_topk_prob=norm, routed_scaling_factor=scale).cpu().numpy()
    ung = moe_ffn(xd, ld, gate, up, down, k, norm_topk_prob=norm, routed_scaling_factor=scale,
                  shared=(sg, su, sd)).cpu().numpy()
    gated = moe_ffn(xd, ld, gate, up, down, k, norm_topk_prob=norm, routed_scaling_factor=scale,
                    shared=(sg, su, sd), shared_gate=gd).cpu().numpy()
    shared_ref = moe.mlp(x, sg_b, su_b, sd_b, orc.Q4K, orc.Q6K, H, Fs).astype(np.float64)
    sh_dev = ung.astype(np.float64) - base.astype(np.float64)
    assert rel_err(sh_dev, shared_ref) <= 1e-3
    sig = 1.0 / (1.0 + np.exp(-(x.astype(np.float64) @ gvec.astype(np.float64))))
    gated_part = gated.astype(np.float64) - base.astype(np.float64)
    assert rel_err(gated_part, sig[:, None] * sh_dev) <= 1e-5

    for got, kw in ((base, {}), (ung, {"shared": (sg_b, su_b, sd_b, orc.Q4K, orc.Q6K)}),
                    (gated, {"shared": (sg_b, su_b, sd_b, orc.Q4K, orc.Q6K), "shared_gate": gvec})):
        ref = moe.moe_ffn(x, lg, gper, uper, dper, orc.Q4K, orc.Q6K, k, renormalize=norm,
                          routed_scaling_factor=scale, **kw)
        cos = float((got * ref).sum() / np.sqrt((got * got).sum() * (ref * ref).sum()))
        assert cos >= 0.99999 and rel_err(got, ref) <= 1e-2, (kw.keys(), cos, rel_err(got, ref))


def test_moe_ffn_shared_expert_arguments_are_checked():
    from inference_amd import QmmError
    E, H, F = 2, 256, 512
    gate, _ = stacked(E, F, H, GgmlDType.Q4K, 740)
    up, _ = stacked(E, F, H, GgmlDType.Q4K, 741)
    down, _ = stacked(E, H, F, GgmlDType.Q6K, 742)
    bad_down, _ = stacked(1, 128, 256, GgmlDType.Q6K, 743)  # output width 128 != hidden 256
    sgw, _ = stacked(1, 256, H, GgmlDType.Q4K, 744)
    x = torch.zeros((4, H), device=DEV)
    lg = torch.zeros((4, E), device=DEV)
    with pytest.raises(QmmError):
        moe_ffn(x, lg, gate, up, down, 1, shared=(sgw, sgw, bad_down))
    with pytest.raises(QmmError):
        moe_ffn(x, lg, gate, up, down, 1, shared_gate=torch.zeros(H, device=DEV))
