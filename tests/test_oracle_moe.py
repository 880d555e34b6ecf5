"""Pins the MoE restatement (oracle/moe.py) with checks that do not retype it:
top-k against a sort of the raw logits (softmax is monotone), weight sums,
a single expert equal to the dense MLP, and identical experts reproducing the
dense MLP whatever the routing."""
import numpy as np

from oracle import moe
from oracle import oracle as orc


def _rng(seed):
    return np.random.default_rng(seed)


def test_route_selects_top_logits_and_normalises():
    logits = _rng(0).standard_normal((64, 8)).astype(np.float32)
    experts, weights = moe.route(logits, 2)
    for t in range(64):
        order = np.argsort(-logits[t], kind="stable")[:2]
        assert list(order) == experts[t]
        assert abs(float(np.sum(weights[t])) - 1.0) < 1e-6
        assert weights[t][0] >= weights[t][1]


def test_route_weights_match_two_way_softmax():
    # renormalised top-2 softmax probabilities equal the softmax of the two logits
    logits = _rng(1).standard_normal((32, 8)).astype(np.float32)
    experts, weights = moe.route(logits, 2)
    for t in range(32):
        a, b = logits[t][experts[t][0]], logits[t][experts[t][1]]
        w0 = 1.0 / (1.0 + np.exp(float(b) - float(a)))
        assert abs(w0 - float(weights[t][0])) < 1e-6


def _experts(seed, E, H, F, same=False):
    r = _rng(seed)
    g = [orc.quantize(orc.Q4K, (r.standard_normal((F, H)) * 0.05).astype(np.float32))]
    u = [orc.quantize(orc.Q4K, (r.standard_normal((F, H)) * 0.05).astype(np.float32))]
    d = [orc.quantize(orc.Q6K, (r.standard_normal((H, F)) * 0.05).astype(np.float32))]
    for _ in range(E - 1):
        if same:
            g.append(g[0]); u.append(u[0]); d.append(d[0])
        else:
            g.append(orc.quantize(orc.Q4K, (r.standard_normal((F, H)) * 0.05).astype(np.float32)))
            u.append(orc.quantize(orc.Q4K, (r.standard_normal((F, H)) * 0.05).astype(np.float32)))
            d.append(orc.quantize(orc.Q6K, (r.standard_normal((H, F)) * 0.05).astype(np.float32)))
    return g, u, d


def test_single_expert_is_the_dense_mlp():
    H, F = 256, 512
    g, u, d = _experts(2, 1, H, F)
    x = _rng(3).standard_normal((5, H)).astype(np.float32)
    logits = np.zeros((5, 1), np.float32)
    y = moe.moe_ffn(x, logits, g, u, d, orc.Q4K, orc.Q6K, k=1)
    assert np.array_equal(y, moe.mlp(x, g[0], u[0], d[0], orc.Q4K, orc.Q6K, H, F))


def test_identical_experts_reproduce_the_dense_mlp():
    H, F = 256, 512
    g, u, d = _experts(4, 4, H, F, same=True)
    x = _rng(5).standard_normal((6, H)).astype(np.float32)
    logits = _rng(6).standard_normal((6, 4)).astype(np.float32)
    y = moe.moe_ffn(x, logits, g, u, d, orc.Q4K, orc.Q6K, k=2)
    dense = moe.mlp(x, g[0], u[0], d[0], orc.Q4K, orc.Q6K, H, F)
    assert np.allclose(y, dense, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# the routed scaling factor and the shared expert (llama.rs:1436-1447, 1476-1486)
# ---------------------------------------------------------------------------

def test_unnormalised_weights_are_the_scaled_probabilities():
    """norm_topk_prob false: each selected weight is its softmax probability (computed here in f64 from
    the logits) times the routed scaling factor; with every expert selected they sum to that factor."""
    logits = _rng(7).standard_normal((40, 6)).astype(np.float32)
    for scale in (1.0, 2.5, 16.0):
        experts, weights = moe.route(logits, 6, renormalize=False, routed_scaling_factor=scale)
        for t in range(40):
            l = logits[t].astype(np.float64)
            p = np.exp(l - l.max()) / np.exp(l - l.max()).sum()
            np.testing.assert_allclose(weights[t], p[experts[t]] * scale, rtol=2e-6)
            assert abs(float(np.sum(weights[t], dtype=np.float64)) - scale) < 4e-6 * scale
        # top-2 without renormalising: the two largest probabilities, scaled, not summing to the factor
        e2, w2 = moe.route(logits, 2, renormalize=False, routed_scaling_factor=scale)
        assert all(e2[t] == experts[t][:2] for t in range(40))
        assert all(np.array_equal(w2[t], weights[t][:2]) for t in range(40))


def test_shared_expert_is_added_after_the_routed_sum():
    """out = routed + shared: with the shared expert's MLP added ungated the difference from the routed
    output is the dense MLP itself; with a zero gate vector sigmoid(0) = 1/2 halves it exactly; with the
    gate along one coordinate it is sigmoid(c * x[:, 0]) of it."""
    H, F, Fs, T = 256, 512, 256, 7
    g, u, d = _experts(8, 4, H, F)
    sg, su, sd = (a[0] for a in _experts(9, 1, H, Fs))
    x = _rng(10).standard_normal((T, H)).astype(np.float32)
    logits = _rng(11).standard_normal((T, 4)).astype(np.float32)
    shared = (sg, su, sd, orc.Q4K, orc.Q6K)
    base = moe.moe_ffn(x, logits, g, u, d, orc.Q4K, orc.Q6K, k=2)
    dense = moe.mlp(x, sg, su, sd, orc.Q4K, orc.Q6K, H, Fs).astype(np.float64)
    ung = moe.moe_ffn(x, logits, g, u, d, orc.Q4K, orc.Q6K, k=2, shared=shared)
    np.testing.assert_allclose(ung - base.astype(np.float64), dense, rtol=1e-5, atol=1e-5)
    half = moe.moe_ffn(x, logits, g, u, d, orc.Q4K, orc.Q6K, k=2, shared=shared,
                       shared_gate=np.zeros(H, np.float32))
    np.testing.assert_allclose(half - base.astype(np.float64), 0.5 * dense, rtol=1e-5, atol=1e-5)
    c = 0.75
    gate = np.zeros(H, np.float32)
    gate[0] = c
    gated = moe.moe_ffn(x, logits, g, u, d, orc.Q4K, orc.Q6K, k=2, shared=shared, shared_gate=gate)
    sig = 1.0 / (1.0 + np.exp(-c * x[:, 0].astype(np.float64)))
    np.testing.assert_allclose(gated - base.astype(np.float64), sig[:, None] * dense, rtol=1e-5, atol=1e-5)
