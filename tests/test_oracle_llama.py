"""Pins the CPU decode-step oracle (oracle/llama.py) before it is trusted as the checker.

Known answers from the reference's own tests (primitives/rope.rs tests,
primitives/sampler.rs:315-325) and properties the mathematics fixes: RoPE is
a rotation of each (i, i + dim/2) pair by pos * inv_freq[i] (complex
multiplication, checked on its own), the identity at position 0, and depends
only on relative position inside a dot product; RMSNorm output has unit RMS
and is scale invariant; attention over one position returns v, over equal
keys the mean of v; a decoder whose o and down projections are zero reduces
to head(rms_norm(embedding)).
"""
import math
from types import SimpleNamespace

import numpy as np
import pytest

from oracle import llama as ol
from oracle import oracle as orc


def std_inv_freq(dim, theta):
    return np.array([1.0 / theta ** (2 * i / dim) for i in range(dim // 2)])


def test_llama3_unit_factor_equals_standard():
    # rope.rs test llama3_with_unit_factor_equals_standard
    l3 = ol.llama3_inv_freq(128, 500000.0, 1.0, 1.0, 4.0, 8192.0)
    np.testing.assert_allclose(l3, std_inv_freq(128, 500000.0), rtol=0, atol=1e-6)


def test_llama3_bands():
    # rope.rs test llama3_scales_low_frequencies_down, plus the pass-through and blended bands
    l3 = ol.llama3_inv_freq(128, 500000.0, 8.0, 1.0, 4.0, 8192.0).astype(np.float64)
    st = std_inv_freq(128, 500000.0)
    assert abs(l3[-1] - st[-1] / 8.0) < 1e-9
    wl = 2 * math.pi / st
    hi, lo = wl < 8192.0 / 4.0, wl > 8192.0
    assert hi.sum() > 0 and lo.sum() > 0 and (~hi & ~lo).sum() > 0
    np.testing.assert_allclose(l3[hi], st[hi], rtol=1e-6)
    np.testing.assert_allclose(l3[lo], st[lo] / 8.0, rtol=1e-6)
    mid = ~hi & ~lo
    assert np.all(l3[mid] < st[mid]) and np.all(l3[mid] > st[mid] / 8.0)
    assert np.all(np.diff(l3) < 0)


def test_rope_position_zero_identity():
    x = np.random.default_rng(1).standard_normal((4, 128)).astype(np.float32)
    c, s = ol.cos_sin(ol.llama3_inv_freq(128, 500000.0, 8.0, 1.0, 4.0, 8192.0), 0)
    np.testing.assert_array_equal(ol.apply_rope(x, c, s), x)


def test_rope_is_pairwise_complex_rotation():
    rng = np.random.default_rng(2)
    inv = ol.llama3_inv_freq(64, 10000.0, 1.0, 1.0, 4.0, 8192.0)
    x = rng.standard_normal(64).astype(np.float32)
    for pos in (1, 7, 100):
        c, s = ol.cos_sin(inv, pos)
        y = ol.apply_rope(x, c, s)
        z = (x[:32].astype(np.complex128) + 1j * x[32:]) * np.exp(1j * pos * inv.astype(np.float64))
        np.testing.assert_allclose(y[:32], z.real, atol=1e-4)
        np.testing.assert_allclose(y[32:], z.imag, atol=1e-4)
        np.testing.assert_allclose(y[:32] ** 2 + y[32:] ** 2, x[:32] ** 2 + x[32:] ** 2, rtol=1e-4)


def test_rope_relative_position():
    rng = np.random.default_rng(3)
    inv = ol.llama3_inv_freq(128, 500000.0, 8.0, 1.0, 4.0, 8192.0)
    q, k = rng.standard_normal((2, 128)).astype(np.float32)

    def dot(m, n):
        cm, sm = ol.cos_sin(inv, m)
        cn, sn = ol.cos_sin(inv, n)
        return float(np.dot(ol.apply_rope(q, cm, sm).astype(np.float64), ol.apply_rope(k, cn, sn)))

    for m, n, d in ((5, 2, 9), (30, 11, 40)):
        assert abs(dot(m, n) - dot(m + d, n + d)) < 2e-4 * (1 + abs(dot(m, n)))


def test_rms_norm_unit_rms_and_scale_invariance():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 4096)).astype(np.float32) * 3.0
    y = ol.rms_norm(x, np.ones(4096, np.float32), 1e-5)
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(axis=1)), 1.0, rtol=1e-5)
    np.testing.assert_allclose(ol.rms_norm(x * 10.0, np.ones(4096, np.float32), 1e-5), y, rtol=1e-5, atol=1e-6)
    w = rng.standard_normal(4096).astype(np.float32)
    np.testing.assert_allclose(ol.rms_norm(x, w, 1e-5), y * w, rtol=1e-6, atol=1e-6)


def test_attention_special_cases():
    rng = np.random.default_rng(5)
    q = rng.standard_normal(128).astype(np.float32)
    k1 = rng.standard_normal((1, 128)).astype(np.float32)
    v1 = rng.standard_normal((1, 128)).astype(np.float32)
    np.testing.assert_allclose(ol.attend_one(q, k1, v1, 0.1), v1[0], rtol=1e-6)
    keys = np.repeat(k1, 9, axis=0)
    vals = rng.standard_normal((9, 128)).astype(np.float32)
    np.testing.assert_allclose(ol.attend_one(q, keys, vals, 0.1), vals.mean(axis=0), rtol=1e-5, atol=1e-6)
    # one key aligned with q at a large scale takes all the weight
    keys = rng.standard_normal((9, 128)).astype(np.float32) * 0.01
    keys[4] = q
    np.testing.assert_allclose(ol.attend_one(q, keys, vals, 10.0), vals[4], rtol=1e-5, atol=1e-6)


def test_argmax_reference_cases():
    # sampler.rs tests argmax_device_matches_host / argmax_ties_break_to_lowest_index
    assert ol.argmax_first(np.array([0.1, 5.0, 0.2, 9.9, 3.0])) == 3
    assert ol.argmax_first(np.array([1.0, 5.0, 5.0, 2.0])) == 1


def tiny_cfg(layers=2):
    return SimpleNamespace(layers=layers, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=300,
                           rope_theta=500000.0, rope_factor=8.0, rope_low=1.0, rope_high=4.0,
                           rope_orig_ctx=8192.0, eps=1e-5,
                           dtypes={"q": orc.Q4K, "k": orc.Q4K, "v": orc.Q6K, "o": orc.Q4K, "gate": orc.Q4K,
                                   "up": orc.Q4K, "down": orc.Q6K, "head": orc.Q6K})


def tiny_export(cfg, rng, zero=()):
    sh = {"q": (cfg.heads * cfg.head_dim, cfg.hidden), "k": (cfg.kv_heads * cfg.head_dim, cfg.hidden),
          "v": (cfg.kv_heads * cfg.head_dim, cfg.hidden), "o": (cfg.hidden, cfg.heads * cfg.head_dim),
          "gate": (cfg.ffn, cfg.hidden), "up": (cfg.ffn, cfg.hidden), "down": (cfg.hidden, cfg.ffn)}

    def q(name, n, k):
        w = np.zeros((n, k), np.float32) if name in zero else rng.standard_normal((n, k)).astype(np.float32) * 0.05
        return orc.quantize(int(cfg.dtypes[name]), w)

    return {"layers": [{nm: q(nm, *sh[nm]) for nm in sh} for _ in range(cfg.layers)],
            "head": q("head", cfg.vocab, cfg.hidden),
            "embed": rng.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float32),
            "attn_norm": [rng.uniform(0.5, 1.5, cfg.hidden).astype(np.float32) for _ in range(cfg.layers)],
            "ffn_norm": [rng.uniform(0.5, 1.5, cfg.hidden).astype(np.float32) for _ in range(cfg.layers)],
            "final_norm": rng.uniform(0.5, 1.5, cfg.hidden).astype(np.float32)}


def test_zero_residual_branches_reduce_to_head_of_embedding():
    cfg = tiny_cfg()
    ex = tiny_export(cfg, np.random.default_rng(6), zero=("o", "down"))
    orl = ol.LlamaOracle(cfg, ex, 8)
    for pos, tok in enumerate((5, 17, 5)):
        lg = orl.step(tok, pos)
        want = orc.matmul(orc.Q6K, ol.rms_norm(ex["embed"][tok], ex["final_norm"], cfg.eps)[None], ex["head"],
                          cfg.hidden)[0]
        np.testing.assert_array_equal(lg, want)


def test_kv_cache_holds_rotated_keys_and_values():
    cfg = tiny_cfg(layers=1)
    ex = tiny_export(cfg, np.random.default_rng(7))
    orl = ol.LlamaOracle(cfg, ex, 8)
    orl.step(9, 0)
    orl.step(11, 1)
    x = ex["embed"][11]
    n = ol.rms_norm(x, ex["attn_norm"][0], cfg.eps)
    k = orc.matmul(orc.Q4K, n[None], ex["layers"][0]["k"], cfg.hidden)[0].reshape(cfg.kv_heads, cfg.head_dim)
    v = orc.matmul(orc.Q6K, n[None], ex["layers"][0]["v"], cfg.hidden)[0].reshape(cfg.kv_heads, cfg.head_dim)
    c, s = ol.cos_sin(orl.inv_freq, 1)
    np.testing.assert_array_equal(orl.kc[0, :, 1], ol.apply_rope(k, c, s))
    np.testing.assert_array_equal(orl.vc[0, :, 1], v)
    assert not orl.kc[0, :, 2:].any()


def test_generate_is_deterministic_and_keeps_prompt():
    cfg = tiny_cfg(layers=1)
    ex = tiny_export(cfg, np.random.default_rng(8))
    a = ol.LlamaOracle(cfg, ex, 16).generate([3, 1, 4], 5)
    b = ol.LlamaOracle(cfg, ex, 16).generate([3, 1, 4], 5)
    assert a == b and a[:3] == [3, 1, 4] and len(a) == 8
    assert all(0 <= t < cfg.vocab for t in a)


@pytest.mark.skipif(not orc.simd_supported(), reason="needs an AVX2 + FMA host")
def test_two_reference_builds_part_at_a_q8k_tie():
    """Candle's generic and AVX2 vec_dot bodies give the same integer block dots and differ only in f32
    summation order. Their decode chains agree to f32 noise until one activation's Q8_K code sits on a
    rounding tie; there the two round apart by one quantum, and the layers after amplify it. Shown on an
    8-layer Llama-shaped model: the first K/V rows to leave noise are preceded, within the same
    position, by a quantization whose inputs still agree to f32 noise but whose codes differ by one at
    tie elements; the logits then differ far beyond f32 noise."""
    from decode_check import assert_tie, first_flip, kv_rel, quant_inputs_from_record, rel_err
    cfg = SimpleNamespace(layers=8, hidden=1024, ffn=2816, heads=8, kv_heads=2, head_dim=128, vocab=2048,
                          rope_theta=500000.0, rope_factor=8.0, rope_low=1.0, rope_high=4.0, rope_orig_ctx=8192.0,
                          eps=1e-5, dtypes={"q": orc.Q4K, "k": orc.Q4K, "v": orc.Q6K, "o": orc.Q4K, "gate": orc.Q4K,
                                            "up": orc.Q4K, "down": orc.Q6K, "head": orc.Q6K})
    rng = np.random.default_rng(1)
    hd = cfg.heads * cfg.head_dim
    sh = {"q": (hd, cfg.hidden), "k": (cfg.kv_heads * cfg.head_dim, cfg.hidden),
          "v": (cfg.kv_heads * cfg.head_dim, cfg.hidden), "o": (cfg.hidden, hd), "gate": (cfg.ffn, cfg.hidden),
          "up": (cfg.ffn, cfg.hidden), "down": (cfg.hidden, cfg.ffn)}

    def q(n, k, dt):
        return orc.quantize(dt, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))

    ex = {"layers": [{nm: q(*sh[nm], cfg.dtypes[nm]) for nm in sh} for _ in range(cfg.layers)],
          "head": q(cfg.vocab, cfg.hidden, orc.Q6K),
          "embed": (rng.standard_normal((cfg.vocab, cfg.hidden)) * 0.02).astype(np.float32),
          "attn_norm": [np.ones(cfg.hidden, np.float32)] * cfg.layers,
          "ffn_norm": [np.ones(cfg.hidden, np.float32)] * cfg.layers, "final_norm": np.ones(cfg.hidden, np.float32)}
    T = 24
    toks = [int(t) for t in np.random.default_rng(2).integers(0, cfg.vocab, T)]
    og, oa = ol.LlamaOracle(cfg, ex, T, orc.GENERIC), ol.LlamaOracle(cfg, ex, T, orc.AVX2)
    first, errs = None, []
    for p in range(T):
        rg, ra = {}, {}
        lg, la = og.step(toks[p], p, rg), oa.step(toks[p], p, ra)
        errs.append(rel_err(la, lg))
        if first is None:
            for li in range(cfg.layers):
                if kv_rel(oa.kc, oa.vc, og.kc, og.vc, li, p) > 5e-5:
                    first, rec = (p, li), (rg, ra)
                    break
            if first is None:
                assert errs[-1] < 1e-4, (p, errs[-1])  # before the chains part: f32 noise
    assert first is not None
    p, li = first
    rg, ra = rec
    lays = range(max(0, li - 1), li + 1)
    assert_tie("AVX2 vs generic chain", first_flip({l: quant_inputs_from_record(ra, l) for l in lays},
                                                   {l: quant_inputs_from_record(rg, l) for l in lays}, li))
    assert max(errs[p + 1:]) > 1e-2
