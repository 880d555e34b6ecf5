"""Config 3 as stated: the 32-layer Llama-3-8B-shape Q4_K_M model (random init, seed 4), a
128-token prompt through the batched prefill, then 256 greedy tokens on the captured step graph
(positions 127..382), against the CPU decode oracle. The reference runs this loop at
crates/llm/candle-llm/src/decode/stream.rs:246-305 over the layer stack of models/llama.rs:671-709.

Checked here:
* op level (the 1e-3 * rms gate of every matmul, exact RoPE / KV append / argmax, attention 1e-4):
  the prefill's m = 127 launches at layers 0, 15 and 31, and the token step's launches at the same
  layers at positions 127, 255 and 382, each against the oracle applied to the device's own inputs;
* end to end: the oracle runs its own chain over all 383 positions, fed the device's tokens, once
  with candle's generic vec_dot bodies (the reference's default build) and once with its AVX2
  bodies (same integer block dots, another f32 summation order). The device's logits are compared
  with the generic chain at every generated position, next to the AVX2 chain's distance from it:
  the reference's own spread between two of its builds. On this random-init 32-layer stack that
  spread is large (max|d|/rms of the logits ~0.4, cosine ~0.995: every last-bit difference that
  lands on a Q8_K rounding tie moves an activation by a quantum, and the stack amplifies it), so
  the bar is that the device's distance stays within 1.25x of it in median and maximum, and that
  the device's greedy token leaves the generic chain's argmax at most 1.25x as often as the AVX2
  chain's does;
* where the chains part: the first (position, layer) whose K/V rows leave f32 noise, and at that
  position the activation quantizations just before it, re-run on the device and in the oracle.
  The first op whose Q8_K codes differ must differ by one quantum at elements whose pre-rounding
  value sits at a rounding tie (or at a tie between a block's two largest magnitudes), with the
  inputs still equal to f32 noise: a requantizing chain amplifies a last-bit difference there, not
  an op error. The same is shown between the two CPU chains.
"""
import numpy as np
import pytest
import torch

from decode_check import (OpChecker, PrefillChecker, assert_tie, cosine, device_rms_norm, first_flip, kv_rel, log,
                          quant_inputs_from_record, rel_err, snap)
from inference_amd.llama_decode import DecodeSession, LlamaConfig, LlamaWeights
from oracle import llama as ol
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

PROMPT, GEN = 128, 256
LAYERS = (0, 15, 31)
POSITIONS = (127, 255, 382)
KV_NOISE = 5e-5  # K/V rows further apart than this (max|d| / rms) have left f32 noise


class DeviceQuantInputs:
    """Token-step trace: the device's inputs to the four activation quantizations of chosen layers
    (norms applied with the oracle's rms_norm; SiLU*mul formed from the device's gate/up)."""

    def __init__(self, sess, ex, layers):
        self.s, self.ex, self.layers, self.out = sess, ex, set(layers), {}

    def __call__(self, op, li):
        if li not in self.layers:
            return
        s, c, ex = self.s, self.s.cfg, self.ex
        d = self.out.setdefault(li, {})
        if op == "qkv":
            d["n_attn"] = ol.rms_norm(snap(s.x), ex["attn_norm"][li], c.eps)
        elif op == "attention":
            d["att"] = snap(s.attn)
        elif op == "gate_up":
            d["n_ffn"] = ol.rms_norm(snap(s.x), ex["ffn_norm"][li], c.eps)
            d["hmid"] = (ol.silu(snap(s.g)) * snap(s.u)).astype(np.float32)


class PrefillQuantInputs:
    """Prefill trace: the same inputs for one row of the batched pass."""

    def __init__(self, sess, ex, layers, row):
        self.s, self.ex, self.layers, self.row, self.out = sess, ex, set(layers), row, {}

    def __call__(self, op, li, b):
        if li not in self.layers:
            return
        w, c, r = self.s.w, self.s.cfg, self.row
        d = self.out.setdefault(li, {})
        # the batched matmuls quantize the library's RMSNorm of the rows: the exact input is available
        if op == "qkv":
            d["n_attn"] = device_rms_norm(b["x"][r], w.attn_norm[li], c.eps)
        elif op == "attention":
            d["att"] = snap(b["att"][r])
        elif op == "gate_up":
            d["n_ffn"] = device_rms_norm(b["x"][r], w.ffn_norm[li], c.eps)
        elif op == "silu_mul":
            d["hmid"] = snap(b["h"][r])


@pytest.mark.timeout(900)
def test_config3_full_workload():
    dev = torch.device("cuda:0")
    cfg = LlamaConfig.llama3_8b()
    max_seq = PROMPT + GEN
    log("[config3] building the 8B-shape Q4_K_M model (seed 4)")
    w = LlamaWeights.random(cfg, 4, dev)
    prompt = [int(t) for t in np.random.default_rng(4).integers(0, cfg.vocab, PROMPT)]
    ex = w.export()

    # ---- device run: batched prefill, then 256 steps (traced at the sampled positions) ----
    sess = DecodeSession(w, max_seq)
    sess.reset(prompt)
    pchk = PrefillChecker(sess, ex, LAYERS)
    rows = sess.prefill(trace=pchk)
    assert rows == PROMPT - 1
    log("[config3] prefill m=127 op level: " + str({k: f"{v:.1e}" for k, v in pchk.worst.items()}))
    hist = torch.zeros((GEN, cfg.vocab), dtype=torch.float32, device=dev)
    chk = OpChecker(sess, ex, LAYERS)
    i = 0
    for p in POSITIONS:
        n = p - (PROMPT - 1 + i)
        if n:
            sess.run(n, history=hist[i:i + n])
            i += n
        sess.run(1, trace=chk, history=hist[i:i + 1])
        i += 1
    assert i == GEN and chk.steps == len(POSITIONS)
    assert sorted(set(chk.checked)) == sorted((p, li) for p in POSITIONS for li in LAYERS)
    log("[config3] step op level at positions 127/255/382, layers 0/15/31: "
        + str({k: f"{v:.1e}" for k, v in chk.worst.items()}))
    for p, li, name, near, plain, net in chk.ties:
        log(f"[config3]   fused-norm {name} at position {p} layer {li}: {near} near-tie activation elements, "
            f"max|d|/rms {plain:.2e}, {net:.2e} net of their exact contributions")
    toks = sess.generated(max_seq)
    assert toks[:PROMPT] == prompt
    H = hist.cpu().numpy()
    kc_dev, vc_dev = snap(sess.kcache), snap(sess.vcache)

    # ---- the two oracle chains in lockstep, fed the device's tokens ----
    og = ol.LlamaOracle(cfg, ex, max_seq, orc.GENERIC)
    oa = ol.LlamaOracle(cfg, ex, max_seq, orc.AVX2) if orc.simd_supported() else None
    dev_first = avx_first = None
    dev_rec = avx_rec = None
    err_dev, err_avx, cos_dev, cos_avx, flips, avx_flips = {}, {}, {}, {}, [], []
    for p in range(max_seq - 1):
        rg, ra = {}, {}
        lg = og.step(toks[p], p, rg)
        la = oa.step(toks[p], p, ra) if oa is not None else None
        if dev_first is None:
            for li in range(cfg.layers):
                if kv_rel(kc_dev, vc_dev, og.kc, og.vc, li, p) > KV_NOISE:
                    dev_first, dev_rec = (p, li), rg
                    break
        if oa is not None and avx_first is None:
            for li in range(cfg.layers):
                if kv_rel(oa.kc, oa.vc, og.kc, og.vc, li, p) > KV_NOISE:
                    avx_first, avx_rec = (p, li), (rg, ra)
                    break
        if p >= PROMPT - 1:
            h = H[p - (PROMPT - 1)]
            err_dev[p], cos_dev[p] = rel_err(h, lg), cosine(h, lg)
            want = ol.argmax_first(lg)
            if la is not None:
                err_avx[p], cos_avx[p] = rel_err(la, lg), cosine(la, lg)
                if ol.argmax_first(la) != want:
                    avx_flips.append(p)
            if toks[p + 1] != want:
                gap = float(lg[want] - lg[toks[p + 1]])
                flips.append((p, gap))
                assert gap <= 2.0 * float(np.abs(h - lg).max()), (p, want, toks[p + 1], gap)
        if p % 64 == 0:
            log(f"[config3] oracle chains at position {p}")
    log(f"[config3] logits max|d|/rms vs the generic chain at positions {POSITIONS}: device "
        + " ".join(f"{err_dev[p]:.2e}" for p in POSITIONS)
        + (" | AVX2 chain " + " ".join(f"{err_avx[p]:.2e}" for p in POSITIONS) if err_avx else ""))
    ed, ea = np.array(list(err_dev.values())), np.array(list(err_avx.values()))
    cd, ca = np.array(list(cos_dev.values())), np.array(list(cos_avx.values()))
    log(f"[config3] over all 256 steps: device max {ed.max():.2e} median {np.median(ed):.2e} "
        f"cos min {cd.min():.5f} median {np.median(cd):.5f} | AVX2 chain max {ea.max():.2e} "
        f"median {np.median(ea):.2e} cos min {ca.min():.5f} median {np.median(ca):.5f}; "
        f"greedy tokens off the generic chain's argmax over the 256 teacher-forced steps: device "
        f"{len(flips)}, AVX2 chain {len(avx_flips)}")
    log(f"[config3] first K/V rows past f32 noise: device {dev_first}, AVX2 chain {avx_first}")

    # ---- the CPU chains: where the AVX2 chain leaves the generic one ----
    if avx_first is not None:
        p, li = avx_first
        rg, ra = avx_rec
        lays = range(max(0, li - 1), li + 1)
        found = first_flip({l: quant_inputs_from_record(ra, l) for l in lays},
                           {l: quant_inputs_from_record(rg, l) for l in lays}, li)
        assert_tie(f"AVX2 vs generic chain, position {p}", found)

    # ---- the device: re-run to the first divergent position and compare its quantizer inputs ----
    if dev_first is not None:
        p, li = dev_first
        lays = list(range(max(0, li - 1), li + 1))
        s2 = DecodeSession(w, max_seq)
        s2.reset(prompt)
        if p < PROMPT - 1:
            cap = PrefillQuantInputs(s2, ex, lays, p)
            s2.prefill(trace=cap)
        else:
            s2.prefill()
            if p > PROMPT - 1:
                s2.run(p - (PROMPT - 1))
            cap = DeviceQuantInputs(s2, ex, lays)
            s2.run(1, trace=cap)
        # the device is deterministic: the re-run wrote the same K/V rows
        np.testing.assert_array_equal(snap(s2.kcache[:, :, : p + 1]), kc_dev[:, :, : p + 1])
        found = first_flip(cap.out, {l: quant_inputs_from_record(dev_rec, l) for l in lays}, li)
        assert_tie(f"device vs generic chain, position {p}", found)

    # ---- the end-to-end bar: the device stays within the reference's own spread between two of its
    # builds (generic vs AVX2 vec_dot), in median and maximum over the 256 steps ----
    assert oa is not None, "the AVX2 chain (the reference's second build) needs an AVX2 + FMA host"
    assert np.median(ed) <= 1.25 * np.median(ea), (np.median(ed), np.median(ea))
    assert ed.max() <= 1.25 * ea.max(), (ed.max(), ea.max())
    assert np.median(cd) >= 1.0 - 1.25 * (1.0 - np.median(ca)), (np.median(cd), np.median(ca))
    assert cd.min() >= 1.0 - 1.25 * (1.0 - ca.min()), (cd.min(), ca.min())
    # greedy tokens: the device's argmax leaves the generic chain's no more often than the AVX2 build's
    # does (both fed the same tokens), within the same 1.25x
    assert len(flips) <= 1.25 * len(avx_flips), (len(flips), len(avx_flips))
