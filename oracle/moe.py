"""CPU restatement of the reference's mixture-of-experts FFN (TEST INFRASTRUCTURE ONLY).

Follows MoeMlp::forward, crates/llm/candle-llm/src/models/llama.rs:1416-1487:
  * probabilities = softmax over the router logits (f32);
  * per token, the top-k experts by probability (ties: lower expert index);
  * weights renormalised over the selected experts (norm_topk_prob), or, when
    not renormalising, times routed_scaling_factor: row[e] / denom * post_scale
    with (denom, post_scale) = (sum, 1) or (1, routed_scaling_factor), :1436-1451;
  * each expert runs LlamaMlp::forward (llama.rs:1386-1391) on its tokens:
    down(silu(gate(x)) * up(x)) with the quantized matmuls of oracle.matmul;
  * the weighted expert outputs are index_add-ed onto zeros in increasing
    expert order (:1461-1474);
  * the always-on shared expert (a LlamaMlp over every token), scaled per
    token by sigmoid(x . shared_gate) when the model has that gate (Qwen2-MoE;
    DeepSeek-V2 adds it ungated), is added last: out + shared (:1476-1486).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline use this.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as orc


def softmax_f32(logits: np.ndarray) -> np.ndarray:
    l = np.asarray(logits, dtype=np.float32)
    mx = l.max(axis=-1, keepdims=True)
    e = np.exp(l - mx, dtype=np.float32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


def route(logits: np.ndarray, k: int, renormalize: bool = True, routed_scaling_factor: float = 1.0):
    """Per token: (experts[k], weights[k]) with experts in descending probability."""
    p = softmax_f32(logits)
    experts, weights = [], []
    for row in p:
        idx = sorted(range(len(row)), key=lambda e: (-float(row[e]), e))[:k]
        sel = np.array([row[e] for e in idx], dtype=np.float32)
        if renormalize:
            denom = np.float32(0.0)
            for v in sel:
                denom = np.float32(denom + v)
            denom = max(denom, np.float32(np.finfo(np.float32).tiny))
            sel = (sel / denom).astype(np.float32)
        else:
            sel = ((sel / np.float32(1.0)) * np.float32(routed_scaling_factor)).astype(np.float32)
        experts.append(idx)
        weights.append(sel)
    return experts, weights


def sigmoid_f32(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.float32)
    return (np.float32(1.0) / (np.float32(1.0) + np.exp(-v, dtype=np.float32))).astype(np.float32)


def silu_f32(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.float32)
    return (v / (np.float32(1.0) + np.exp(-v, dtype=np.float32))).astype(np.float32)


def mlp(x: np.ndarray, gate: bytes, up: bytes, down: bytes, dt_gu: int, dt_down: int, hidden: int, ffn: int):
    """LlamaMlp::forward with quantized projections (rows of x through gate/up/down)."""
    g = orc.matmul(dt_gu, x, gate, hidden)
    u = orc.matmul(dt_gu, x, up, hidden)
    h = (silu_f32(g) * u).astype(np.float32)
    return orc.matmul(dt_down, h, down, ffn)


def moe_ffn(x, logits, gate_experts, up_experts, down_experts, dt_gu, dt_down, k, renormalize=True,
            routed_scaling_factor=1.0, shared=None, shared_gate=None):
    """x f32 [T, H]; *_experts: per-expert GGML byte arrays ([F, H] for gate/up, [H, F] for down);
    shared: (gate, up, down, dt_gu, dt_down) GGML bytes of the shared expert ([Fs, H], [Fs, H], [H, Fs]);
    shared_gate: its f32 [H] sigmoid gate vector (None: ungated)."""
    x = np.asarray(x, dtype=np.float32)
    T, H = x.shape
    E = len(gate_experts)
    F = np.asarray(gate_experts[0]).size // orc.row_bytes(dt_gu, H)
    experts, weights = route(logits, k, renormalize, routed_scaling_factor)
    out = np.zeros((T, H), dtype=np.float32)
    for e in range(E):
        toks = [(t, weights[t][experts[t].index(e)]) for t in range(T) if e in experts[t]]
        if not toks:
            continue
        idx = [t for t, _ in toks]
        w = np.array([wt for _, wt in toks], dtype=np.float32)[:, None]
        ye = mlp(x[idx], gate_experts[e], up_experts[e], down_experts[e], dt_gu, dt_down, H, F)
        ye = (ye * w).astype(np.float32)
        for j, t in enumerate(idx):
            out[t] = (out[t] + ye[j]).astype(np.float32)
    if shared is None:
        return out
    sgate, sup, sdown, sdt_gu, sdt_down = shared
    Fs = np.asarray(sgate).size // orc.row_bytes(sdt_gu, H)
    sh = mlp(x, sgate, sup, sdown, sdt_gu, sdt_down, H, Fs)
    if shared_gate is not None:
        sg = sigmoid_f32((x @ np.asarray(shared_gate, np.float32)).astype(np.float32))
        sh = (sh * sg[:, None]).astype(np.float32)
    return (out + sh).astype(np.float32)
