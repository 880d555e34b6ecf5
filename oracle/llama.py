"""CPU restatement of the reference's Llama decode step (TEST INFRASTRUCTURE ONLY).

One token at position p through a Llama-3-shaped decoder whose projections
are quantized matmuls (oracle.matmul: Q8_K activation quantization + the
k-quant block dot), everything else f32:
  * embedding row gather, CausalLm embed (crates/llm/candle-llm/src/models/llama.rs:397-408);
  * per layer, LlamaLayer::forward / combine_ffn (llama.rs:913-975):
      h  = x + o(attn(rms_norm(x, input_ln)))
      x' = h + down(silu(gate(n)) * up(n)),  n = rms_norm(h, post_ln);
  * rms_norm = x / sqrt(mean(x^2) + eps) * w (primitives/nn.rs:22-31);
  * q/k/v projections, NeoX half-split RoPE on q and k (LlamaAttention::project,
    llama.rs:1066-1100; apply_rope, primitives/rope.rs:289-323) with Llama-3
    scaled inverse frequencies (Rope::llama3, rope.rs:117-150) and the
    cat(freqs, freqs) angle table (rope.rs:176-208);
  * KV append, repeat_kv over the GQA groups, eager attention for one query:
    softmax((q . k_j) * scale) then the weighted sum of v (attention.rs:154-186);
  * final rms_norm and the output head, greedy argmax with the lowest index
    on ties (primitives/sampler.rs:216-219).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline use this.
"""
from __future__ import annotations

import math
from typing import List

import numpy as np

from oracle import oracle as orc

f32 = np.float32


def llama3_inv_freq(head_dim: int, theta: float, factor: float, low: float, high: float, orig_ctx: float):
    """Rope::llama3 (rope.rs:117-150), every operation in f32."""
    half = head_dim // 2
    low_wl = f32(orig_ctx) / f32(low)
    high_wl = f32(orig_ctx) / f32(high)
    two_pi = f32(2.0) * f32(math.pi)
    out = np.zeros(half, dtype=np.float32)
    for i in range(half):
        expo = f32(2 * i) / f32(head_dim)
        inv = f32(1.0) / f32(np.power(f32(theta), expo, dtype=np.float32))
        wl = two_pi / inv
        if wl > low_wl:
            out[i] = inv / f32(factor)
        elif wl < high_wl:
            out[i] = inv
        else:
            s = (f32(orig_ctx) / wl - f32(low)) / (f32(high) - f32(low))
            out[i] = (f32(1.0) - s) * inv / f32(factor) + s * inv
    return out


def cos_sin(inv_freq: np.ndarray, pos: int):
    """Rope::cos_sin_at for one position, NeoX layout cat(freqs, freqs) (rope.rs:176-208)."""
    fr = (f32(pos) * inv_freq).astype(np.float32)
    emb = np.concatenate([fr, fr])
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [..., dim]: x * cos + cat(-x2, x1) * sin (rope.rs:315-321)."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return (x * cos + rot * sin).astype(np.float32)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """primitives/nn.rs:22-31: x / sqrt(mean(x^2) + eps) * w over the last axis."""
    x = np.asarray(x, dtype=np.float32)
    ms = (x * x).mean(axis=-1, keepdims=True, dtype=np.float32)
    den = np.sqrt(ms + f32(eps)).astype(np.float32)
    return (x / den * w).astype(np.float32)


def silu(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.float32)
    return (v / (f32(1.0) + np.exp(-v, dtype=np.float32))).astype(np.float32)


def attend_one(q: np.ndarray, keys: np.ndarray, values: np.ndarray, scale: float) -> np.ndarray:
    """One query over positions 0..n-1 of one kv head: softmax(q.k * scale) @ v (attention.rs:154-186)."""
    s = (keys.astype(np.float32) @ q.astype(np.float32)).astype(np.float32) * f32(scale)
    e = np.exp(s - s.max(), dtype=np.float32)
    p = (e / e.sum(dtype=np.float32)).astype(np.float32)
    return (p @ values.astype(np.float32)).astype(np.float32)


def argmax_first(logits: np.ndarray) -> int:
    """Greedy argmax, lowest index on ties (sampler.rs:216-219)."""
    return int(np.argmax(np.asarray(logits, dtype=np.float32)))


class LlamaOracle:
    """CPU decoder over exported weights: ex['layers'][l][name] GGML bytes, f32 embed and norms.

    cfg provides layers, hidden, ffn, heads, kv_heads, head_dim, vocab, eps, dtypes (GGML type per
    projection name) and the Llama-3 RoPE parameters.
    """

    def __init__(self, cfg, ex: dict, max_seq: int, impl: int = orc.GENERIC):
        """impl picks the vec_dot bodies (orc.GENERIC: candle's generic ones, the reference's default
        build; orc.AVX2: its AVX2 + FMA ones). Both give the same integer block dots."""
        self.cfg, self.ex, self.max_seq, self.impl = cfg, ex, max_seq, impl
        self.inv_freq = llama3_inv_freq(cfg.head_dim, cfg.rope_theta, cfg.rope_factor, cfg.rope_low,
                                        cfg.rope_high, cfg.rope_orig_ctx)
        self.scale = float(f32(cfg.head_dim) ** f32(-0.5))
        kv = (cfg.layers, cfg.kv_heads, max_seq, cfg.head_dim)
        self.kc = np.zeros(kv, dtype=np.float32)
        self.vc = np.zeros(kv, dtype=np.float32)

    def _mm(self, name: str, li: int, x: np.ndarray, k: int) -> np.ndarray:
        w = self.ex["head"] if name == "head" else self.ex["layers"][li][name]
        return orc.matmul(int(self.cfg.dtypes[name]), x.reshape(1, k), w, k, impl=self.impl)[0]

    def step(self, token: int, pos: int, record: dict = None) -> np.ndarray:
        """Logits of the token at `pos` (the cache holds positions < pos). With `record`, record[layer]
        receives the f32 inputs of the layer's four activation quantizations: "n_attn" (normalised
        x before q/k/v), "att" (attention output before o), "n_ffn" (normalised x before gate/up) and
        "hmid" (silu(gate) * up before down), plus "x_attn" / "x_ffn" (the residual before each norm)."""
        c = self.cfg
        hd, H = c.head_dim, c.hidden
        x = self.ex["embed"][token].astype(np.float32).copy()
        cos, sin = cos_sin(self.inv_freq, pos)
        groups = c.heads // c.kv_heads
        for li in range(c.layers):
            n = rms_norm(x, self.ex["attn_norm"][li], c.eps)
            rec = record.setdefault(li, {}) if record is not None else {}
            rec["x_attn"], rec["n_attn"] = x, n
            q = self._mm("q", li, n, H).reshape(c.heads, hd)
            k = self._mm("k", li, n, H).reshape(c.kv_heads, hd)
            v = self._mm("v", li, n, H).reshape(c.kv_heads, hd)
            q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
            self.kc[li, :, pos] = k
            self.vc[li, :, pos] = v
            att = np.stack([attend_one(q[h], self.kc[li, h // groups, : pos + 1],
                                       self.vc[li, h // groups, : pos + 1], self.scale) for h in range(c.heads)])
            rec["att"] = att.reshape(-1)
            x = (x + self._mm("o", li, att.reshape(-1), c.heads * hd)).astype(np.float32)
            n = rms_norm(x, self.ex["ffn_norm"][li], c.eps)
            rec["x_ffn"], rec["n_ffn"] = x, n
            hmid = (silu(self._mm("gate", li, n, H)) * self._mm("up", li, n, H)).astype(np.float32)
            rec["hmid"] = hmid
            x = (x + self._mm("down", li, hmid, c.ffn)).astype(np.float32)
        return self._mm("head", 0, rms_norm(x, self.ex["final_norm"], c.eps), H)

    def generate(self, prompt: List[int], steps: int) -> List[int]:
        """Greedy continuation: prompt tokens are fed in order, then argmax tokens."""
        toks = list(prompt)
        for p in range(len(prompt) + steps - 1):
            lg = self.step(toks[p], p)
            if p + 1 >= len(toks):
                toks.append(argmax_first(lg))
        return toks
