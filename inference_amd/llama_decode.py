"""Greedy decode of a Llama-style decoder whose projections run on the quantized path.

Mirrors the reference engine's decode for a Llama-3-shaped model
(CausalLm::decode_logits -> run_decoder_stack -> LlamaLayer::forward,
crates/llm/candle-llm/src/models/llama.rs:410-433, 654-725, 913-975, 1066-1120,
1386-1391; the loop of decode/stream.rs:246-305) with the GGUF Q4_K_M tensor
mix: Q4_K for attn_q/attn_k/attn_o/ffn_gate/ffn_up, Q6_K for attn_v/ffn_down
and the output head, dense f32 embedding and RMSNorm weights.

One token step is a fixed sequence of device launches (no host sync):
embedding gather; per layer q/k and v projections with RMSNorm fused into
their quantization prologue, RoPE + KV append, GQA attention, o projection
added into the residual, gate/up projections (norm fused), SiLU*mul -> Q8_K,
down projection added into the residual; final norm + head; greedy argmax
that writes the next token and advances the position. The position and the
token ids live in device memory, so the step is captured once into a HIP
graph and replayed for every token (prompt tokens are fed through the same
step: the argmax does not overwrite a slot that still holds a prompt token).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional

import numpy as np
import torch

from . import qmm
from .qmm import GgmlDType, QTensor

Q4K, Q6K = GgmlDType.Q4K, GgmlDType.Q6K


@dataclass
class LlamaConfig:
    layers: int = 32
    hidden: int = 4096
    ffn: int = 14336
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 128256
    rope_theta: float = 500000.0
    rope_factor: float = 8.0
    rope_low: float = 1.0
    rope_high: float = 4.0
    rope_orig_ctx: float = 8192.0
    eps: float = 1e-5
    # Q4_K_M tensor types
    dtypes: Dict[str, GgmlDType] = field(default_factory=lambda: {
        "q": Q4K, "k": Q4K, "v": Q6K, "o": Q4K, "gate": Q4K, "up": Q4K, "down": Q6K, "head": Q6K})

    @staticmethod
    def llama3_8b() -> "LlamaConfig":
        return LlamaConfig()

    def shapes(self) -> Dict[str, tuple]:
        return {"q": (self.heads * self.head_dim, self.hidden), "k": (self.kv_heads * self.head_dim, self.hidden),
                "v": (self.kv_heads * self.head_dim, self.hidden), "o": (self.hidden, self.heads * self.head_dim),
                "gate": (self.ffn, self.hidden), "up": (self.ffn, self.hidden), "down": (self.hidden, self.ffn),
                "head": (self.vocab, self.hidden)}

    def weight_bytes_per_token(self) -> int:
        """Quantized weight bytes streamed per decoded token (all layers + head)."""
        sh = self.shapes()
        total = 0
        for name, (n, k) in sh.items():
            dt = self.dtypes[name]
            b = n * (k // 256) * (144 if dt == Q4K else 210)
            total += b * (1 if name == "head" else self.layers)
        return total


def llama3_inv_freq(cfg: LlamaConfig) -> np.ndarray:
    """Rope::llama3 (crates/llm/candle-llm/src/primitives/rope.rs:117-150), f32 arithmetic."""
    f32 = np.float32
    dim = cfg.head_dim
    low_wl = f32(cfg.rope_orig_ctx) / f32(cfg.rope_low)
    high_wl = f32(cfg.rope_orig_ctx) / f32(cfg.rope_high)
    out = np.empty(dim // 2, dtype=np.float32)
    for i in range(dim // 2):
        inv = f32(1.0) / np.power(f32(cfg.rope_theta), f32(2 * i) / f32(dim), dtype=np.float32)
        wavelen = f32(2.0) * f32(math.pi) / inv
        if wavelen > low_wl:
            out[i] = inv / f32(cfg.rope_factor)
        elif wavelen < high_wl:
            out[i] = inv
        else:
            smooth = (f32(cfg.rope_orig_ctx) / wavelen - f32(cfg.rope_low)) / (f32(cfg.rope_high) - f32(cfg.rope_low))
            out[i] = (f32(1.0) - smooth) * inv / f32(cfg.rope_factor) + smooth * inv
    return out


def rope_tables(cfg: LlamaConfig, max_seq: int):
    """cos/sin [max_seq][head_dim] of Rope::cos_sin_at (NeoX: cat(freqs, freqs)), rope.rs:176-208."""
    inv = llama3_inv_freq(cfg)
    pos = np.arange(max_seq, dtype=np.float32)[:, None]
    freqs = (pos * inv[None, :]).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


class LlamaWeights:
    """Device weights: quantized projections per layer, dense f32 embedding and norms."""

    def __init__(self, cfg: LlamaConfig, layers: List[Dict[str, QTensor]], head: QTensor, embed: torch.Tensor,
                 attn_norm: List[torch.Tensor], ffn_norm: List[torch.Tensor], final_norm: torch.Tensor):
        self.cfg = cfg
        self.layers = layers
        self.head = head
        self.embed = embed
        self.attn_norm = attn_norm
        self.ffn_norm = ffn_norm
        self.final_norm = final_norm

    @classmethod
    def random(cls, cfg: LlamaConfig, seed: int, device: torch.device, std: float = 0.02) -> "LlamaWeights":
        """N(0, std^2) weights, quantized on the GPU; norms = 1. Each tensor is SplitMix64 + Box-Muller
        (synth.normal_torch, generated on the device, the same values as synth.normal on the host) with
        its own seed: seed * 1000003 + 16 * layer + j for projection j of q, k, v, o, gate, up, down, then
        16 * layers for the head and 16 * layers + 1 for the embedding."""
        from .synth import normal_torch
        sh = cfg.shapes()
        base = seed * 1000003

        def q(name, s):
            w = normal_torch(base + s, sh[name], std, device)
            t = QTensor.quantize(w, cfg.dtypes[name])
            del w
            return t

        names = ("q", "k", "v", "o", "gate", "up", "down")
        layers = [{name: q(name, 16 * li + j) for j, name in enumerate(names)} for li in range(cfg.layers)]
        head = q("head", 16 * cfg.layers)
        embed = normal_torch(base + 16 * cfg.layers + 1, (cfg.vocab, cfg.hidden), std, device)
        ones = lambda: torch.ones(cfg.hidden, dtype=torch.float32, device=device)  # noqa: E731
        return cls(cfg, layers, head, embed, [ones() for _ in range(cfg.layers)],
                   [ones() for _ in range(cfg.layers)], ones())

    @classmethod
    def from_gguf(cls, path, device: torch.device) -> "LlamaWeights":
        """Resident load of a llama-architecture GGUF file (the engine's GgufCheckpoint::open,
        crates/llm/candle-llm/src/gguf.rs:63-170, without its dequantize -> re-quantize): projections
        go straight into device QTensors (q/k rows un-permuted from llama.cpp's order on the quantized
        rows), the token embedding is dequantized to f32 on the device, norms are read as f32, and a
        missing output.weight ties the head to the embedding's quantized tensor. The configuration
        follows reconstruct_config (gguf.rs:361-428): absent llama3 RoPE-scaling keys mean standard
        RoPE (factor 1)."""
        from .gguf import GgufFile, GGML_Q4K, GGML_Q6K
        f = path if isinstance(path, GgufFile) else GgufFile.open(path)
        arch = f.meta_str("general.architecture")
        if arch != "llama":
            raise qmm.QmmError(qmm.QMM_ERR_UNSUPPORTED, f"gguf: architecture {arch!r} (llama only)")

        def req(k):
            v = f.meta_u64(f"{arch}.{k}")
            if v is None:
                raise qmm.QmmError(qmm.QMM_ERR_INVALID, f"gguf: missing metadata {arch}.{k}")
            return v

        heads = req("attention.head_count")
        kv = f.meta_u64(f"{arch}.attention.head_count_kv") or heads
        hidden = req("embedding_length")
        head_dim = f.meta_u64(f"{arch}.attention.key_length") or hidden // heads
        infos = {t.name: t for t in f.tensors}
        if "token_embd.weight" not in infos:
            raise qmm.QmmError(qmm.QMM_ERR_INVALID, "gguf: no token embedding tensor")
        low = f.meta_f64(f"{arch}.rope.scaling.low_freq_factor")
        high = f.meta_f64(f"{arch}.rope.scaling.high_freq_factor")
        llama3 = f.meta_str(f"{arch}.rope.scaling.type") == "llama3" or low is not None or high is not None
        cfg = LlamaConfig(
            layers=req("block_count"), hidden=hidden, ffn=req("feed_forward_length"), heads=heads, kv_heads=kv,
            head_dim=head_dim, vocab=infos["token_embd.weight"].shape[0],
            rope_theta=f.meta_f64(f"{arch}.rope.freq_base") or 10000.0,
            rope_factor=(f.meta_f64(f"{arch}.rope.scaling.factor") or 8.0) if llama3 else 1.0,
            rope_low=low if low is not None else 1.0, rope_high=high if high is not None else 4.0,
            rope_orig_ctx=float(f.meta_u64(f"{arch}.rope.scaling.original_context_length") or 8192),
            eps=f.meta_f64(f"{arch}.attention.layer_norm_rms_epsilon") or 1e-5)

        def tensor(name):
            if name not in infos:
                raise qmm.QmmError(qmm.QMM_ERR_INVALID, f"gguf: missing tensor {name}")
            return infos[name]

        names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
                 "up": "ffn_up", "down": "ffn_down"}
        layers, attn_norm, ffn_norm = [], [], []
        for li in range(cfg.layers):
            lw = {}
            for key, gname in names.items():
                info = tensor(f"blk.{li}.{gname}.weight")
                if info.ggml_type not in (GGML_Q4K, GGML_Q6K):
                    raise qmm.QmmError(qmm.QMM_ERR_UNSUPPORTED,
                                       f"gguf: {info.name} has GGML type {info.ggml_type} (Q4_K / Q6_K projections)")
                unperm = cfg.heads if key == "q" else cfg.kv_heads if key == "k" else 0
                lw[key] = f.load_qtensor(info, device, unperm)
            layers.append(lw)
            attn_norm.append(f.load_dense(tensor(f"blk.{li}.attn_norm.weight"), device).float())
            ffn_norm.append(f.load_dense(tensor(f"blk.{li}.ffn_norm.weight"), device).float())
        emb_info = infos["token_embd.weight"]
        embed = f.load_dense(emb_info, device).float().contiguous()
        head_info = infos.get("output.weight", emb_info)
        head = f.load_qtensor(head_info, device)
        cfg.dtypes = {k: v.dtype() for k, v in layers[0].items()}
        cfg.dtypes["head"] = head.dtype()
        return cls(cfg, layers, head, embed, attn_norm, ffn_norm,
                   f.load_dense(tensor("output_norm.weight"), device).float())

    def export(self) -> dict:
        """Host copies for the CPU reference: GGML bytes per tensor, f32 embedding and norms."""
        return {"layers": [{n: t.to_ggml() for n, t in lw.items()} for lw in self.layers],
                "head": self.head.to_ggml(), "embed": self.embed.cpu().numpy(),
                "attn_norm": [w.cpu().numpy() for w in self.attn_norm],
                "ffn_norm": [w.cpu().numpy() for w in self.ffn_norm], "final_norm": self.final_norm.cpu().numpy()}


class DecodeSession:
    """Device state and the launch sequence of one token step."""

    def __init__(self, weights: LlamaWeights, max_seq: int, warm_gate_up_rows: int = 3, warm: bool = True):
        """`warm`: the attention launch also loads the o projection's rows and the first
        `warm_gate_up_rows` gate/up rows of every wave of the following launches into the L2 of the XCD
        that reads them (qmm_decode_rope_attention_warm; the results are the same either way)."""
        cfg = weights.cfg
        self.cfg, self.w, self.max_seq = cfg, weights, max_seq
        dev = weights.embed.device
        self.dev = dev
        L = qmm.lib()
        self.L = L
        # the attention's geometry and cache length are checked before anything is allocated
        wsa = int(L.qmm_decode_attention_workspace_size(cfg.heads, cfg.kv_heads, cfg.head_dim, max_seq))
        if wsa == 0:
            raise qmm.QmmError(1, "unsupported attention geometry: " + qmm.last_error())
        f32 = dict(dtype=torch.float32, device=dev)
        self.x = torch.zeros(cfg.hidden, **f32)
        self.q = torch.zeros(cfg.heads * cfg.head_dim, **f32)
        self.k = torch.zeros(cfg.kv_heads * cfg.head_dim, **f32)
        self.v = torch.zeros(cfg.kv_heads * cfg.head_dim, **f32)
        self.attn = torch.zeros(cfg.heads * cfg.head_dim, **f32)
        self.g = torch.zeros(cfg.ffn, **f32)
        self.u = torch.zeros(cfg.ffn, **f32)
        self.hq = torch.zeros(cfg.ffn // 256 * 292, dtype=torch.uint8, device=dev)
        self.logits = torch.zeros(cfg.vocab, **f32)
        self.tokens = torch.zeros(max_seq, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        kv = (cfg.layers, cfg.kv_heads, max_seq, cfg.head_dim)
        self.kcache = torch.zeros(kv, **f32)
        self.vcache = torch.zeros(kv, **f32)
        cos, sin = rope_tables(cfg, max_seq)
        self.cos = torch.from_numpy(cos).to(dev)
        self.sin = torch.from_numpy(sin).to(dev)
        self.scale = float(np.float32(cfg.head_dim) ** np.float32(-0.5))
        self.prompt_len = 0
        self.steps_done = 0
        self._graph = None
        # workspaces of the attention (per-kv-head counters, then chunk partials) and of the
        # argmax; their counters start at zero and every launch leaves them at zero
        self.ws_attn = torch.zeros(wsa, dtype=torch.uint8, device=dev)
        self.ws_argmax = torch.zeros(int(L.qmm_greedy_workspace_size(cfg.vocab)), dtype=torch.uint8, device=dev)
        # launch arguments prepared once (ctypes arrays of handles / outputs)
        self._arr = []

        def arr(ctype, vals):
            a = (ctype * len(vals))(*vals)
            self._arr.append(a)
            return a

        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        # q, k (Q4_K) and v (Q6_K) share the normalised activation: one launch
        self._qkv = [arr(vp, [lw["q"].handle.value, lw["k"].handle.value, lw["v"].handle.value])
                     for lw in weights.layers]
        self._qkv_y = arr(vp, [self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr()])
        self._qkv_ld = arr(i64, [self.q.numel(), self.k.numel(), self.v.numel()])
        self._o = [arr(vp, [lw["o"].handle.value]) for lw in weights.layers]
        self._x_y = arr(vp, [self.x.data_ptr()])
        self._x_ld = arr(i64, [cfg.hidden])
        self._gu = [arr(vp, [lw["gate"].handle.value, lw["up"].handle.value]) for lw in weights.layers]
        self._gu_y = arr(vp, [self.g.data_ptr(), self.u.data_ptr()])
        self._gu_ld = arr(i64, [cfg.ffn, cfg.ffn])
        self._head = arr(vp, [weights.head.handle.value])
        self._lg_y = arr(vp, [self.logits.data_ptr()])
        self._lg_ld = arr(i64, [cfg.vocab])
        ci = ctypes.c_int
        self._warm = [arr(vp, [lw["o"].handle.value, lw["gate"].handle.value, lw["up"].handle.value])
                      for lw in weights.layers] if warm else None
        self._warm_launch = arr(ci, [0, 1, 1])
        self._warm_rows = arr(ci, [1, int(warm_gate_up_rows)])

    # -- one token step --------------------------------------------------
    def step(self, trace: Optional[Callable[[str, int], None]] = None):
        """Enqueue one token step on the current stream (no host synchronisation).

        `trace(op, layer)`, when given, is called after each launch is enqueued (ops: embed, qkv,
        attention (RoPE + KV append + attention in one launch), o, gate_up, silu_mul, down, head,
        argmax); it lets a checker inspect the session's buffers between launches. Captured steps
        take no trace.
        """
        cfg, L, w = self.cfg, self.L, self.w
        s = qmm._stream(self.dev)
        eps = ctypes.c_float(cfg.eps)
        hd, H = cfg.head_dim, cfg.hidden
        tr = trace if trace is not None else (lambda op, li: None)
        qmm._check(L.qmm_embed_rows(w.embed.data_ptr(), H, cfg.vocab, self.tokens.data_ptr(), self.pos.data_ptr(),
                                    self.x.data_ptr(), H, s))
        tr("embed", -1)
        kv_stride = cfg.kv_heads * self.max_seq * hd
        for li in range(cfg.layers):
            an, fn = w.attn_norm[li].data_ptr(), w.ffn_norm[li].data_ptr()
            qmm._check(L.qmm_matmul_ex(self._qkv[li], 3, self.x.data_ptr(), 1, H, an, eps, 0, self._qkv_y,
                                       self._qkv_ld, None, 0, s))
            tr("qkv", li)
            kc = self.kcache.data_ptr() + 4 * li * kv_stride
            vc = self.vcache.data_ptr() + 4 * li * kv_stride
            if self._warm is not None:
                # the o / gate / up launches' first rows are loaded into L2 during the attention
                qmm._check(L.qmm_decode_rope_attention_warm(
                    self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.cos.data_ptr(),
                    self.sin.data_ptr(), self.pos.data_ptr(), kc, vc, self.attn.data_ptr(), cfg.heads,
                    cfg.kv_heads, hd, self.max_seq, ctypes.c_float(self.scale), self.ws_attn.data_ptr(),
                    self.ws_attn.numel(), self._warm[li], self._warm_launch, 3, self._warm_rows, s))
            else:
                qmm._check(L.qmm_decode_rope_attention(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                                                       self.cos.data_ptr(), self.sin.data_ptr(),
                                                       self.pos.data_ptr(), kc, vc, self.attn.data_ptr(),
                                                       cfg.heads, cfg.kv_heads, hd, self.max_seq,
                                                       ctypes.c_float(self.scale), self.ws_attn.data_ptr(),
                                                       self.ws_attn.numel(), s))
            tr("attention", li)
            qmm._check(L.qmm_matmul_ex(self._o[li], 1, self.attn.data_ptr(), 1, cfg.heads * hd, None, eps, 1,
                                       self._x_y, self._x_ld, None, 0, s))
            tr("o", li)
            qmm._check(L.qmm_matmul_ex(self._gu[li], 2, self.x.data_ptr(), 1, H, fn, eps, 0, self._gu_y,
                                       self._gu_ld, None, 0, s))
            tr("gate_up", li)
            # silu(gate) * up -> Q8_K in its own launch, then down (qmm_silu_mul_matmul fuses the two, but
            # every GEMV workgroup would then recompute the 14336-wide activation: 2.5 us slower per layer)
            qmm._check(L.qmm_silu_mul_quantize(self.g.data_ptr(), self.u.data_ptr(), 1, cfg.ffn, cfg.ffn,
                                               self.hq.data_ptr(), s))
            tr("silu_mul", li)
            qmm._check(L.qmm_matmul_q_ex(w.layers[li]["down"].handle, self.hq.data_ptr(), 1, self.x.data_ptr(), H,
                                         1, None, 0, s))
            tr("down", li)
        qmm._check(L.qmm_matmul_ex(self._head, 1, self.x.data_ptr(), 1, H, w.final_norm.data_ptr(), eps, 0,
                                   self._lg_y, self._lg_ld, None, 0, s))
        tr("head", -1)
        qmm._check(L.qmm_greedy_advance(self.logits.data_ptr(), cfg.vocab, self.tokens.data_ptr(), self.max_seq,
                                        self.pos.data_ptr(), self.prompt_len, self.ws_argmax.data_ptr(),
                                        self.ws_argmax.numel(), s))
        tr("argmax", -1)

    # -- batched prefill -----------------------------------------------------
    def prefill(self, trace: Optional[Callable[[str, int, Dict[str, torch.Tensor]], None]] = None) -> int:
        """Run the prompt's positions 0 .. prompt_len - 2 in one pass per layer (matmuls with m = rows on
        the MFMA GEMM path, batched RoPE + KV append, causal attention over the prompt), then leave the
        session at position prompt_len - 1, where the captured step takes over: it processes the last
        prompt token and produces the first generated one. Same operations and order per row as the
        token-by-token steps, so the KV cache and the following logits match them to f32 accumulation
        order. Returns the number of rows run. Call right after reset().

        `trace(op, layer, bufs)`, when given, is called after each launch is enqueued (ops: embed, qkv,
        rope_kv, attention, o, gate_up, silu_mul, down); `bufs` holds the pass's row buffers (x, q, k, v,
        att, g, u, h), so a checker can read them between launches. Without a trace the feed-forward
        block is one qmm_ffn call (gate / up split sums, SiLU and the down GEMM's quantization in one
        launch), which gives the same bits as those three traced launches; likewise q / k / v with RoPE
        and the KV append are one qmm_qkv_rope_kv_append_n call. Without a trace the last layer also
        stops after its K/V append: the rows' hidden states after it feed nothing (the step recomputes
        the last prompt token's), so its attention, o and feed-forward block over the rows are skipped."""
        if self.prompt_len == 0 or self.steps_done != 0:
            raise qmm.QmmError(1, "prefill() needs the state reset() leaves")
        cfg, L, w = self.cfg, self.L, self.w
        rows = self.prompt_len - 1
        if rows == 0:
            return 0
        dev, s = self.dev, qmm._stream(self.dev)
        H, F, hd = cfg.hidden, cfg.ffn, cfg.head_dim
        nq, nkv = cfg.heads * hd, cfg.kv_heads * hd
        f32 = dict(dtype=torch.float32, device=dev)
        x = torch.empty((rows, H), **f32)
        q = torch.empty((rows, nq), **f32)
        k = torch.empty((rows, nkv), **f32)
        v = torch.empty((rows, nkv), **f32)
        att = torch.empty((rows, nq), **f32)
        g = torch.empty((rows, F), **f32)
        u = torch.empty((rows, F), **f32)
        hh = torch.empty((rows, F), **f32)
        wsb = 0
        for lw in w.layers:
            for t in lw.values():
                wsb = max(wsb, int(L.qmm_matmul_ex_workspace_size(t.handle, rows, 1)))
            if trace is None:
                wsb = max(wsb, int(L.qmm_ffn_workspace_size(lw["gate"].handle, lw["up"].handle,
                                                             lw["down"].handle, rows, 1)),
                          int(L.qmm_qkv_rope_kv_append_n_workspace_size(lw["q"].handle, lw["k"].handle,
                                                                        lw["v"].handle, rows, 1)),
                          int(L.qmm_prefill_attention_o_workspace_size(lw["o"].handle, rows)))
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        eps = ctypes.c_float(cfg.eps)
        qkv_y = (vp * 3)(q.data_ptr(), k.data_ptr(), v.data_ptr())
        qkv_ld = (i64 * 3)(nq, nkv, nkv)
        x_y, x_ld = (vp * 1)(x.data_ptr()), (i64 * 1)(H)
        gu_y, gu_ld = (vp * 2)(g.data_ptr(), u.data_ptr()), (i64 * 2)(F, F)
        kv_stride = cfg.kv_heads * self.max_seq * hd
        bufs = {"x": x, "q": q, "k": k, "v": v, "att": att, "g": g, "u": u, "h": hh}
        tr = (lambda op, li: trace(op, li, bufs)) if trace is not None else (lambda op, li: None)
        qmm._check(L.qmm_embed_rows_n(w.embed.data_ptr(), H, cfg.vocab, self.tokens.data_ptr(), 0, rows, x.data_ptr(),
                                      H, s))
        tr("embed", -1)
        for li in range(cfg.layers):
            lw = w.layers[li]
            kc = self.kcache.data_ptr() + 4 * li * kv_stride
            vc = self.vcache.data_ptr() + 4 * li * kv_stride
            if trace is None:
                qmm._check(L.qmm_qkv_rope_kv_append_n(lw["q"].handle, lw["k"].handle, lw["v"].handle, x.data_ptr(),
                                                      rows, H, w.attn_norm[li].data_ptr(), eps, self.cos.data_ptr(),
                                                      self.sin.data_ptr(), 0, q.data_ptr(), nq, kc, vc, cfg.heads,
                                                      cfg.kv_heads, hd, self.max_seq, ws.data_ptr(), ws.numel(), s))
                if li == cfg.layers - 1:
                    break  # the last layer's K/V is all that the following steps read
            else:
                qmm._check(L.qmm_matmul_ex(self._qkv[li], 3, x.data_ptr(), rows, H, w.attn_norm[li].data_ptr(), eps,
                                           0, qkv_y, qkv_ld, ws.data_ptr(), ws.numel(), s))
                tr("qkv", li)
                qmm._check(L.qmm_rope_kv_append_n(q.data_ptr(), k.data_ptr(), v.data_ptr(), nq, nkv, nkv,
                                                  self.cos.data_ptr(), self.sin.data_ptr(), 0, rows, kc, vc,
                                                  cfg.heads, cfg.kv_heads, hd, self.max_seq, s))
                tr("rope_kv", li)
            if trace is None:
                # attention + o + residual in one entry (the attention launch writes the o GEMM's planes)
                qmm._check(L.qmm_prefill_attention_o(q.data_ptr(), nq, kc, vc, 0, rows, cfg.heads, cfg.kv_heads, hd,
                                                     self.max_seq, ctypes.c_float(self.scale), lw["o"].handle,
                                                     x.data_ptr(), H, ws.data_ptr(), ws.numel(), s))
            else:
                qmm._check(L.qmm_prefill_attention(q.data_ptr(), nq, kc, vc, 0, rows, att.data_ptr(), nq, cfg.heads,
                                                   cfg.kv_heads, hd, self.max_seq, ctypes.c_float(self.scale), s))
                tr("attention", li)
                qmm._check(L.qmm_matmul_ex((vp * 1)(lw["o"].handle.value), 1, att.data_ptr(), rows, nq, None, eps, 1,
                                           x_y, x_ld, ws.data_ptr(), ws.numel(), s))
                tr("o", li)
            if trace is None:
                qmm._check(L.qmm_ffn(lw["gate"].handle, lw["up"].handle, lw["down"].handle, x.data_ptr(), rows, H,
                                     w.ffn_norm[li].data_ptr(), eps, 1, x.data_ptr(), H, ws.data_ptr(), ws.numel(),
                                     s))
                continue
            qmm._check(L.qmm_matmul_ex(self._gu[li], 2, x.data_ptr(), rows, H, w.ffn_norm[li].data_ptr(), eps, 0,
                                       gu_y, gu_ld, ws.data_ptr(), ws.numel(), s))
            tr("gate_up", li)
            qmm._check(L.qmm_silu_mul(g.data_ptr(), u.data_ptr(), hh.data_ptr(), rows * F, s))
            tr("silu_mul", li)
            qmm._check(L.qmm_matmul_ex((vp * 1)(lw["down"].handle.value), 1, hh.data_ptr(), rows, F, None, eps, 1,
                                       x_y, x_ld, ws.data_ptr(), ws.numel(), s))
            tr("down", li)
        self.pos.fill_(rows)
        self.steps_done = rows
        return rows

    # -- driver ------------------------------------------------------------
    def reset(self, prompt: List[int]):
        """Load a prompt; the next step processes position 0."""
        if len(prompt) < 1 or len(prompt) > self.max_seq:
            raise qmm.QmmError(1, f"prompt length {len(prompt)} outside 1..{self.max_seq}")
        if min(prompt) < 0 or max(prompt) >= self.cfg.vocab:
            raise qmm.QmmError(1, f"prompt token ids must lie in [0, {self.cfg.vocab})")
        if self.prompt_len != len(prompt):
            self._graph = None  # the prompt length is a launch argument of the captured step
        self.tokens.zero_()
        self.tokens[: len(prompt)] = torch.tensor(prompt, dtype=torch.int32, device=self.dev)
        self.pos.zero_()
        self.kcache.zero_()
        self.vcache.zero_()
        self.prompt_len = len(prompt)
        self.steps_done = 0

    def capture(self):
        """Capture one step into a HIP graph, from any state. An eager warm-up step (which loads the
        kernels) runs first and its effect is undone: the position and the token slot after it are
        restored; the KV rows it wrote at the position are written again, identically, by the next
        real step."""
        p = int(self.pos.item())
        nxt = self.tokens[p + 1].clone() if p + 1 < self.max_seq else None
        self.step()
        torch.cuda.synchronize()
        self.pos.fill_(p)
        if nxt is not None:
            self.tokens[p + 1] = nxt
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        torch.cuda.synchronize()
        self._graph = g

    def run(self, steps: int, use_graph: bool = True, history: Optional[torch.Tensor] = None,
            trace: Optional[Callable[[str, int], None]] = None):
        """Run `steps` token steps from the current position; with `history`, row i receives the
        logits of step i (copied between graph replays). A `trace` runs the steps eagerly."""
        if self.prompt_len == 0:
            raise qmm.QmmError(1, "reset() with a prompt before run()")
        if self.steps_done + steps > self.max_seq:
            raise qmm.QmmError(1, f"{self.steps_done} + {steps} steps exceed max_seq {self.max_seq}")
        use_graph = use_graph and trace is None
        if use_graph and self._graph is None:
            self.capture()
        self.steps_done += steps
        for i in range(steps):
            if use_graph:
                self._graph.replay()
            else:
                self.step(trace)
            if history is not None:
                history[i].copy_(self.logits)

    def generated(self, total: int) -> List[int]:
        return self.tokens[:total].cpu().tolist()
