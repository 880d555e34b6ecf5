"""Checkers shared by the decode tests (not collected: no test_ prefix).

* OpChecker: DecodeSession.step trace callback; each launch of a token step
  against the CPU oracle's operation applied to the device's own inputs to
  that launch (optionally only at chosen layers).
* PrefillChecker: the same for DecodeSession.prefill's batched launches.
* q8k_flips: where two f32 activation rows quantize to different Q8_K codes,
  and how close each differing element sat to a rounding tie.

Bars: matmuls (with the fused RMSNorm prologue or the accumulate epilogue)
max|d| <= 1e-3 * rms; embedding, RoPE + KV append and argmax exact;
attention 1e-4 * rms; SiLU*mul -> Q8_K within one quantum.
"""
import ctypes

import numpy as np
import torch

from oracle import llama as ol
from oracle import oracle as orc

MM_TOL = 1e-3
# A normalised activation computed in another f32 order than numpy's differs by a few ulps; in Q8_K
# units (|iscale * x| <= 128) that is below 1e-4, so an element within TIE_EPS of a half-integer may
# round either way on the device.
TIE_EPS = 1e-4


def rel_err(got, want):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    return float(np.abs(got - want).max() / np.sqrt((want ** 2).mean()))


def cosine(a, b):
    a, b = np.asarray(a, np.float64).reshape(-1), np.asarray(b, np.float64).reshape(-1)
    return float(a @ b / np.sqrt((a @ a) * (b @ b)))


def snap(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy().copy()


def device_rms_norm(x, w, eps):
    """The library's row RMSNorm (qmm_rms_norm) on device rows: the kernel the staged matmul path
    (m > 2) runs before quantizing, so its output is the exact f32 activation that path quantizes."""
    from inference_amd import qmm
    x = x.contiguous()
    out = torch.empty_like(x)
    m, k = (1, x.numel()) if x.dim() == 1 else x.shape
    qmm._check(qmm.lib().qmm_rms_norm(x.data_ptr(), m, k, k, w.data_ptr(), ctypes.c_float(eps), out.data_ptr(), k,
                                      qmm._stream(x.device)))
    return snap(out)


def norm_matmul_err(dt, y_dev, xn, wbytes, k):
    """max|y_dev - y| / rms(y) for y = the oracle's matmul of the normalised activation xn (one row), with
    the contribution of every near-tie element removed from the deviation: where |iscale * xn| lies within
    TIE_EPS of a half-integer the device's own normalisation may round the other way, which moves each
    output by exactly d_x * W[n, i] (the dequantized weight column). Returns (plain error, error net of
    near-tie elements, number of near-tie elements)."""
    xn = np.asarray(xn, np.float32).reshape(1, k)
    y = orc.matmul(dt, xn, wbytes, k)[0]
    dev = np.abs(np.asarray(y_dev, np.float64).reshape(-1) - y)
    rms = float(np.sqrt((y.astype(np.float64) ** 2).mean()))
    plain = float(dev.max() / rms)
    if plain <= MM_TOL:
        return plain, plain, 0
    _, v, _ = q8k_scaled(xn)
    av = np.abs(v.reshape(-1).astype(np.float64))
    near = np.nonzero(np.abs(av - np.floor(av) - 0.5) < TIE_EPS)[0]
    xq = orc.quantize(orc.Q8K, xn).reshape(-1, 292)
    dx = np.abs(xq[:, :4].copy().view(np.float32).reshape(-1).astype(np.float64))
    n = y.shape[0]
    bb = orc.block_bytes(dt)
    wb = np.ascontiguousarray(wbytes, np.uint8).reshape(n, k // 256, bb)
    slack = np.zeros(n)
    for i in near:
        col = orc.dequantize(dt, np.ascontiguousarray(wb[:, i // 256]), n * 256).reshape(n, 256)[:, i % 256]
        slack += dx[i // 256] * np.abs(col.astype(np.float64))
    net = float(np.maximum(dev - 1.0001 * slack, 0.0).max() / rms)
    return plain, net, len(near)


class OpChecker:
    """DecodeSession.step trace callback: checks each launch against the oracle on the device's inputs.

    With `layers`, only those layers' launches are checked (the embedding, head and argmax always)."""

    def __init__(self, sess, ex, layers=None):
        self.s, self.ex, self.cfg = sess, ex, sess.cfg
        c = sess.cfg
        self.inv = ol.llama3_inv_freq(c.head_dim, c.rope_theta, c.rope_factor, c.rope_low, c.rope_high,
                                      c.rope_orig_ctx)
        self.layers = None if layers is None else set(layers)
        self.worst = {}
        self.steps = 0
        self.checked = []
        self.ties = []  # (position, layer, op, near-tie elements, plain error, error net of them)

    def note(self, op, err, tol):
        self.worst[op] = max(self.worst.get(op, 0.0), err)
        assert err <= tol, (op, self.p, err)

    def mm(self, name, li, x, k):
        w = self.ex["head"] if name == "head" else self.ex["layers"][li][name]
        return orc.matmul(int(self.cfg.dtypes[name]), np.asarray(x, np.float32).reshape(1, k), w, k)[0]

    def norm_mm(self, name, li, y_dev, xn, k):
        """A matmul whose launch normalises its own input (the fused RMSNorm -> Q8_K prologue)."""
        w = self.ex["head"] if name == "head" else self.ex["layers"][li][name]
        plain, net, near = norm_matmul_err(int(self.cfg.dtypes[name]), y_dev, xn, w, k)
        if near:
            self.ties.append((self.p, li, name, near, plain, net))
        self.note(name, net, MM_TOL)

    def __call__(self, op, li):
        s, c, ex = self.s, self.cfg, self.ex
        hd = c.head_dim
        if op == "embed":
            self.p = int(s.pos.item())
            x = snap(s.x)
            np.testing.assert_array_equal(x, ex["embed"][int(s.tokens[self.p].item())])
            return
        if op == "head":
            self.x = snap(s.x)
            self.lg = snap(s.logits)
            self.norm_mm("head", 0, self.lg, ol.rms_norm(self.x, ex["final_norm"], c.eps), c.hidden)
            return
        if op == "argmax":
            assert int(s.pos.item()) == self.p + 1
            if self.p + 1 >= s.prompt_len:
                assert int(s.tokens[self.p + 1].item()) == ol.argmax_first(self.lg)
            self.steps += 1
            return
        if self.layers is not None and li not in self.layers:
            return
        if op == "qkv":
            self.checked.append((self.p, li))
            self.x = snap(s.x)  # the layer input: q/k/v do not write the residual
            self.n = ol.rms_norm(self.x, ex["attn_norm"][li], c.eps)
            self.q0, self.k0, self.v0 = snap(s.q), snap(s.k), snap(s.v)
            self.norm_mm("q", li, self.q0, self.n, c.hidden)
            self.norm_mm("k", li, self.k0, self.n, c.hidden)
            self.norm_mm("v", li, self.v0, self.n, c.hidden)
        elif op == "attention":
            cs, sn = ol.cos_sin(self.inv, self.p)
            q1 = ol.apply_rope(self.q0.reshape(-1, hd), cs, sn)
            k1 = ol.apply_rope(self.k0.reshape(-1, hd), cs, sn)
            kc, vc, att = snap(s.kcache[li]), snap(s.vcache[li]), snap(s.attn)
            # rotated k and v appended at p (same f32 operations as the oracle: bit-equal)
            np.testing.assert_array_equal(kc[:, self.p], k1)
            np.testing.assert_array_equal(vc[:, self.p], self.v0.reshape(-1, hd))
            # q and k buffers keep the unrotated projections
            np.testing.assert_array_equal(snap(s.q), self.q0)
            g = c.heads // c.kv_heads
            want = np.stack([ol.attend_one(q1[h], kc[h // g, : self.p + 1], vc[h // g, : self.p + 1], s.scale)
                             for h in range(c.heads)])
            self.note("attention", rel_err(att, want), 1e-4)
            self.att = att
        elif op == "o":
            x1 = snap(s.x)
            self.note("o", rel_err(x1 - self.x, self.mm("o", li, self.att, c.heads * hd)), MM_TOL)
            self.x = x1
        elif op == "gate_up":
            n2 = ol.rms_norm(self.x, ex["ffn_norm"][li], c.eps)
            self.g, self.u = snap(s.g), snap(s.u)
            self.norm_mm("gate", li, self.g, n2, c.hidden)
            self.norm_mm("up", li, self.u, n2, c.hidden)
        elif op == "silu_mul":
            self.hq = snap(s.hq)
            h = (ol.silu(self.g) * self.u).astype(np.float32)
            want = orc.quantize(orc.Q8K, h[None]).reshape(-1)
            dg = orc.dequantize(orc.Q8K, self.hq, c.ffn).reshape(-1, 256)
            dw = orc.dequantize(orc.Q8K, want, c.ffn).reshape(-1, 256)
            quantum = np.abs(h).reshape(-1, 256).max(axis=1, keepdims=True) / 127.0
            self.note("silu_mul_quanta", float((np.abs(dg - dw) / (quantum + 1e-30)).max()), 1.01)
        elif op == "down":
            x2 = snap(s.x)
            want = orc.matmul_prequant(int(c.dtypes["down"]), self.hq[None], ex["layers"][li]["down"], c.ffn)[0]
            self.note("down", rel_err(x2 - self.x, want), MM_TOL)
            self.x = x2
        elif op == "silu_down":
            # the activation is quantized inside the launch: the oracle quantizes silu(g) * u itself
            x2 = snap(s.x)
            h = (ol.silu(self.g) * self.u).astype(np.float32)
            hq = orc.quantize(orc.Q8K, h[None])
            want = orc.matmul_prequant(int(c.dtypes["down"]), hq, ex["layers"][li]["down"], c.ffn)[0]
            self.note("down", rel_err(x2 - self.x, want), MM_TOL)
            self.x = x2


class PrefillChecker:
    """DecodeSession.prefill trace callback: every batched launch at the chosen layers against the oracle
    applied to the device's row buffers (all rows of the pass)."""

    def __init__(self, sess, ex, layers):
        self.s, self.ex, self.cfg = sess, ex, sess.cfg
        c = sess.cfg
        self.inv = ol.llama3_inv_freq(c.head_dim, c.rope_theta, c.rope_factor, c.rope_low, c.rope_high,
                                      c.rope_orig_ctx)
        self.layers = set(layers)
        self.worst = {}
        self.rows = None

    def note(self, op, err, tol):
        self.worst[op] = max(self.worst.get(op, 0.0), err)
        assert err <= tol, (op, self.li, err)

    def mm(self, name, li, x, k):
        return orc.matmul(int(self.cfg.dtypes[name]), np.asarray(x, np.float32).reshape(-1, k),
                          self.ex["layers"][li][name], k)

    def norm(self, xd, wd, wh):
        """The rows the batched matmul quantizes: the library's RMSNorm of the device rows (its staged path
        runs that kernel first), checked against the oracle's rms_norm to f32 rounding."""
        xn = device_rms_norm(xd, wd, self.cfg.eps)
        self.note("rms_norm", rel_err(xn, ol.rms_norm(snap(xd), wh, self.cfg.eps)), 1e-5)
        return xn

    def __call__(self, op, li, b):
        s, c, ex = self.s, self.cfg, self.ex
        hd = c.head_dim
        if op == "embed":
            x = snap(b["x"])
            self.rows = x.shape[0]
            toks = snap(s.tokens)[: self.rows]
            np.testing.assert_array_equal(x, ex["embed"][toks])
            return
        if li not in self.layers:
            return
        self.li = li
        R = self.rows
        if op == "qkv":
            self.x = snap(b["x"])
            n = self.norm(b["x"], s.w.attn_norm[li], ex["attn_norm"][li])
            self.q0, self.k0, self.v0 = snap(b["q"]), snap(b["k"]), snap(b["v"])
            for name, got in (("q", self.q0), ("k", self.k0), ("v", self.v0)):
                self.note(name, rel_err(got, self.mm(name, li, n, c.hidden)), MM_TOL)
        elif op == "rope_kv":
            # q and k rows rotated in place (the same f32 operations as the oracle: bit-equal), k and v
            # appended to the caches at the rows' positions
            kc, vc = snap(s.kcache[li]), snap(s.vcache[li])
            q1, k1 = snap(b["q"]), snap(b["k"])
            for r in range(R):
                cs, sn = ol.cos_sin(self.inv, r)
                kr = ol.apply_rope(self.k0[r].reshape(-1, hd), cs, sn)
                np.testing.assert_array_equal(q1[r].reshape(-1, hd), ol.apply_rope(self.q0[r].reshape(-1, hd), cs, sn))
                np.testing.assert_array_equal(k1[r].reshape(-1, hd), kr)
                np.testing.assert_array_equal(kc[:, r], kr)
                np.testing.assert_array_equal(vc[:, r], self.v0[r].reshape(-1, hd))
            self.kc, self.vc, self.q1 = kc, vc, q1
        elif op == "attention":
            att = snap(b["att"])
            g = c.heads // c.kv_heads
            want = np.empty_like(att)
            for r in range(R):
                q1 = self.q1[r].reshape(-1, hd)
                want[r] = np.concatenate([ol.attend_one(q1[h], self.kc[h // g, : r + 1], self.vc[h // g, : r + 1],
                                                        s.scale) for h in range(c.heads)])
            self.note("attention", rel_err(att, want), 1e-4)
            self.att = att
        elif op == "o":
            x1 = snap(b["x"])
            self.note("o", rel_err(x1 - self.x, self.mm("o", li, self.att, c.heads * hd)), MM_TOL)
            self.x = x1
        elif op == "gate_up":
            n2 = self.norm(b["x"], s.w.ffn_norm[li], ex["ffn_norm"][li])
            self.g, self.u = snap(b["g"]), snap(b["u"])
            self.note("gate", rel_err(self.g, self.mm("gate", li, n2, c.hidden)), MM_TOL)
            self.note("up", rel_err(self.u, self.mm("up", li, n2, c.hidden)), MM_TOL)
        elif op == "silu_mul":
            self.h = snap(b["h"])
            self.note("silu_mul", rel_err(self.h, (ol.silu(self.g) * self.u).astype(np.float32)), 1e-5)
        elif op == "down":
            x2 = snap(b["x"])
            self.note("down", rel_err(x2 - self.x, self.mm("down", li, self.h, c.ffn)), MM_TOL)
            self.x = x2


def q8k_scaled(x):
    """Q8_K codes of f32 rows (the oracle's quantizer) and the f32 values iscale * x they round from,
    with the index of each 256-block's max-|x| element (first wins)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 256)
    codes = orc.quantize(orc.Q8K, x).reshape(-1, 292)[:, 4:260].view(np.int8).astype(np.int32)
    imax = np.abs(x).argmax(axis=1)
    mx = x[np.arange(x.shape[0]), imax]
    with np.errstate(divide="ignore", invalid="ignore"):
        iscale = np.where(mx != 0, np.float32(-128.0) / mx, np.float32(0)).astype(np.float32)
    v = (iscale[:, None] * x).astype(np.float32)
    return codes, v, imax


def q8k_flips(a, b):
    """Elements whose Q8_K codes differ between rows a and b (same length, multiple of 256).

    Returns (flips, max_moves): flips lists (element, code_a, code_b, tie_margin_a) for elements of
    blocks whose max element is the same in a and b, tie_margin = | |v| - floor(|v|) - 1/2 | of a's
    pre-rounding value (0 at an exact tie); max_moves lists the blocks whose max-|x| element differs
    (a tie between the two largest magnitudes: every code of the block may then change)."""
    ca, va, ia = q8k_scaled(a)
    cb, _, ib = q8k_scaled(b)
    flips, moves = [], []
    for blk in range(ca.shape[0]):
        if ia[blk] != ib[blk]:
            moves.append(int(blk))
            continue
        for e in np.nonzero(ca[blk] != cb[blk])[0]:
            v = abs(float(va[blk, e]))
            flips.append((int(blk * 256 + e), int(ca[blk, e]), int(cb[blk, e]), abs(v - np.floor(v) - 0.5)))
    return flips, moves


# ---- where two decode chains part: the activation quantizations of one position ----
QUANT_OPS = ("n_attn", "att", "n_ffn", "hmid")
TIE_MARGIN = 2e-3  # |frac(|iscale * x|) - 1/2| of a flipped element: f32 noise on a value below 128


def log(msg):
    print(msg, flush=True)


def kv_rel(kc_a, vc_a, kc_b, vc_b, li, p):
    """max|d| / rms between two chains' K and V rows of layer li at position p ([layer][kv][pos][dim])."""
    a = np.concatenate([kc_a[li, :, p].ravel(), vc_a[li, :, p].ravel()])
    b = np.concatenate([kc_b[li, :, p].ravel(), vc_b[li, :, p].ravel()])
    return rel_err(a, b)


def quant_inputs_from_record(rec, li):
    return {op: rec[li][op] for op in QUANT_OPS}


def window(li):
    """The activation quantizations that lie between layer li - 1's K/V rows (still at noise) and layer
    li's (past it), in chain order."""
    return ([(li - 1, op) for op in QUANT_OPS[1:]] if li > 0 else []) + [(li, "n_attn")]


def first_flip(dev_in, orc_in, li):
    """Walk window(li); return the first quantization whose Q8_K codes differ, as (layer, op, input
    rel error, flips, max moves), or None."""
    for l, op in window(li):
        a, b = orc_in[l][op], dev_in[l][op]
        flips, moves = q8k_flips(a, b)
        if flips or moves:
            return l, op, rel_err(b, a), flips, moves
    return None


def assert_tie(where, found):
    assert found is not None, f"{where}: chains part but no activation quantization differs"
    li, op, in_err, flips, moves = found
    log(f"{where}: first Q8_K difference at layer {li} {op}: inputs max|d|/rms {in_err:.2e}, "
        f"{len(flips)} flipped codes, {len(moves)} blocks with a moved max; "
        + ", ".join(f"elem {e}: {a}->{b} (tie margin {m:.1e})" for e, a, b, m in flips[:6]))
    assert in_err <= 1e-4, (where, li, op, in_err)
    for e, a, b, m in flips:
        assert abs(a - b) == 1, (where, li, op, e, a, b)
        assert m <= TIE_MARGIN, (where, li, op, e, m)


