"""Resident GGUF loads on the GPU: quantized blocks straight into device QTensors.

A GGUF image's Q4_K / Q6_K / Q8_0 tensor must land in a QTensor whose GGML
bytes (qmm_qtensor_to_ggml) equal the file's, bit for bit; with the q/k
un-permute, they equal the file's rows gathered by candle-llm gguf.rs:333-356's
index. A llama GGUF written from a decode model's weights (q/k in llama.cpp's
row order) must load into a model that decodes the same tokens.
"""
import numpy as np
import pytest
import torch

from inference_amd import GgmlDType, QTensor
from inference_amd.gguf import Content, GgufFile, unpermute_rows
from inference_amd.llama_decode import DecodeSession, LlamaConfig, LlamaWeights
from oracle import oracle as orc
import gguf_writer as W

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("dt,tag,odt", [(GgmlDType.Q4K, 12, orc.Q4K), (GgmlDType.Q6K, 14, orc.Q6K),
                                        (GgmlDType.Q8_0, 8, orc.Q8_0)])
@pytest.mark.parametrize("heads", [0, 4])
def test_load_qtensor_bit_exact(tmp_path, dt, tag, odt, heads):
    rng = np.random.default_rng(tag + heads)
    n, k = 256, 1024
    raw = orc.quantize(odt, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    img = W.build([("general.architecture", W.T_STRING, "llama")], [("w", (n, k), tag, raw.tobytes())],
                  alignment=64 if heads else 32)
    p = tmp_path / "w.gguf"
    p.write_bytes(img)
    c = Content.read(p)
    qt = c.tensor("w", DEV, unpermute_heads=heads)
    assert qt.dtype() == dt
    got = qt.to_ggml().reshape(n, -1)
    want = raw.reshape(n, -1)
    if heads:
        want = want[unpermute_rows(n, heads)]
    np.testing.assert_array_equal(got, want)
    # the same blocks through QTensor.from_ggml (QStorage::from_data) give the same device tensor
    ref = QTensor.from_ggml(want.reshape(-1), dt, (n, k), device=DEV)
    torch.testing.assert_close(qt.dequantize(), ref.dequantize(), rtol=0, atol=0)


def test_load_dense_types():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((3, 8)).astype(np.float32)
    h = a.astype(np.float16)
    bf = (a.view(np.uint32) >> 16).astype(np.uint16)
    q = orc.quantize(orc.Q6K, rng.standard_normal((2, 256)).astype(np.float32))
    img = W.build([], [("f32", (3, 8), 0, a.tobytes()), ("f16", (3, 8), 1, h.tobytes()),
                       ("bf16", (3, 8), 30, bf.tobytes()), ("q6k", (2, 256), 14, q.tobytes())])
    g = GgufFile.parse(img)
    t = {x.name: x for x in g.tensors}
    np.testing.assert_array_equal(g.load_dense(t["f32"], DEV).cpu().numpy(), a)
    np.testing.assert_array_equal(g.load_dense(t["f16"], DEV).cpu().numpy(), h.astype(np.float32))
    np.testing.assert_array_equal(g.load_dense(t["bf16"], DEV).cpu().numpy(),
                                  (bf.astype(np.uint32) << 16).view(np.float32))
    np.testing.assert_array_equal(g.load_dense(t["q6k"], DEV).cpu().numpy(),
                                  orc.dequantize(orc.Q6K, q, 512).reshape(2, 256))


def test_resident_loader_errors():
    from inference_amd import QmmError
    img = W.build([], [("f32", (4, 256), 0, bytes(4096)), ("q4k3d", (2, 2, 256), 12, bytes(4 * 144)),
                       ("q4k", (6, 256), 12, bytes(6 * 144))])
    g = GgufFile.parse(img)
    t = {x.name: x for x in g.tensors}
    for name, heads in (("f32", 0), ("q4k3d", 0), ("q4k", 4), ("q4k", 2)):  # dense, 3-D, 6 rows / 4 heads, hd 3
        with pytest.raises(QmmError):
            g.load_qtensor(t[name], DEV, heads)


def small_cfg():
    return LlamaConfig(layers=2, hidden=512, ffn=1024, heads=8, kv_heads=2, head_dim=64, vocab=1000)


def test_llama_gguf_decodes_like_the_in_memory_model(tmp_path):
    cfg = small_cfg()
    w = LlamaWeights.random(cfg, 21, DEV)
    ex = w.export()
    # non-trivial norms so that a swapped norm tensor would show
    rng = np.random.default_rng(2)
    for i in range(cfg.layers):
        ex["attn_norm"][i] = rng.uniform(0.5, 1.5, cfg.hidden).astype(np.float32)
        ex["ffn_norm"][i] = rng.uniform(0.5, 1.5, cfg.hidden).astype(np.float32)
        w.attn_norm[i].copy_(torch.from_numpy(ex["attn_norm"][i]))
        w.ffn_norm[i].copy_(torch.from_numpy(ex["ffn_norm"][i]))
    p = tmp_path / "llama.gguf"
    p.write_bytes(W.llama_image(cfg, ex))
    w2 = LlamaWeights.from_gguf(p, DEV)
    c2 = w2.cfg
    assert (c2.layers, c2.hidden, c2.ffn, c2.heads, c2.kv_heads, c2.head_dim, c2.vocab) == \
        (cfg.layers, cfg.hidden, cfg.ffn, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.vocab)
    assert (c2.rope_theta, c2.rope_factor, c2.rope_low, c2.rope_high, c2.rope_orig_ctx) == \
        (cfg.rope_theta, cfg.rope_factor, cfg.rope_low, cfg.rope_high, cfg.rope_orig_ctx)
    assert c2.eps == pytest.approx(cfg.eps)
    ex2 = w2.export()
    for a, b in zip(ex["layers"], ex2["layers"]):
        for name in a:
            np.testing.assert_array_equal(a[name], b[name])  # q/k back in half-split order, bit for bit
    np.testing.assert_array_equal(ex["head"], ex2["head"])
    np.testing.assert_array_equal(ex["embed"], ex2["embed"])
    prompt = [3, 141, 59, 26]
    toks = []
    for weights in (w, w2):
        s = DecodeSession(weights, 64)
        s.reset(prompt)
        s.run(20)
        toks.append(s.generated(21))
    assert toks[0] == toks[1]
