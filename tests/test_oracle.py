"""Pins the CPU oracle before anything is compared against it.

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong nibble/bit index, a sign, a tie rule) fails it:
  * the reference's own known-answer tests (crates/llm/mlx-llm/src/gguf/dequant.rs:751-913);
  * an independent vectorised numpy decoder written from the byte maps of
    dequant.rs:284-290, 379-416, 452-474 (a second implementation, not a retyping);
  * closed forms: the integer block-dot decomposition equals the f64 brute-force
    dot of the dequantized operands; hand-computed quantizer outputs;
  * numpy's float16 conversion for the f16 codec;
  * the reference's tolerance tests for the quantized matmul (quant.rs:52-80,
    candle-gen/src/quant/mod.rs:1141-1172, candle-gen/tests/cuda_quant_smoke.rs:24-35).
"""
import numpy as np
import pytest

from oracle import oracle as orc

Q8_0, Q4K, Q6K, Q8K = orc.Q8_0, orc.Q4K, orc.Q6K, orc.Q8K


# ---------------------------------------------------------------------------
# independent numpy decoders (spec restatement, vectorised over blocks)
# ---------------------------------------------------------------------------

def f16(b: np.ndarray) -> np.ndarray:
    return b.copy().view(np.float16).astype(np.float32)


def np_dequant_q8_0(raw: np.ndarray) -> np.ndarray:
    blk = raw.reshape(-1, 34)
    d = f16(blk[:, 0:2].copy()).reshape(-1, 1)
    q = blk[:, 2:34].view(np.int8).astype(np.float32)
    return (q * d).reshape(-1)


def np_scale_min_k4(scales: np.ndarray):
    """scales: [nb, 12] uint8 -> (sc[nb, 8], m[nb, 8]) per get_scale_min_k4."""
    s = scales.astype(np.int32)
    sc = np.zeros((s.shape[0], 8), np.int32)
    m = np.zeros((s.shape[0], 8), np.int32)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def np_q4k_ints(raw: np.ndarray):
    blk = raw.reshape(-1, 144)
    d = f16(blk[:, 0:2].copy()).reshape(-1)
    dmin = f16(blk[:, 2:4].copy()).reshape(-1)
    sc, m = np_scale_min_k4(blk[:, 4:16])
    qs = blk[:, 16:144].reshape(-1, 4, 32).astype(np.int32)
    q = np.concatenate([qs & 0xF, qs >> 4], axis=2).reshape(-1, 256)  # chunk c: low 32 then high 32
    return d, dmin, sc, m, q


def np_dequant_q4k(raw: np.ndarray) -> np.ndarray:
    d, dmin, sc, m, q = np_q4k_ints(raw)
    sub = np.repeat(np.arange(8), 32)
    d1 = (d[:, None] * sc.astype(np.float32))[:, sub]
    m1 = (dmin[:, None] * m.astype(np.float32))[:, sub]
    return (d1 * q.astype(np.float32) - m1).reshape(-1)


def np_q6k_ints(raw: np.ndarray):
    blk = raw.reshape(-1, 210)
    ql = blk[:, 0:128].astype(np.int32)
    qh = blk[:, 128:192].astype(np.int32)
    sc = blk[:, 192:208].view(np.int8).astype(np.int32)
    d = f16(blk[:, 208:210].copy()).reshape(-1)
    q = np.zeros((blk.shape[0], 256), np.int32)
    for h in range(2):
        qlp = ql[:, 64 * h:64 * h + 64]
        qhp = qh[:, 32 * h:32 * h + 32]
        base = 128 * h
        q[:, base:base + 32] = ((qlp[:, :32] & 0xF) | ((qhp & 3) << 4)) - 32
        q[:, base + 32:base + 64] = ((qlp[:, 32:] & 0xF) | (((qhp >> 2) & 3) << 4)) - 32
        q[:, base + 64:base + 96] = ((qlp[:, :32] >> 4) | (((qhp >> 4) & 3) << 4)) - 32
        q[:, base + 96:base + 128] = ((qlp[:, 32:] >> 4) | (((qhp >> 6) & 3) << 4)) - 32
    return d, sc, q


def np_dequant_q6k(raw: np.ndarray) -> np.ndarray:
    d, sc, q = np_q6k_ints(raw)
    sub = np.repeat(np.arange(16), 16)
    s = (d[:, None] * sc.astype(np.float32))[:, sub]
    return (s * q.astype(np.float32)).reshape(-1)


def np_q8k(raw: np.ndarray):
    blk = raw.reshape(-1, 292)
    d = blk[:, 0:4].copy().view(np.float32).reshape(-1)
    q = blk[:, 4:260].view(np.int8).astype(np.int32)
    bs = blk[:, 260:292].copy().view(np.int16).astype(np.int32)
    return d, q, bs


# ---------------------------------------------------------------------------
# reference known-answer tests (dequant.rs:751-913)
# ---------------------------------------------------------------------------

def test_block_geometry_matches_reference_kat():
    # dequant.rs:752-773
    assert (orc.lib().orc_block_elems(Q8_0), orc.lib().orc_block_bytes(Q8_0)) == (32, 34)
    assert (orc.lib().orc_block_elems(Q4K), orc.lib().orc_block_bytes(Q4K)) == (256, 144)
    assert (orc.lib().orc_block_elems(Q6K), orc.lib().orc_block_bytes(Q6K)) == (256, 210)
    # quantized.cu:428-433 block_q8_K = f32 + 256 + 16*i16
    assert (orc.lib().orc_block_elems(Q8K), orc.lib().orc_block_bytes(Q8K)) == (256, 292)
    assert orc.lib().orc_block_bytes(9) == 0  # unknown/unsupported tag


def test_partial_blocks_are_refused_before_the_c_routines():
    """The C routines convert every element they are handed, so a row of a partial block would run
    past the buffer sized from whole blocks; the wrappers refuse it first."""
    x = np.zeros((3, 4160), np.float32)  # 130 Q8_0 blocks, 16.25 k-quant blocks
    assert orc.quantize(Q8_0, x).shape == (3, 130 * 34)
    for dt in (Q4K, Q6K, Q8K):
        with pytest.raises(ValueError, match="whole number"):
            orc.quantize(dt, x)
        with pytest.raises(ValueError, match="whole number"):
            orc.row_bytes(dt, 4160)
    with pytest.raises(ValueError, match="whole number"):
        orc.row_bytes(Q8_0, 48)


def test_q8_0_block_dequant_kat():
    # dequant.rs:834-848: d = 0.5, quants -16..15 -> q * 0.5
    b = np.zeros(34, np.uint8)
    b[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    b[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    out = orc.dequantize(Q8_0, b, 32)
    np.testing.assert_array_equal(out, (np.arange(32) - 16) * 0.5)


def test_q6_k_centered_is_zero_kat():
    # dequant.rs:889-913: ql nibbles 0, qh 2-bit groups = 2 -> every q == 32 -> 0
    b = np.zeros(210, np.uint8)
    b[128:192] = 0xAA
    b[192:208] = 5
    b[208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    out = orc.dequantize(Q6K, b, 256)
    assert np.all(out == 0.0)


# ---------------------------------------------------------------------------
# f16 codec vs numpy
# ---------------------------------------------------------------------------

def test_f16_codec_matches_numpy():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 4000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32),
    ]).astype(np.float32)
    L = orc.lib()
    got = np.array([L.orc_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)
    bits = np.arange(0, 65536, 7, dtype=np.uint16)
    bits = bits[(bits & 0x7C00) != 0x7C00]  # finite halves
    back = np.array([L.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    np.testing.assert_array_equal(back, bits.view(np.float16).astype(np.float32))


# ---------------------------------------------------------------------------
# independent decoder agreement on random bytes
# ---------------------------------------------------------------------------

def _random_blocks(dt, nblocks, seed):
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(nblocks, orc.block_bytes(dt)), dtype=np.uint8)
    # keep the f16 scales finite and modest
    if dt == Q8_0:
        raw[:, 0:2] = np.frombuffer(rng.uniform(-2, 2, nblocks).astype(np.float16).tobytes(), np.uint8).reshape(-1, 2)
    elif dt == Q4K:
        raw[:, 0:2] = np.frombuffer(rng.uniform(0, 0.1, nblocks).astype(np.float16).tobytes(), np.uint8).reshape(-1, 2)
        raw[:, 2:4] = np.frombuffer(rng.uniform(0, 0.1, nblocks).astype(np.float16).tobytes(), np.uint8).reshape(-1, 2)
    elif dt == Q6K:
        raw[:, 208:210] = np.frombuffer(rng.uniform(-0.01, 0.01, nblocks).astype(np.float16).tobytes(), np.uint8).reshape(-1, 2)
    return raw


@pytest.mark.parametrize("dt,dec", [(Q8_0, np_dequant_q8_0), (Q4K, np_dequant_q4k), (Q6K, np_dequant_q6k)])
def test_dequant_matches_independent_decoder(dt, dec):
    raw = _random_blocks(dt, 64, seed=dt)
    n = 64 * orc.block_elems(dt)
    np.testing.assert_array_equal(orc.dequantize(dt, raw, n), dec(raw))


def test_q4k_scale_min_unpack_high_bits():
    # sub-blocks 4..7 take their top two bits from bytes 0..3 (scales) / 4..7 (mins)
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    b[4:16] = [0xC1, 0x02, 0x03, 0x04, 0x85, 0x06, 0x07, 0x08, 0x29, 0x3A, 0x4B, 0x5C]
    b[16:] = 0x11  # every nibble = 1
    out = orc.dequantize(Q4K, b, 256)
    # j=0: sc = 0xC1&63 = 1, m = 0x85&63 = 5 -> 1*1 - 5 = -4
    assert np.all(out[0:32] == -4.0)
    # j=4: sc = (0x29&0xF) | ((0xC1>>6)<<4) = 9 | 48 = 57 ; m = (0x29>>4) | ((0x85>>6)<<4) = 2 | 32 = 34
    assert np.all(out[128:160] == 57.0 - 34.0)
    # j=5 (high nibbles of chunk 2): sc = 0xA | ((0x02>>6)<<4) = 10 ; m = 3 | 0 = 3
    assert np.all(out[160:192] == 10.0 - 3.0)


# ---------------------------------------------------------------------------
# closed form: integer block dots == f64 brute force of dequantized operands
# ---------------------------------------------------------------------------

def _rand_x(k, seed):
    return np.random.default_rng(seed).standard_normal(k).astype(np.float32)


@pytest.mark.parametrize("dt", [Q8_0, Q4K, Q6K])
def test_block_dots_equal_bruteforce(dt):
    k = 1024
    rng = np.random.default_rng(10 + dt)
    w_raw = _random_blocks(dt, 4 * k // orc.block_elems(dt), seed=20 + dt).reshape(4, -1)
    vt = orc.VEC_DOT_TYPE[dt]
    xq = orc.quantize(vt, rng.standard_normal((1, k)).astype(np.float32))
    dots = orc.block_dots(dt, w_raw, xq, k)
    x_deq = orc.dequantize(vt, xq, k).astype(np.float64)
    for n in range(4):
        w_deq = orc.dequantize(dt, w_raw[n], k).astype(np.float64)
        be = orc.block_elems(dt)
        for b in range(k // be):
            brute = float(np.dot(w_deq[b * be:(b + 1) * be], x_deq[b * be:(b + 1) * be]))
            if dt == Q8_0:
                blk = w_raw[n].reshape(-1, 34)[b]
                xb = xq.reshape(-1, 34)[b]
                dw = float(f16(blk[0:2].copy())[0])
                dx = float(f16(xb[0:2].copy())[0])
                closed = dw * dx * float(dots[0, n, b])
            elif dt == Q4K:
                blk = w_raw[n].reshape(-1, 144)[b]
                dw = float(f16(blk[0:2].copy())[0]); dmin = float(f16(blk[2:4].copy())[0])
                dx = float(xq.reshape(-1, 292)[b, 0:4].copy().view(np.float32)[0])
                closed = dw * dx * float(dots[0, n, b, 0]) - dmin * dx * float(dots[0, n, b, 1])
            else:
                blk = w_raw[n].reshape(-1, 210)[b]
                dw = float(f16(blk[208:210].copy())[0])
                dx = float(xq.reshape(-1, 292)[b, 0:4].copy().view(np.float32)[0])
                closed = dw * dx * float(dots[0, n, b])
            # the dequantized operands carry one f32 rounding each
            scale = np.sum(np.abs(w_deq[b * be:(b + 1) * be]) * np.abs(x_deq[b * be:(b + 1) * be])) + 1e-30
            assert abs(brute - closed) <= 4e-7 * scale, (n, b, brute, closed)


def test_block_dot_ranges_fit_int32():
    # worst-case magnitudes: |q8| <= 128, Q4_K sc*q <= 63*15 per element
    assert 256 * 128 * 63 * 15 < 2 ** 31
    assert 256 * 128 * 32 * 128 < 2 ** 31  # Q6_K |sc| <= 128, |q6-32| <= 32


# ---------------------------------------------------------------------------
# activation quantizers: hand-computed outputs
# ---------------------------------------------------------------------------

def test_q8k_ramp_closed_form_and_ties_away():
    x = np.arange(1, 257, dtype=np.float32)
    raw = orc.quantize(Q8K, x)
    d, q, bs = np_q8k(raw)
    # max = 256 -> iscale = -0.5, q = round(-i/2) with ties away from zero, d = -2
    assert d[0] == -2.0
    want = -np.ceil(np.arange(1, 257) / 2).astype(np.int32)
    np.testing.assert_array_equal(q[0], want)
    np.testing.assert_array_equal(bs[0], want.reshape(16, 16).sum(1))


def test_q8k_first_max_wins_and_clamp():
    x = np.zeros(256, np.float32)
    x[3] = -2.0   # first element of max |x| -> max = -2, iscale = 64
    x[7] = 2.0    # same |x|, later -> would give +128, clamped to 127
    x[9] = 0.5
    raw = orc.quantize(Q8K, x)
    d, q, _ = np_q8k(raw)
    assert d[0] == np.float32(1.0) / np.float32(64.0)
    assert q[0, 3] == -128 and q[0, 7] == 127 and q[0, 9] == 32


def test_q8k_all_zero_block():
    raw = orc.quantize(Q8K, np.zeros(256, np.float32))
    assert not raw.any()


def test_q8_0_ties_away_from_zero():
    x = np.array([127.0, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, -127.0] + [0.0] * 24, np.float32)
    raw = orc.quantize(Q8_0, x)
    assert f16(raw[0, 0:2].copy())[0] == 1.0
    q = raw[0, 2:].view(np.int8)
    np.testing.assert_array_equal(q[:8], [127, -3, -2, -1, 1, 2, 3, -127])


def test_q8_0_roundtrip_error_bound():
    x = _rand_x(32 * 256, 3)
    raw = orc.quantize(Q8_0, x)
    y = orc.dequantize(Q8_0, raw, x.size)
    d = f16(raw.reshape(-1, 34)[:, 0:2].copy()).reshape(-1)
    # |x - d16*q| <= d/2 plus the f16 rounding of d (|q| <= 127)
    err = np.abs(x - y).reshape(-1, 32).max(1)
    assert np.all(err <= d * 0.5 + 127 * np.abs(d) * 2.0 ** -11 + 1e-12)


def test_q8k_roundtrip_error_bound():
    x = _rand_x(256 * 64, 4)
    raw = orc.quantize(Q8K, x)
    y = orc.dequantize(Q8K, raw, x.size)
    d, _, _ = np_q8k(raw)
    err = np.abs(x - y).reshape(-1, 256)
    # clamp at +127 may cost one extra step for the element opposite the max
    assert np.all(err.max(1) <= np.abs(d) * 1.0 + 1e-12)
    assert np.all(np.sort(err, 1)[:, -2] <= np.abs(d) * 0.5 * (1 + 1e-6))


# ---------------------------------------------------------------------------
# weight quantizers: structure + the reference's tolerance tests
# ---------------------------------------------------------------------------

def test_q4k_constant_subblocks_give_zero_scales():
    x = np.full(256, 0.25, np.float32)
    raw = orc.quantize(Q4K, x)
    # make_qkx1_quants returns (0, 0) for max == min -> d = dmin = 0, all quants 0
    assert not raw.any()


def test_q6k_all_zero_block_reconstructs_zero():
    raw = orc.quantize(Q6K, np.zeros(256, np.float32))
    assert np.all(orc.dequantize(Q6K, raw, 256) == 0.0)


@pytest.mark.parametrize("dt,max_rel", [(Q8_0, 0.01), (Q4K, 0.12), (Q6K, 0.03)])
def test_weight_quantizer_reconstruction(dt, max_rel):
    x = (np.random.default_rng(5).standard_normal(256 * 64) * 0.02).astype(np.float32)
    y = orc.dequantize(dt, orc.quantize(dt, x), x.size)
    rel = np.sqrt(np.mean((x - y) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert rel < max_rel, rel


def test_q4k_codes_within_range():
    x = _rand_x(256 * 32, 6)
    _, _, sc, m, q = np_q4k_ints(orc.quantize(Q4K, x))
    assert sc.max() <= 63 and m.max() <= 63 and q.max() <= 15 and q.min() >= 0


# ---------------------------------------------------------------------------
# weight quantizers: the sub-block fits and the super-block packing pinned by
# what the mathematics fixes (exact grids, the extremal codes, monotone fits).
# nearest_int (round half away from zero) is the same function the Q8_0 and
# Q8_K tie tests above pin.
# ---------------------------------------------------------------------------

def _q4k_grid_block(rng):
    """A Q4_K block whose every element lies on its sub-block's grid d_j * l - m_j (l in 0..15, both ends
    present), d_j = 2^-8 sc_j, m_j = 2^-9 mn_j with 6-bit sc_j, mn_j, one sub-block at sc = 63 and one at
    mn = 63: every step of the quantizer is exact, so the block must come back bit for bit."""
    sc = rng.integers(1, 64, 8)
    mn = rng.integers(0, 64, 8)
    sc[rng.integers(8)] = 63
    mn[rng.integers(8)] = 63
    x = np.zeros(256, np.float32)
    for j in range(8):
        l = rng.integers(0, 16, 32)
        l[rng.choice(32, 2, replace=False)] = [0, 15]
        x[32 * j:32 * j + 32] = np.float32(sc[j] / 256.0) * l.astype(np.float32) - np.float32(mn[j] / 512.0)
    return x, sc, mn


def test_qkx1_fit_recovers_exact_grid():
    rng = np.random.default_rng(30)
    for _ in range(200):
        d = np.float32(rng.integers(1, 64) / 256.0)
        m = np.float32(rng.integers(0, 64) / 512.0)
        l = rng.integers(0, 16, 32)
        l[rng.choice(32, 2, replace=False)] = [0, 15]
        x = (d * l.astype(np.float32) - m).astype(np.float32)
        scale, neg_min = orc.make_qkx1_quants(x)
        assert scale == d and neg_min == m, (scale, d, neg_min, m)


def test_qkx1_min_never_above_zero_and_constant_subblock():
    """The fitted min is clamped to <= 0 (so -min >= 0 even for sub-blocks entirely above zero, where
    the least-squares min would be positive); a constant sub-block gives (0, 0)."""
    rng = np.random.default_rng(36)
    for t in range(300):
        x = (rng.standard_normal(32) * 0.1 + (np.float32(1.0) if t % 2 else 0.0)).astype(np.float32)
        scale, neg_min = orc.make_qkx1_quants(x)
        assert neg_min >= 0.0 and scale > 0.0, t
    # every element at or above 1 and the top one far out: the least-squares min of the first fit is > 0
    x = np.full(32, 1.0, np.float32)
    x[0] = 3.0
    assert orc.make_qkx1_quants(x)[1] == 0.0
    assert orc.make_qkx1_quants(np.full(32, -0.75, np.float32)) == (0.0, 0.0)


def _qkx1_err(x, scale, neg_min):
    """Squared error of the best 4-bit codes for a given (scale, min)."""
    x = x.astype(np.float64)
    l = np.clip(np.floor((x + neg_min) / scale + 0.5), 0, 15) if scale > 0 else np.zeros_like(x)
    return float(((x - (scale * l - neg_min)) ** 2).sum())


def test_qkx1_fit_never_worse_than_its_start():
    """Each pass re-rounds, then solves the least-squares scale and the (non-positive) least-squares min,
    so the fit's error can only fall from that of its first rounding at iscale = 15 / (max - min(min, 0))."""
    rng = np.random.default_rng(31)
    for t in range(400):
        x = (rng.standard_normal(32) * (0.02 if t % 2 else 1.0) + (0.03 if t % 3 == 0 else 0.0)).astype(np.float32)
        mn0 = min(float(x.min()), 0.0)
        iscale0 = 15.0 / (float(x.max()) - mn0)
        l0 = np.clip(np.floor(iscale0 * (x.astype(np.float64) - mn0) + 0.5), 0, 15)
        e0 = float(((x - (l0 / iscale0 + mn0)) ** 2).sum())
        scale, neg_min = orc.make_qkx1_quants(x)
        assert _qkx1_err(x, scale, neg_min) <= e0 * (1 + 1e-5) + 1e-12, t


def test_qx_fit_recovers_exact_grid():
    rng = np.random.default_rng(32)
    for _ in range(200):
        s = np.float32(2.0 ** -rng.integers(4, 12))
        l = rng.integers(-31, 32, 16)
        l[rng.integers(16)] = -32  # the largest magnitude: iscale = -32 / max = 1 / s
        x = (s * l.astype(np.float32)).astype(np.float32)
        scale, lq = orc.make_qx_quants(x)
        assert scale == s and np.array_equal(lq, l), (scale, s)


def test_qx_refinement_never_increases_weighted_error():
    """rmse_type 1 (weights x^2): both refinement loops accept a change only when the weighted
    least-squares objective improves, so the final codes fit no worse than the first rounding."""
    rng = np.random.default_rng(33)
    for t in range(400):
        x = (rng.standard_normal(16) * (0.02 if t % 2 else 3.0)).astype(np.float32)
        if t % 5 == 0:
            x[rng.integers(16)] *= 8.0  # an outlier
        xd = x.astype(np.float64)
        w = xd * xd
        i = int(np.argmax(np.abs(x)))
        iscale = -32.0 / float(x[i])
        l0 = np.clip(np.where(iscale * xd >= 0, np.floor(iscale * xd + 0.5), np.ceil(iscale * xd - 0.5)), -32, 31)

        def werr(l):
            sl2 = (w * l * l).sum()
            return float((w * xd * xd).sum() - ((w * xd * l).sum() ** 2) / sl2) if sl2 > 0 else float((w * xd * xd).sum())

        scale, lq = orc.make_qx_quants(x)
        assert lq.min() >= -32 and lq.max() <= 31
        assert werr(lq.astype(np.float64)) <= werr(l0) * (1 + 1e-5) + 1e-18, t
        # the second loop stops when no single-code move it proposes (l_i -> the least-squares code of
        # element i given the others) improves sum(w x l)^2 / sum(w l^2): the result is locally optimal
        lf = lq.astype(np.float64)
        sx, s2 = (w * xd * lf).sum(), (w * lf * lf).sum()
        for k in range(16):
            slx, sl2 = sx - w[k] * xd[k] * lf[k], s2 - w[k] * lf[k] * lf[k]
            if slx <= 0:
                continue
            v = xd[k] * sl2 / slx
            nl = float(np.clip(np.floor(v + 0.5) if v >= 0 else np.ceil(v - 0.5), -32, 31))
            if nl != lf[k] and sl2 + w[k] * nl * nl > 0:
                nx, n2 = slx + w[k] * xd[k] * nl, sl2 + w[k] * nl * nl
                # (the loop compares f32 sums: an improvement below their rounding may go unseen)
                assert nx * nx * s2 <= sx * sx * n2 * (1 + 2e-5), (t, k)
        # the returned scale is the weighted least-squares scale of the returned codes
        lf = lq.astype(np.float64)
        assert abs(scale - (w * xd * lf).sum() / (w * lf * lf).sum()) <= 1e-5 * abs(scale)


def test_q4k_grid_block_roundtrips_exactly():
    rng = np.random.default_rng(34)
    for _ in range(50):
        x, sc, mn = _q4k_grid_block(rng)
        raw = orc.quantize(Q4K, x)
        d, dmin, scq, mq, _ = np_q4k_ints(raw)
        assert d[0] == 2.0 ** -8 and dmin[0] == 2.0 ** -9
        assert np.array_equal(scq[0], sc) and np.array_equal(mq[0], mn)
        np.testing.assert_array_equal(orc.dequantize(Q4K, raw, 256), x)


def test_k_quant_extremal_codes():
    """The super-block scale maps the largest sub-block scale (and min) to the top code: 63 for Q4_K's
    6-bit scales and mins, -128 for Q6_K's signed 8-bit scales (iscale = -128 / the signed largest)."""
    rng = np.random.default_rng(35)
    x = (rng.standard_normal(256 * 200) * np.repeat(rng.uniform(0.01, 3.0, 200), 256)).astype(np.float32)
    _, _, sc, m, _ = np_q4k_ints(orc.quantize(Q4K, x))
    assert np.all(sc.max(1) == 63)
    assert np.all(m.max(1) == 63)
    q6 = orc.quantize(Q6K, x).reshape(-1, 210)
    s6 = q6[:, 192:208].view(np.int8).astype(np.int32)
    big = np.take_along_axis(s6, np.abs(s6).argmax(1)[:, None], 1)[:, 0]
    assert np.all(big == -128)


def _cos(a, b):
    a = a.astype(np.float64).ravel(); b = b.astype(np.float64).ravel()
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-12))


def test_reference_q8_matmul_approximates_linear():
    # crates/llm/candle-llm/src/primitives/quant.rs:52-80
    out, inn = 4, 256
    i = np.arange(out * inn)
    w = (((i * 7) % 13).astype(np.float32) / np.float32(13.0) - np.float32(0.5)).reshape(out, inn)
    x = (np.arange(inn, dtype=np.float32) / np.float32(inn) - np.float32(0.5)).reshape(1, inn)
    dense = x @ w.T
    quant = orc.matmul(Q8_0, x, orc.quantize(Q8_0, w), inn)
    assert np.all(np.abs(dense - quant) < 0.05)


def test_reference_q4k_matmul_cosine():
    # crates/media/candle-gen/candle-gen/src/quant/mod.rs:1141-1172 (Q4_K 64x256, x 4x256, cos > 0.99)
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((64, 256)) * 0.1).astype(np.float32)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    y = orc.matmul(Q4K, x, orc.quantize(Q4K, w), 256)
    assert _cos(y, x @ w.T) > 0.99


def pseudo_random(n):
    """cuda_quant_smoke.rs:24-35 splitmix-style hash of the index, mapped to [-1, 1)."""
    z = np.arange(n, dtype=np.uint64) + np.uint64(0x9E3779B97F4A7C15)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    z ^= z >> np.uint64(31)
    return ((z >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)) * np.float32(2.0) - np.float32(1.0)


@pytest.mark.parametrize("dt,min_cos", [(Q8_0, 0.999), (Q4K, 0.99), (Q6K, 0.999)])
def test_reference_smoke_shapes_cosine(dt, min_cos):
    # cuda_quant_smoke.rs:88-128 shapes (n, k, m) = (512, 1024, 8); CPU side vs dense
    n, k, m = 512, 1024, 8
    w = pseudo_random(n * k).reshape(n, k)
    x = pseudo_random(m * k).reshape(m, k)
    y = orc.matmul(dt, x, orc.quantize(dt, w), k)
    assert _cos(y, x @ w.T) > min_cos


@pytest.mark.parametrize("dt", [Q8_0, Q4K, Q6K])
def test_matmul_equals_sum_of_block_terms(dt):
    k, n, m = 512, 8, 3
    rng = np.random.default_rng(30 + dt)
    w = orc.quantize(dt, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = orc.matmul(dt, x, w, k)
    vt = orc.VEC_DOT_TYPE[dt]
    xq = orc.quantize(vt, x)
    dots = orc.block_dots(dt, w, xq, k).astype(np.float64)
    if dt == Q8_0:
        dw = f16(w.reshape(n, -1, 34)[:, :, 0:2].copy()).reshape(n, -1).astype(np.float64)
        dx = f16(xq.reshape(m, -1, 34)[:, :, 0:2].copy()).reshape(m, -1).astype(np.float64)
        ref = np.einsum("nb,mb,mnb->mn", dw, dx, dots)
    elif dt == Q4K:
        wb = w.reshape(n, -1, 144)
        dw = f16(wb[:, :, 0:2].copy()).reshape(n, -1).astype(np.float64)
        dm = f16(wb[:, :, 2:4].copy()).reshape(n, -1).astype(np.float64)
        dx = xq.reshape(m, -1, 292)[:, :, 0:4].copy().view(np.float32).reshape(m, -1).astype(np.float64)
        ref = np.einsum("nb,mb,mnb->mn", dw, dx, dots[..., 0]) - np.einsum("nb,mb,mnb->mn", dm, dx, dots[..., 1])
    else:
        dw = f16(w.reshape(n, -1, 210)[:, :, 208:210].copy()).reshape(n, -1).astype(np.float64)
        dx = xq.reshape(m, -1, 292)[:, :, 0:4].copy().view(np.float32).reshape(m, -1).astype(np.float64)
        ref = np.einsum("nb,mb,mnb->mn", dw, dx, dots)
    rms = np.sqrt(np.mean(ref ** 2))
    assert np.max(np.abs(y - ref)) / rms < 1e-5


@pytest.mark.skipif(not orc.simd_supported(), reason="needs an AVX2 + FMA host")
@pytest.mark.parametrize("dt,k", [(orc.Q8_0, 4096), (orc.Q4K, 4096), (orc.Q4K, 14336), (orc.Q6K, 14336)])
def test_avx2_vec_dot_equals_generic(dt, k):
    """The AVX2 + FMA bodies (candle's x86 SIMD vec_dot) against the generic ones: the integer block dots
    are the same, so the f32 results agree to summation-order rounding; extreme codes (all-max weights
    against -128/+127 activations) included, where a saturating pair sum would show."""
    rng = np.random.default_rng(k + dt)
    n = 64
    w = orc.quantize(dt, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((3, k)).astype(np.float32)
    x[1] = np.where(np.arange(k) % 2 == 0, -1.0, 0.9921875).astype(np.float32)  # codes -128 / +127 (Q8_K)
    ext = np.ones((n, k), np.float32) * np.where(np.arange(k) % 3 == 0, -1.0, 1.0).astype(np.float32)
    we = orc.quantize(dt, ext * 0.05)
    for wq in (w, we):
        a = orc.matmul(dt, x, wq, k, impl=orc.GENERIC)
        b = orc.matmul(dt, x, wq, k, impl=orc.AVX2)
        scale = np.abs(a.astype(np.float64)).max() + 1e-30
        assert np.abs(a - b).max() <= 1e-5 * scale * np.sqrt(k / 256), (dt, k, np.abs(a - b).max(), scale)
