"""Pins the oracle's weight quantizers where the exact-grid and monotonicity checks of test_oracle.py
leave them open: the rounding rule at every place the quantizers round, the fit's convergence, and the
arguments the super-block quantizers pass to their sub-block fits.

The quantizers are candle's `BlockQ4K::from_float` / `BlockQ6K::from_float` / `BlockQ8_0::from_float`
(candle-core k_quants.rs at rev 1e6aa85e, called at crates/llm/candle-llm/src/primitives/quant.rs:27), whose
`nearest_int` is `f32::round`: half away from zero.

* Ties: tests/quant_ties.py builds blocks from exact binary grids with one value per rounding step placed
  exactly on k + 0.5, and writes down the codes that half-away-from-zero gives; rounding half to even
  (`rintf`) gives a different code at each of them.
* Division or reciprocal: Q4_K and Q6_K divide by the sub-block scale, Q8_0 multiplies by f32(1 / d);
  inputs one f32 step from a half, at scales whose reciprocal is inexact, round apart under the two
  readings. The Q6_K int8 sub-block scale saturates at 127 (a sub-block that is the negation of the
  largest one reaches 128).
* Convergence: make_qkx1_quants iterates round -> least-squares refit up to five times and stops when no
  code changes, so the codes at the (scale, min) it returns nearly always survive one more pass of that
  loop. A fit cut short leaves measurably more sub-blocks whose codes still move. make_qx_quants' first
  loop (checked through an oracle hook that stops after it) ends at a fixed point or after three passes,
  and its coordinate pass takes a move only when the f32 objective strictly rises.
* Call sites: a Q4_K block's d and dmin are the largest of its eight sub-block fits (make_qkx1_quants with
  nmax 15 and 5 tries) over 63; a Q6_K block's d is the signed largest of its sixteen fits
  (make_qx_quants with nmax 32 and the x^2 weights, rmse_type 1) over -128. Each check compares the
  quantizer's f16 bytes with the fit hook run at those documented arguments, so a call site that passes
  other arguments (one try, unweighted fits) fails it.
"""
import numpy as np

import quant_ties as qt
from oracle import oracle as orc
from test_oracle import f16, np_q4k_ints, np_q6k_ints

Q8_0, Q4K, Q6K = orc.Q8_0, orc.Q4K, orc.Q6K
F32 = np.float32


def _rint_half_even(v):
    return np.rint(np.asarray(v, np.float64)).astype(np.int64)


# ---------------------------------------------------------------------------
# ties
# ---------------------------------------------------------------------------

def test_q4k_scale_min_and_code_ties_round_away_from_zero():
    x, sc, mn, checks = qt.q4k_block()
    raw = orc.quantize(Q4K, x)
    d, dmin, scq, mq, q = np_q4k_ints(raw)
    assert d[0] == 2.0 ** -6 and dmin[0] == 2.0 ** -6
    # sub-block 1's scale sits at 20.5 and sub-block 2's min at 12.5: codes 21 and 13 (half to even: 20, 12)
    assert scq[0, 1] == 21 and mq[0, 2] == 13, (scq[0], mq[0])
    np.testing.assert_array_equal(scq[0], sc)
    np.testing.assert_array_equal(mq[0], mn)
    # sub-block 3: one element at (x + dm) / d = 6.5 -> 7 (half to even: 6); the others on their grid
    idx = np.array([i for i, _ in checks])
    want = np.array([c for _, c in checks])
    assert want[0] == 7 and _rint_half_even(6.5) == 6
    np.testing.assert_array_equal(q[0, idx], want)


def test_q6k_scale_and_code_ties_round_away_from_zero():
    x, scales, checks = qt.q6k_block()
    raw = orc.quantize(Q6K, x)
    d, scq, q = np_q6k_ints(raw)
    assert d[0] == -(2.0 ** -10)
    # sub-block 1: iscale * scale = -2.5 -> -3 (half to even: -2)
    assert scq[0, 1] == -3, scq[0]
    np.testing.assert_array_equal(scq[0], scales)
    # sub-block 2: x / d = 4.5 and -10.5 -> 5 and -11 (half to even: 4 and -10)
    idx = np.array([i for i, _ in checks])
    want = np.array([c for _, c in checks])
    assert list(want[:2]) == [5, -11]
    np.testing.assert_array_equal(q[0, idx], want)


def test_qkx1_first_rounding_ties_round_away_from_zero():
    """ntry = 1: one rounding at iscale = 4 (exact), then the least-squares scale and non-positive min of
    those codes. The expected values come from the hand-written codes; the same sums over the codes half
    to even would give is a different scale, so the rounding rule decides the outcome."""
    x, codes = qt.qkx1_first_rounding_case()
    scale, neg_min = orc.make_qkx1_quants(x, ntry=1)

    def fit(l):
        xd, lf = x.astype(np.float64), l.astype(np.float64)
        s = (xd * lf).sum() / (lf * lf).sum()  # min = 0 in the rounding (x >= 0)
        m = min((xd - s * lf).sum() / x.size, 0.0)
        return s, -m

    s_away, m_away = fit(codes)
    even = _rint_half_even(4.0 * x.astype(np.float64))
    s_even, _ = fit(even)
    assert abs(s_away - s_even) > 1e-3 * s_away  # the two rules part
    assert abs(scale - s_away) <= 1e-6 * s_away, (scale, s_away, s_even)
    # the min is a mean of f32 differences: its rounding is relative to the elements, not to the min
    assert abs(neg_min - m_away) <= 1e-6 * float(np.abs(x).max()), (neg_min, m_away)


def test_qx_first_rounding_ties_round_away_from_zero():
    """make_qx_quants with rmse_type 0 is the bare first rounding at iscale = -nmax / max."""
    x, codes = qt.qx_first_rounding_case()
    scale, l = orc.make_qx_quants(x, nmax=32, rmse_type=0)
    assert scale == 1.0
    np.testing.assert_array_equal(l, codes)


def test_q8_0_weight_ties_round_away_from_zero():
    x = qt.q8_0_tie_row(256)
    raw = orc.quantize(Q8_0, x).reshape(-1, 34)
    assert np.all(f16(raw[:, 0:2].copy()) == 2.0 ** -3)
    q = raw[:, 2:].view(np.int8).astype(np.int64)
    np.testing.assert_array_equal(q[:, :12], np.tile([127, -3, 3, 1, -1, 7, -7, 101, -127, 11, 2, -2], (8, 1)))


# ---------------------------------------------------------------------------
# division against multiplication by the reciprocal, and the int8 scale's clamp
# ---------------------------------------------------------------------------

def _div_codes(v, d):
    q = (np.asarray(v, F32) / F32(d)).astype(F32)
    return np.sign(q) * np.floor(np.abs(q.astype(np.float64)) + 0.5)


def _recip_codes(v, d):
    q = (np.asarray(v, F32) * (F32(1) / F32(d))).astype(F32)
    return np.sign(q) * np.floor(np.abs(q.astype(np.float64)) + 0.5)


def test_q4k_codes_divide_by_the_sub_block_scale():
    """BlockQ4K::from_float forms the codes as (x + dm) / d. Sub-blocks 4 (d = 41 * 2^-6) and 5
    (d = 11 * 2^-6) hold elements where f32 division and multiplication by f32(1 / d) round apart; their
    min code is 0, so dm = 0 and the code is x / d."""
    x, sc, mn, checks = qt.q4k_block()
    _, _, scq, mq, q = np_q4k_ints(orc.quantize(Q4K, x))
    for j, code in ((4, 41), (5, 11)):
        assert scq[0, j] == code and mq[0, j] == 0
        d = F32(2.0 ** -6) * F32(code)
        xs = x[32 * j:32 * j + 32]
        div = _div_codes(xs, d)
        parted = np.flatnonzero(div != _recip_codes(xs, d))
        assert parted.size == 3, parted  # the three moved elements
        np.testing.assert_array_equal(q[0, 32 * j:32 * j + 32], np.clip(div, 0, 15))
        want = {i: c for i, c in checks}
        np.testing.assert_array_equal(q[0, 32 * j + parted], [want[32 * j + i] for i in parted])


def test_q6k_codes_divide_by_the_sub_block_scale():
    """BlockQ6K::from_float forms the codes as x / d with d = f16(d_super) * int8 scale. Sub-block 3
    (d = 13 * 2^-10) holds four elements where division and multiplication by f32(1 / d) round apart."""
    x, scales, checks = qt.q6k_block()
    dsup, scq, q = np_q6k_ints(orc.quantize(Q6K, x))
    assert scq[0, 3] == -13
    d = F32(dsup[0]) * F32(-13)
    assert d == F32(13 * 2.0 ** -10)
    xs = x[48:64]
    div = _div_codes(xs, d)
    parted = np.flatnonzero(div != _recip_codes(xs, d))
    assert parted.size == 4, parted
    np.testing.assert_array_equal(q[0, 48:64], np.clip(div, -32, 31))
    assert sorted(div[parted].astype(int).tolist()) == [-19, -9, 16, 19]


def test_q8_0_codes_multiply_by_the_reciprocal():
    """BlockQ8_0::from_float forms the codes as round(x * id) with id = 1 / d in f32. With d = 3 * 2^-5
    (f32(1 / d) rounds up) the row's elements sit one f32 step toward zero from a half: x * id rounds to
    the half exactly (-> one further from zero) while x / d falls short of it (-> j)."""
    x = qt.q8_0_recip_row(256)
    raw = orc.quantize(Q8_0, x).reshape(-1, 34)
    d = F32(3 * 2.0 ** -5)
    assert np.all(f16(raw[:, 0:2].copy()) == d)
    ks = np.array(qt.Q8_0_RECIP_KS)
    vals = x[1:1 + ks.size]
    prod = (vals * (F32(1) / d)).astype(F32)
    np.testing.assert_array_equal(prod, np.sign(ks) * (np.abs(ks) + 0.5))  # on the half exactly
    np.testing.assert_array_equal(_div_codes(vals, d), ks)  # what a division would give
    want = np.concatenate([[127], ks + np.sign(ks)])
    q = raw[:, 2:2 + want.size].view(np.int8).astype(np.int64)
    np.testing.assert_array_equal(q, np.tile(want, (8, 1)))


def test_q6k_int8_scale_saturates_at_127():
    """A sub-block whose scale is the negative of the block's largest gets iscale * scale = 128, which
    BlockQ6K::from_float clamps to 127 (an int8 holds -128..127): scale bytes -128 and 127, sub-block 1's
    codes equal sub-block 0's, and sub-block 1 dequantizes to 127/128 of its input."""
    x, scales, l0 = qt.q6k_saturating_block()
    raw = orc.quantize(Q6K, x)
    dsup, scq, q = np_q6k_ints(raw)
    assert dsup[0] == -(2.0 ** -10)
    np.testing.assert_array_equal(scq[0], scales)
    assert scq[0, 0] == -128 and scq[0, 1] == 127
    np.testing.assert_array_equal(q[0, 0:16], l0)
    np.testing.assert_array_equal(q[0, 16:32], l0)
    y = orc.dequantize(Q6K, raw, 256)
    np.testing.assert_array_equal(y[16:32], (x[16:32].astype(np.float64) * 127 / 128).astype(F32))


def test_tie_rows_hold_their_blocks():
    """The GPU quantizer test's tie rows are the blocks checked above, tiled."""
    rows = qt.weight_tie_rows(1024)
    b4, b6 = qt.q4k_block()[0], qt.q6k_block()[0]
    assert rows.shape == (6, 1024)
    np.testing.assert_array_equal(rows[0, 256:512], b4)
    np.testing.assert_array_equal(rows[1, 512:768], b6)
    np.testing.assert_array_equal(rows[2, 256:512], b6)
    np.testing.assert_array_equal(rows[3], qt.q8_0_tie_row(1024))
    np.testing.assert_array_equal(rows[4, 768:1024], qt.q6k_saturating_block()[0])
    np.testing.assert_array_equal(rows[5], qt.q8_0_recip_row(1024))


# ---------------------------------------------------------------------------
# convergence of the Q4_K fit
# ---------------------------------------------------------------------------

def _codes(xd, scale, mn):
    return np.clip(np.floor((xd - mn) / scale + 0.5), 0, 15)


def _fixed_point_share(ntry, n=2000, seed=90):
    """Share of Gaussian sub-blocks whose codes at the returned (scale, min) survive one more pass of
    the documented loop: round at (scale, min), least-squares scale at that min, non-positive
    least-squares min at that scale, round again (f64)."""
    rng = np.random.default_rng(seed)
    fixed = 0
    for t in range(n):
        x = (rng.standard_normal(32) * (0.02 if t % 2 else 1.0)).astype(np.float32)
        scale, neg_min = orc.make_qkx1_quants(x, ntry=ntry)
        xd = x.astype(np.float64)
        l1 = _codes(xd, scale, -neg_min)
        s2 = ((xd + neg_min) * l1).sum() / (l1 * l1).sum()
        m2 = min((xd - s2 * l1).sum() / x.size, 0.0)
        fixed += np.array_equal(_codes(xd, s2, m2), l1)
    return fixed / n


def test_qkx1_fit_ends_at_a_fixed_point():
    """The five-try fit leaves 94% of Gaussian sub-blocks with codes that one more pass keeps (the rest
    hit the try cap mid-cycle); a fit cut to one try leaves 70%, to three 88%."""
    assert _fixed_point_share(5) >= 0.92
    assert _fixed_point_share(1) <= 0.8


# ---------------------------------------------------------------------------
# the two refinement loops of the Q6_K fit (make_qx_quants, rmse_type 1)
# ---------------------------------------------------------------------------

def _wobj(xd, l):
    """The weighted least-squares objective the fit raises: (sum w x l)^2 / sum w l^2 with w = x^2 (f64)."""
    w = xd * xd
    return (w * xd * l).sum() ** 2 / (w * l * l).sum()


def test_qx_first_loop_ends_at_a_fixed_point_or_after_three_passes():
    """The first loop re-rounds every element at 1 / scale and refits, and keeps going while the codes change
    and the objective rises, for at most three passes. The oracle's hook stops the fit after that loop and
    returns its accepted passes: never above three, and when under three, rounding once more at
    f32(1 / scale) changes no code or does not raise the objective (f64, 1e-5 slack for the f32 sums).
    On 4000 Gaussian sub-blocks about a fifth take a pass, a few percent two and a few take all three; a
    loop cut to one or two passes leaves 35 or 4 sub-blocks where another pass still gains."""
    rng = np.random.default_rng(91)
    X = rng.standard_normal((4000, 16)).astype(F32)
    passes = np.zeros(4, np.int64)
    gains = 0
    for x in X:
        scale, l, p = orc.make_qx_quants_first(x)
        assert 0 <= p <= 3, p
        passes[p] += 1
        if p == 3:
            continue
        again = (x * (F32(1) / F32(scale))).astype(np.float64)
        l2 = np.clip(np.sign(again) * np.floor(np.abs(again) + 0.5), -32, 31)
        if np.any(l2 != l) and _wobj(x.astype(np.float64), l2) > _wobj(x.astype(np.float64), l) * (1 + 1e-5):
            gains += 1
    assert gains == 0
    assert passes[1] > 400 and passes[2] > 40 and passes[3] > 0, passes


def test_qx_second_loop_takes_a_code_only_when_the_objective_rises():
    """The coordinate pass moves an element to round(x * sl2 / slx) only when slx^2 * suml2 > sumlx^2 * sl2,
    strictly. Sub-block: x0 = -32.25 (the largest magnitude, so iscale = -32 / -32.25), fourteen elements at
    +-31 and x15 = 0.5 + 2^-9. The first rounding gives x15 the code 0 (x15 * iscale < 1/2); the fitted scale
    of those codes is ~1.0006, at which x15 rounds to 1. But x15's weighted terms at code 1 (w x = 0.126,
    w = 0.252) are below half an ulp of the f32 sums (~1.4e7, ulp 1), so moving it leaves both sums and the
    two compared products equal: the code stays 0 (a >= comparison would take 1)."""
    x = np.array([-32.25] + [31.0, -31.0] * 7 + [0.5 + 2.0 ** -9], F32)
    grid = np.array([-32] + [31, -31] * 7 + [0])
    # the mechanism, in f32: the sums over the first fifteen elements do not move when x15's terms are added
    w = x * x
    slx = np.float32(0)
    sl2 = np.float32(0)
    for i in range(15):
        slx = F32(slx + w[i] * x[i] * F32(grid[i]))
        sl2 = F32(sl2 + w[i] * F32(grid[i] * grid[i]))
    assert 2.0 ** 23 <= slx < 2.0 ** 24 and 2.0 ** 23 <= sl2 < 2.0 ** 24
    assert F32(slx + w[15] * x[15]) == slx and F32(sl2 + w[15]) == sl2
    assert round(float(x[15]) * float(sl2) / float(slx)) == 1 and x[15] * (F32(32) / F32(32.25)) < 0.5
    # the first loop leaves the codes of the first rounding; the coordinate pass keeps x15 at 0
    _, l1, p = orc.make_qx_quants_first(x)
    np.testing.assert_array_equal(l1, grid)
    assert p == 0
    scale, l = orc.make_qx_quants(x, nmax=32, rmse_type=1)
    np.testing.assert_array_equal(l, grid)
    assert abs(scale - float(slx) / float(sl2)) <= 1e-6


# ---------------------------------------------------------------------------
# call sites of the sub-block fits
# ---------------------------------------------------------------------------

def _f16(v):
    """f32 -> f16 (round to nearest even) -> f32, numpy's conversion."""
    return np.float32(np.float16(np.float32(v)))


def _blocks(seed, n):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, 256)) * np.repeat(rng.uniform(0.005, 2.0, n), 256).reshape(n, 256)).astype(np.float32)


def test_q4k_super_scales_are_the_largest_five_try_fits():
    x = _blocks(91, 300)
    d, dmin, _, _, _ = np_q4k_ints(orc.quantize(Q4K, x))
    for b in range(x.shape[0]):
        fits = [orc.make_qkx1_quants(x[b, 32 * j:32 * j + 32], nmax=15, ntry=5) for j in range(8)]
        max_scale = max(f[0] for f in fits)
        max_min = max(f[1] for f in fits)
        assert d[b] == _f16(np.float32(max_scale) / np.float32(63.0)), b
        assert dmin[b] == _f16(np.float32(max_min) / np.float32(63.0)), b


def test_q6k_super_scale_is_the_largest_x2_weighted_fit():
    x = _blocks(92, 300)
    d, _, _ = np_q6k_ints(orc.quantize(Q6K, x))
    for b in range(x.shape[0]):
        scales = [orc.make_qx_quants(x[b, 16 * j:16 * j + 16], nmax=32, rmse_type=1)[0] for j in range(16)]
        big = max(scales, key=abs)  # the first of the largest magnitude
        iscale = np.float32(-128.0) / np.float32(big)
        want = _f16(np.float32(1.0) / iscale)
        assert d[b] == want, (b, d[b], want)
