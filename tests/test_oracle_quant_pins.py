"""Pins the oracle's weight quantizers where the exact-grid and monotonicity checks of test_oracle.py
leave them open: the rounding rule at every place the quantizers round, the fit's convergence, and the
arguments the super-block quantizers pass to their sub-block fits.

The quantizers are candle's `BlockQ4K::from_float` / `BlockQ6K::from_float` / `BlockQ8_0::from_float`
(candle-core k_quants.rs at rev 1e6aa85e, called at crates/llm/candle-llm/src/primitives/quant.rs:27), whose
`nearest_int` is `f32::round`: half away from zero.

* Ties: tests/quant_ties.py builds blocks from exact binary grids with one value per rounding step placed
  exactly on k + 0.5, and writes down the codes that half-away-from-zero gives; rounding half to even
  (`rintf`) gives a different code at each of them.
* Convergence: make_qkx1_quants iterates round -> least-squares refit up to five times and stops when no
  code changes, so the codes at the (scale, min) it returns nearly always survive one more pass of that
  loop. A fit cut short leaves measurably more sub-blocks whose codes still move.
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


def test_tie_rows_hold_their_blocks():
    """The GPU quantizer test's tie rows are the blocks checked above, tiled."""
    rows = qt.weight_tie_rows(1024)
    b4, b6 = qt.q4k_block()[0], qt.q6k_block()[0]
    assert rows.shape == (4, 1024)
    np.testing.assert_array_equal(rows[0, 256:512], b4)
    np.testing.assert_array_equal(rows[1, 512:768], b6)
    np.testing.assert_array_equal(rows[2, 256:512], b6)
    np.testing.assert_array_equal(rows[3], qt.q8_0_tie_row(1024))


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
