"""Weight-quantizer inputs that put a rounding step exactly on k + 0.5, with the codes that rounding half
away from zero gives there (candle's `nearest_int` is `f32::round`). The codes are written down by hand
from the construction, not computed by the quantizer: each block is built from exact binary grids so that
every value before the tied rounding is exact, then one value is placed on the half-way point.

Shared by the CPU pinning tests (tests/test_oracle_quant_pins.py) and the GPU quantizer test
(tests/test_gpu_parity.py::test_weight_quantizer_bit_exact), so both sides see the same tied inputs.

Places where the quantizers round (the `from_float` steps of BlockQ4K / BlockQ6K, candle-core k_quants.rs
at rev 1e6aa85e, called from crates/llm/candle-llm/src/primitives/quant.rs:27):
  Q4_K  (a) the fit's first rounding iscale * (x - min)          -> `qkx1_first_rounding_case`
        (b) the 6-bit scale / min codes inv_scale * scl[j]       -> `q4k_block` sub-blocks 1, 2
        (c) the final codes (x + dm) / d                         -> `q4k_block` sub-block 3
  Q6_K  (d) the int8 sub-block scales iscale * scales[j]         -> `q6k_block` sub-block 1
        (e) the final codes x / d                                -> `q6k_block` sub-block 2
        (f) the fit's first rounding iscale * x (rmse_type 0)    -> `qx_first_rounding_case`
  Q8_0  (g) the codes x * id                                     -> `q8_0_tie_row`

The same places also depend on how the quotient is formed. Q4_K and Q6_K divide by d
(`(x + dm) / d`, `x / d`) while Q8_0 multiplies by id = 1 / d, and for a d whose reciprocal is not
exact in f32 the two readings round some inputs to different codes. `q4k_block` sub-blocks 4 and 5,
`q6k_block` sub-block 3 and `q8_0_recip_row` place inputs where they part. A last case is the int8
sub-block scale of Q6_K, which saturates at 127 when a sub-block's scale is the negative of the
largest one (`q6k_saturating_block`).
"""
from __future__ import annotations

import numpy as np

F = np.float32


def _grid4(d: float, m: float, l: np.ndarray) -> np.ndarray:
    """x = d * l - m, exact in f32 for the d, m used here (small integers times powers of two)."""
    return (F(d) * l.astype(F) - F(m)).astype(F)


def _below_half(d, k: int):
    """The f32 one step toward zero from sign(k) * d * (|k| + 0.5)."""
    h = F(F(d) * F(abs(k) + 0.5))
    return F(np.sign(k + 0.5)) * np.nextafter(h, F(0), dtype=F)


def q4k_block():
    """One 256-element Q4_K block and what its bytes must hold.

    sub-block 0: grid d = 63 * 2^-6, m = 63 * 2^-6 (the largest scale and min: the fit returns them
                 exactly, so max_scale = max_min = 63 * 2^-6, inv_scale = inv_min = 64, and the
                 super-block d = dmin = f16(2^-6) = 2^-6).
    sub-block 1: grid d = 41 * 2^-7 (fit exact): inv_scale * scl = 64 * 41 * 2^-7 = 20.5 -> scale code 21.
    sub-block 2: grid m = 25 * 2^-7 (fit exact): inv_min * min = 12.5 -> min code 13.
    sub-block 3: grid d = 40 * 2^-6, m = 10 * 2^-6 (codes 40 and 10) with one element moved to
                 d * (6 + 0.5) - m: its final code is (x + dm) / d = 6.5 exactly -> 7. The move shifts
                 the sub-block's least-squares fit far less than half a scale / min code, so the codes
                 stay 40 / 10 (asserted separately from the tie).
    sub-block 4: grid d = 41 * 2^-6, m = 0 (codes 41 and 0) with three elements moved to d * (k + 0.5) for
                 k = 0, 3, 6: (x + 0) / d = k + 0.5 exactly -> k + 1, while x * f32(1 / d) lies just below the
                 half in f32 (1 / d rounds down) -> k.
    sub-block 5: grid d = 11 * 2^-6, m = 0 (codes 11 and 0) with three elements one f32 step below
                 d * (k + 0.5) for k = 2, 4, 8: x / d rounds to just below the half -> k, while
                 x * f32(1 / d) rounds to k + 0.5 exactly (1 / d rounds up) -> k + 1.
    sub-blocks 6-7: plain grids (d = (8 + j) * 2^-6, m = (4 + j) * 2^-6).
    Returns x, the expected scale codes, min codes, and a list of (element index, expected 4-bit code).
    """
    rng = np.random.default_rng(1234)
    x = np.zeros(256, F)

    def lvec():
        lv = rng.integers(0, 16, 32)
        lv[rng.choice(32, 2, replace=False)] = [0, 15]  # both ends present: min and max of the grid
        return lv

    sc = np.zeros(8, np.int64)
    mn = np.zeros(8, np.int64)
    checks = []
    # 0: the maxima
    l0 = lvec()
    x[0:32] = _grid4(63 * 2.0 ** -6, 63 * 2.0 ** -6, l0)
    sc[0], mn[0] = 63, 63
    # 1: scale 41 * 2^-7 -> 20.5 -> 21 ; min 0
    l1 = lvec()
    x[32:64] = _grid4(41 * 2.0 ** -7, 0.0, l1)
    sc[1], mn[1] = 21, 0
    # 2: min 25 * 2^-7 -> 12.5 -> 13 ; scale 2^-3 -> 64 * 2^-3 = 8
    l2 = lvec()
    x[64:96] = _grid4(2.0 ** -3, 25 * 2.0 ** -7, l2)
    sc[2], mn[2] = 8, 13
    # 3: codes 40 / 10 and one final-code tie at 6.5
    l3 = lvec()
    t = int(np.flatnonzero((l3 != 0) & (l3 != 15))[0])
    x[96:128] = _grid4(40 * 2.0 ** -6, 10 * 2.0 ** -6, l3)
    x[96 + t] = F(40 * 2.0 ** -6) * F(6.5) - F(10 * 2.0 ** -6)
    sc[3], mn[3] = 40, 10
    checks.append((96 + t, 7))
    for i in range(32):
        if i != t:
            checks.append((96 + i, int(l3[i])))
    # 4, 5: division against multiplication by the reciprocal
    for j, code, moves in ((4, 41, ((0, 0), (3, 0), (6, 0))), (5, 11, ((2, -1), (4, -1), (8, -1)))):
        lj = lvec()
        d = F(code * 2.0 ** -6)
        x[32 * j:32 * j + 32] = _grid4(d, 0.0, lj)
        sc[j], mn[j] = code, 0
        free = [i for i in range(32) if lj[i] not in (0, 15)]
        moved = {}
        for (k, step), i in zip(moves, free):
            moved[i] = k + 1 if step == 0 else k
            x[32 * j + i] = _below_half(d, k) if step else F(d * F(k + 0.5))
        for i in range(32):
            checks.append((32 * j + i, moved.get(i, int(lj[i]))))
    for j in range(6, 8):  # d_j = (8 + j) * 2^-6, m_j = (4 + j) * 2^-6: codes 8 + j and 4 + j
        lj = lvec()
        x[32 * j:32 * j + 32] = _grid4((8 + j) * 2.0 ** -6, (4 + j) * 2.0 ** -6, lj)
        sc[j], mn[j] = 8 + j, 4 + j
    return x, sc, mn, checks


def q6k_block():
    """One 256-element Q6_K block and what its bytes must hold.

    sub-block 0: grid s = 2^-3, codes in [-32, 31] with -32 present (the largest magnitude): the fit
                 returns 2^-3, the largest scale, so iscale = -128 / 2^-3 = -1024 and the super-block
                 d = f16(1 / iscale) = -2^-10; this sub-block's int8 scale is -128.
    sub-block 1: grid s = 5 * 2^-11 with codes in {-32, 0, +-2, +-4}: every x^2-weighted sum of the fit is
                 exact, so the fit returns 5 * 2^-11 and iscale * s = -2.5 -> int8 scale -3.
    sub-block 2: grid s = 7 * 2^-10 (int8 scale -7: d = -2^-10 * -7 = s) with one element at s * 4.5 and
                 one at -s * 10.5: x / d = 4.5 and -10.5 exactly -> codes 5 and -11. The two moved
                 elements shift the fit far less than half an int8 scale step (asserted separately).
    sub-block 3: grid s = 13 * 2^-10 (int8 scale -13: d = s) with elements one f32 step toward zero from
                 s * (|k| + 0.5) * sign(k) for k = 19, 16, -19, -9: x / d falls just short of the half -> k,
                 while x * f32(1 / d) rounds to the half exactly -> one further from zero.
    sub-blocks 4-15: plain grids s = 2^-10 * (10 + j).
    Returns x, the expected int8 scales, and a list of (element index, expected signed code q - 32).
    """
    rng = np.random.default_rng(4321)
    x = np.zeros(256, F)
    scales = np.zeros(16, np.int64)
    checks = []

    def lvec():
        lv = rng.integers(-31, 32, 16)
        lv[rng.integers(16)] = -32
        return lv

    l0 = lvec()
    x[0:16] = (F(2.0 ** -3) * l0.astype(F)).astype(F)
    scales[0] = -128
    l1 = rng.choice(np.array([0, 2, -2, 4, -4]), 16)
    l1[3] = -32
    x[16:32] = (F(5 * 2.0 ** -11) * l1.astype(F)).astype(F)
    scales[1] = -3
    s2 = F(7 * 2.0 ** -10)
    l2 = lvec()
    x[32:48] = (s2 * l2.astype(F)).astype(F)
    # two ties, away from the -32 element (which fixes the fit's first rounding)
    free = [i for i in range(16) if l2[i] != -32]
    ta, tb = free[0], free[1]
    x[32 + ta] = s2 * F(4.5)
    x[32 + tb] = s2 * F(-10.5)
    scales[2] = -7
    checks += [(32 + ta, 5), (32 + tb, -11)]
    for i in range(16):
        if i not in (ta, tb):
            checks.append((32 + i, int(l2[i])))
    s3 = F(13 * 2.0 ** -10)
    l3 = lvec()
    x[48:64] = (s3 * l3.astype(F)).astype(F)
    scales[3] = -13
    free = [i for i in range(16) if l3[i] != -32]
    moved = {}
    for k, i in zip((19, 16, -19, -9), free):
        x[48 + i] = _below_half(s3, k)
        moved[i] = k
    for i in range(16):
        checks.append((48 + i, moved.get(i, int(l3[i]))))
    for j in range(4, 16):
        lj = lvec()
        x[16 * j:16 * j + 16] = (F(2.0 ** -10 * (10 + j)) * lj.astype(F)).astype(F)
        scales[j] = -(10 + j)
    return x, scales, checks


def q6k_saturating_block():
    """A Q6_K block whose sub-block 1 is the negation of sub-block 0.

    sub-block 0: grid s = 2^-3 with codes in [-32, 31] and -32 present (x = -4, the block's largest
                 magnitude): the fit returns 2^-3, so iscale = -1024, the super-block d = -2^-10 and this
                 sub-block's int8 scale is -128.
    sub-block 1: -x0. Its fit rounds the same codes at the negated iscale, so its scale is -2^-3 exactly and
                 does not replace sub-block 0's as the largest (ties keep the first). iscale * -2^-3 = 128,
                 which an int8 cannot hold: candle clamps it to 127. The codes are then
                 x / (-2^-10 * 127) = l0 * 128 / 127, which rounds to l0 for |l0| <= 32.
    sub-blocks 2-15: plain grids s = 2^-10 * (10 + j).
    Returns x, the expected int8 scales, and the expected signed codes of sub-block 1.
    """
    rng = np.random.default_rng(777)
    x = np.zeros(256, F)
    scales = np.zeros(16, np.int64)
    l0 = rng.integers(-31, 32, 16)
    l0[5] = -32
    x[0:16] = (F(2.0 ** -3) * l0.astype(F)).astype(F)
    x[16:32] = -x[0:16]
    scales[0], scales[1] = -128, 127
    for j in range(2, 16):
        lj = rng.integers(-31, 32, 16)
        lj[rng.integers(16)] = -32
        x[16 * j:16 * j + 16] = (F(2.0 ** -10 * (10 + j)) * lj.astype(F)).astype(F)
        scales[j] = -(10 + j)
    return x, scales, l0.astype(np.int64)


def qkx1_first_rounding_case():
    """A 32-element sub-block for the Q4_K fit at ntry = 1: min = 0 and max = 15 * 2^-2, so
    iscale = 15 / 3.75 = 4 exactly and the elements at 2^-2 * (l + 0.5) round from l + 0.5 exactly.
    Returns x and the codes of that first rounding (half away from zero: l + 1)."""
    l = np.array([0, 15] + [2, 4, 6, 8, 10, 12, 1, 3, 5, 7, 9, 11, 13, 14, 0] * 2, np.int64)
    x = (F(2.0 ** -2) * l.astype(F)).astype(F)
    codes = l.copy()
    for i in (2, 3, 4, 5, 6, 7):  # even l moved to l + 0.5: ties; half away from zero gives l + 1
        x[i] = F(2.0 ** -2) * F(l[i] + 0.5)
        codes[i] = l[i] + 1
    for i in (8, 9, 10):  # odd l moved to l + 0.5: l + 1 under either tie rule
        x[i] = F(2.0 ** -2) * F(l[i] + 0.5)
        codes[i] = l[i] + 1
    return x, codes


def qx_first_rounding_case():
    """16 elements for make_qx_quants(16, 32, x, L, 0): the first element -32 is the largest magnitude,
    so iscale = -32 / -32 = 1 and every x is rounded as it stands. Returns x and the codes l."""
    x = np.array([-32.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 4.5, -4.5, 30.5, -30.5, 6.5, 3.0, -7.0, 0.0, 12.5], F)
    codes = np.array([-32, 3, -3, 1, -1, 2, -2, 5, -5, 31, -31, 7, 3, -7, 0, 13], np.int64)
    return x, codes


def q8_0_tie_row(k: int) -> np.ndarray:
    """A k-wide row whose Q8_0 blocks have amax = 127 * 2^-3 (d = 2^-3, 1 / d = 8 exactly) and
    elements at 2^-3 * (k + 0.5): exact ties of round(x / d)."""
    x = np.zeros(k, F)
    vals = np.array([127.0, -2.5, 2.5, 0.5, -0.5, 6.5, -6.5, 100.5, -126.5, 10.5, 1.5, -1.5], F) * F(2.0 ** -3)
    for b in range(0, k, 32):
        x[b:b + vals.size] = vals
    return x


Q8_0_RECIP_KS = (2, 4, 8, 10, 16, 20, 32, -2, -9, -17, -33)


def q8_0_recip_row(k: int) -> np.ndarray:
    """A k-wide row whose Q8_0 blocks have amax = 127 * 3 * 2^-5 (d = 3 * 2^-5 exactly; f32(1 / d) rounds
    up) and elements one f32 step toward zero from sign(j) * d * (|j| + 0.5) for the j of Q8_0_RECIP_KS:
    candle's x * id rounds to the half exactly and gives the code one further from zero than j, while
    x / d would give j."""
    x = np.zeros(k, F)
    d = F(3 * 2.0 ** -5)
    vals = np.array([F(127) * d] + [_below_half(d, j) for j in Q8_0_RECIP_KS], F)
    for b in range(0, k, 32):
        x[b:b + vals.size] = vals
    return x


def weight_tie_rows(k: int) -> np.ndarray:
    """Rows for the GPU quantizer test: the Q4_K and Q6_K tie blocks tiled across a k-wide row, the Q8_0
    tie row, the saturating Q6_K block tiled, and the Q8_0 reciprocal row (k a multiple of 256)."""
    b4 = q4k_block()[0]
    b6 = q6k_block()[0]
    r4 = np.tile(b4, k // 256)
    r6 = np.tile(b6, k // 256)
    mixed = np.concatenate([b4 if i % 2 == 0 else b6 for i in range(k // 256)])
    sat = np.tile(q6k_saturating_block()[0], k // 256)
    return np.stack([r4, r6, mixed, q8_0_tie_row(k), sat, q8_0_recip_row(k)]).astype(F)
