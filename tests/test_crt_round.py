"""The rounding step of the byte-digit CRT kernel (magnitude40 in oztt_amd/csrc/oz2_crt.hip), emulated
with numpy's IEEE binary64 operations and checked against exact rational arithmetic: the sequence as
first written (round_limbs, which tracks the first stage that rounds) and the one the kernel runs now
(round_limbs_direct, which reads the fix off every stage's error).

The kernel rounds V = sum_l Y_l 2^(40 l) (normalized limbs: integers in [0, 2^40), at most 5) to the
nearest FP64 value, ties to even, with a cascade of exact FP64 additions from the top limb down:
s_j = RN(s_(j-1) + T_j) with T_j the j-th limb from the top at its weight, and the error of each
stage from FastTwoSum. At most one stage rounds (the terms below a rounding stage are worth less
than half an ulp of it), so s is RN(V) except when the first rounding stage left exactly +ulp/2 and a
nonzero term remains below it: then V lies above the midpoint and s moves one ulp up. The limbs
carry the kernel's scale of 2^-90, which changes no rounding. CPU only."""
from fractions import Fraction

import numpy as np

SCALE = 2.0 ** -90


def half_ulp(s: float) -> float:
    e = np.frexp(s)[1] - 1  # s in [2^e, 2^(e+1))
    return 2.0 ** (e - 53)


def round_limbs(y):
    """The kernel's sequence on scaled limbs y (y[l] = Y_l 2^-90), in float64."""
    L = len(y)
    T = [float(np.ldexp(y[L - 1 - j], 40 * (L - 1 - j))) for j in range(L)]
    s = T[0]
    have, ek, hk, lower = False, 0.0, 0.0, False
    for j in range(1, L):
        sn = s + T[j]
        if have:
            lower = lower or T[j] != 0.0
        else:
            e = T[j] - (sn - s)
            if e != 0.0:
                have, ek, hk = True, e, half_ulp(sn)
        s = sn
    if have and ek == hk and lower:
        s = s + 2.0 * hk
    return s


def round_limbs_direct(y):
    """The kernel's present sequence: the same cascade with every stage's FastTwoSum error kept, and the
    fix read off directly. Only the first stage that rounds can leave an error of exactly h = ulp(s)/2
    (a later stage's error is its whole term, below the grid unit of the rounding stage, which is at
    most h), and the sum s no longer moves after it, so h is that of the final s: s moves one ulp up
    exactly when some stage j has e_j == h and a nonzero term follows it."""
    L = len(y)
    T = [float(np.ldexp(y[L - 1 - j], 40 * (L - 1 - j))) for j in range(L)]
    s = T[0]
    e = [0.0] * L
    for j in range(1, L):
        sn = s + T[j]
        e[j] = T[j] - (sn - s)
        s = sn
    if s == 0.0:
        return s
    h = half_ulp(s)
    fix, below = False, False
    for j in range(L - 1, 0, -1):
        fix = fix or (below and e[j] == h)
        below = below or T[j] != 0.0
    return s + 2.0 * h if fix else s


def exact_rn(Y) -> float:
    v = sum(Fraction(int(t)) * 2 ** (40 * l) for l, t in enumerate(Y)) * Fraction(1, 2 ** 90)
    return float(v)  # Python rounds a Fraction to the nearest double, ties to even


def check(Y):
    y = [float(t) * SCALE for t in Y]
    want = exact_rn(Y)
    got = round_limbs(y)
    assert got == want, (Y, got, want)
    got = round_limbs_direct(y)
    assert got == want, ("direct", Y, got, want)


def test_random_limbs():
    rng = np.random.default_rng(40)
    for L in (2, 3, 4, 5):
        for _ in range(20000):
            Y = [int(v) for v in rng.integers(0, 1 << 40, L)]
            top = int(rng.integers(0, L))
            for l in range(top + 1, L):  # leading zero limbs of every length
                Y[l] = 0
            if rng.random() < 0.5:
                Y[top] = int(rng.integers(1, 1 << int(rng.integers(1, 41))))  # short top limb
            check(Y)


def test_ties_and_near_ties():
    """V exactly at, just above and just below a midpoint of the FP64 grid, for the rounding falling
    in every limb position and every length of the top limb."""
    rng = np.random.default_rng(41)
    for L in (3, 4, 5):
        for _ in range(4000):
            V = int(rng.integers(1, 1 << 62)) << int(rng.integers(0, 40 * L - 62))
            n = V.bit_length()
            if n <= 53:
                continue
            g = n - 53  # the rounding position
            base = (V >> g) << g
            mid = base + (1 << (g - 1))
            for v in (mid, mid + 1, mid - 1, base, mid + (1 << max(g - 45, 0))):
                if v.bit_length() > 40 * L:
                    continue
                Y = [(v >> (40 * l)) & ((1 << 40) - 1) for l in range(L)]
                check(Y)


def test_zero_and_single_bits():
    for L in (2, 4, 5):
        check([0] * L)
        for p in range(40 * L):
            Y = [0] * L
            Y[p // 40] = 1 << (p % 40)
            check(Y)
