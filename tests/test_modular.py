"""The FP64 modular product of the product kernels' epilogues (oz2::mod_mul_f64 in
oztt_amd/csrc/oz2_modular.hpp), emulated with numpy's IEEE binary64 operations and checked against
exact integer arithmetic.

The device function computes t = RN(c * yr) with yr = RN(y / m), f = t - floor(t) clamped below 1
(v_fract_f64), and RN(f * m + 2^52) (v_fma_f64), whose low 32 bits are the result: a representative
of (c * y) mod m in [0, m], m standing for 0. The emulation rounds f * m + 2^52 in 80-bit extended
precision before binary64; f * m lies within 2^-13 of an integer r, so neither rounding can move the
sum off 2^52 + r. The kernels use it for the CRT digit of an int32 product
(|c| < 2^31, y < m <= 255: reference recon_crt.cpp:293's residue step) and for the FP8 route's terms
(|P| < 2^24, coef < m <= 2401). CPU only.
"""
import numpy as np


def mod_mul_f64(c: np.ndarray, y: np.ndarray, m: np.ndarray) -> np.ndarray:
    md = m.astype(np.float64)
    yr = y.astype(np.float64) / md
    t = c.astype(np.float64) * yr
    f = np.minimum(t - np.floor(t), np.nextafter(1.0, 0.0))
    p = f.astype(np.longdouble) * md.astype(np.longdouble)
    # the margin the rounding relies on: f m is within 1/4 of an integer
    assert np.all(np.abs(p - np.rint(p)) < 0.25)
    g = (p + np.longdouble(2.0**52)).astype(np.float64)
    assert np.all((g >= 2.0**52) & (g < 2.0**53))
    return (g.view(np.uint64) & np.uint64(0xFFFFFFFF)).astype(np.int64)


def _check(c, y, m):
    got = mod_mul_f64(c, y, m)
    want = np.array([(int(a) * int(b)) % int(q) for a, b, q in zip(c, y, m)], dtype=np.int64)
    assert np.all((got >= 0) & (got <= m))
    np.testing.assert_array_equal(got % m, want)


def test_int8_digit_range_random():
    rng = np.random.default_rng(7)
    n = 200_000
    m = rng.integers(2, 256, n)
    y = rng.integers(0, 1 << 30, n) % m
    c = rng.integers(-(1 << 31), 1 << 31, n)
    _check(c, y, m)


def test_fp8_term_range_random():
    rng = np.random.default_rng(8)
    n = 200_000
    m = rng.integers(2, 2402, n)
    y = rng.integers(0, 1 << 30, n) % m
    c = rng.integers(-(1 << 24) + 1, 1 << 24, n)
    _check(c, y, m)


def test_exact_multiples_and_extremes():
    # x/m an integer: the floor may land one below, the select must map r = m back to 0
    rows = []
    for m in (2, 3, 5, 7, 127, 251, 253, 255, 256, 1021, 2401):
        for y in (1, 2, m - 1, (m - 1) // 2 or 1):
            for c in (0, m, -m, 3 * m, -(3 * m), (2**31 - 1) // m * m, -((2**31) // m) * m,
                      2**31 - 1, -(2**31), 2**31 - 2, -(2**31) + 1, (1 << 24) - 1, -(1 << 24) + 1):
                rows.append((c, y, m))
    c, y, m = (np.array(v, dtype=np.int64) for v in zip(*rows))
    _check(c, y, m)


def test_every_product_for_small_moduli():
    # all residues c mod m and all y < m, for a few moduli, shifted by large multiples of m
    for m in (2, 9, 251, 255):
        c0 = np.arange(m, dtype=np.int64)
        cc, yy = np.meshgrid(c0, np.arange(m, dtype=np.int64))
        for shift in (0, (2**31 - m) // m * m, -((2**31) // m) * m):
            _check(cc.ravel() + shift, yy.ravel(), np.full(cc.size, m))
