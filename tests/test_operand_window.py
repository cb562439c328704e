"""The operands' own CRT window (plan2.cpp plan_scheme2), on the CPU.

The reference sizes the moduli product M for the worst case |C'_ij| <= K 2^(2b) of the integer product
C' = A'B' (moduli.hpp:338-344). The plan also bounds max |C'_ij| from the operands (Cauchy-Schwarz on
the rows of A' and the columns of B': Plan2.bound_log2) and computes with a smaller set when that set's
M still exceeds twice the bound; the exact CRT then recovers the same C' and C is bit for bit the same.

Pinned here with exact integers: A' and B' are rebuilt from the oracle's scale and digits (the
reference's split, scale_bits.h:34-62 and digits.h:80-112) as Python integers, C' = A'B' exactly, and
max |C'| must stay below 2^bound_log2 on heavy-tailed rows, spikes, elements 600 binades below their
row's maximum, and on inputs that make Cauchy-Schwarz tight (equal magnitudes, maxima just below a
power of two), where the bound must also lie within 1/8 bit of the exact maximum: a bound too low fails the
first check, one too loose (norms taken over the maxima, a dropped power of two) the second. The whole
oracle chain then gives the same C from the smaller set and from the reference's.
"""
import math

import numpy as np
import pytest

import oztt_amd as oz
from tests.oracle_chains import oz2_chain


def exact_operands(oracle, A, B, b, nd):
    """A' (M x K) and B' (K x N) as Python integers: the digits of x 2^delta, top digit first, weights
    2^(20 (nd - 1 - j))."""
    M, K = A.shape
    N = B.shape[1]
    shift = b - 20 * (nd - 1)
    dA, fA = oracle.scale(A, M, K, 0, 1, shift)
    dB, fB = oracle.scale(B, K, N, 1, 1, shift)
    assert fA == 0 and fB == 0
    out = []
    for X, rows, cols, mode, d in ((A, M, K, 0, dA), (B, K, N, 1, dB)):
        dig = oracle.digits(X, rows, cols, mode, d, nd).astype(np.int64)
        x = np.zeros((rows, cols), dtype=object)
        for j in range(nd):
            x = x + dig[..., j].astype(object) * (1 << (20 * (nd - 1 - j)))
        out.append(x)
    return out


def max_abs_product(Ai, Bi) -> int:
    return max(abs(int(v)) for v in np.dot(Ai, Bi).ravel())


def cases():
    rng = np.random.default_rng(11)
    K = 512
    heavy = lambda phi, r, c: (rng.random((r, c)) - 0.5) * np.exp(phi * rng.standard_normal((r, c)))
    flat = np.full((16, K), 0.75)
    flat[1::2] *= -1.0
    below = np.full((16, K), 1.0 - 2.0 ** -52)  # maxima just below a power of two: A' = 2^b (1 - 2^-52)
    spike = heavy(0.5, 16, K) * 2.0 ** -40
    spike[:, 7] = 3.0
    deep = heavy(1.0, 16, K)
    deep[:, 1:] *= 2.0 ** -600  # every element but the first 600 binades below the row's maximum
    return [
        ("uniform", heavy(0.0, 16, K), heavy(0.0, K, 16)),
        ("phi 0.5", heavy(0.5, 16, K), heavy(0.5, K, 16)),
        ("phi 4", heavy(4.0, 16, K), heavy(4.0, K, 16)),
        ("equal magnitudes", flat, np.full((K, 16), 0.75)),
        ("just below 1", below, below.T.copy()),
        ("spikes", spike, spike.T.copy()),
        ("600 binades", deep, deep.T.copy()),
    ]


@pytest.mark.parametrize("name,A,B", cases(), ids=[c[0] for c in cases()])
def test_bound_holds_on_the_exact_integer_product(oracle, name, A, B):
    M, K = A.shape
    N = B.shape[1]
    p = oz.plan2(A, B, M, N, K, oz.Format.INT8)
    assert math.isfinite(p.bound_log2)
    Ai, Bi = exact_operands(oracle, A, B, p.b, p.nd)
    # the premise of the bound: |A'_ik| <= 2^b |a_ik| / 2^ceil(log2 max_k |a_ik|) + 2
    for X, Xi, axis in ((A, Ai, 1), (B, Bi, 0)):
        t = np.exp2(np.ceil(np.log2(np.abs(X).max(axis=axis, keepdims=True))))
        lim = np.abs(X) / t * 2.0 ** p.b + 2.0
        assert all(abs(int(v)) <= float(w) for v, w in zip(Xi.ravel(), lim.ravel()))
    c = max_abs_product(Ai, Bi)
    assert c > 0 and math.log2(c) < p.bound_log2
    # never above the planned window, and within 1/8 bit of the exact maximum where the operands make
    # Cauchy-Schwarz tight (equal magnitudes and signs within every row and column)
    assert p.bound_log2 <= 2 * p.b + math.log2(K) + 1e-9
    if name in ("equal magnitudes", "just below 1"):
        assert p.bound_log2 - math.log2(c) < 0.125
    # the execution set covers twice the bound; the set it replaced is the window's
    assert p.log2M > p.bound_log2 + 1.0
    if p.S_window:
        full = oz.plan2(A, B, M, N, K, oz.Format.INT8, full_window=True)
        assert full.S_window == 0 and full.S == p.S_window > p.S and full.S == p.rS


def test_smaller_set_gives_the_same_c(oracle):
    """Where the bound saves a modulus (K = 8192, phi 0.5: the C3 distribution), the oracle's whole chain
    gives the same C from the execution set and from the reference's set for the window K 2^(2b)."""
    M = N = 32
    K = 8192
    a, b = oz.eval_inputs(3, 0.5, M * K, K * N)
    A, B = a.reshape(M, K), b.reshape(K, N)
    p = oz.plan2(A, B, M, N, K, oz.Format.INT8, reconstruction=oz.Reconstruction.TwoPass)
    assert p.S_window == p.rS and p.S < p.rS
    ms = [p.m[i] for i in range(p.S)]
    rm = [p.rm[i] for i in range(p.rS)]
    c_small = oz2_chain(oracle, A, B, ms, p.b, p.nd)
    c_full = oz2_chain(oracle, A, B, rm, p.b, p.nd)
    np.testing.assert_array_equal(c_small.view(np.uint64), c_full.view(np.uint64))


def test_window_bound_is_not_used_without_measured_operands():
    """A width fixed by the caller with a fixed pass count measures nothing: the window stays K 2^(2b)."""
    M = N = 64
    K = 4096
    a, b = oz.eval_inputs(7, 0.5, M * K, K * N)
    p = oz.plan2(a, b, M, N, K, oz.Format.INT8, fixed_bits=54, reconstruction=oz.Reconstruction.OnePass)
    assert math.isinf(p.bound_log2) and p.S_window == 0 and p.S == p.rS



def test_fp8_fewest_products_set(oracle):
    """On the FP8 route the execution set is the one of fewest e4m3 digit products for the window: at C4's
    K = 16384 (phi 2) it mixes one-digit moduli (at most 33, residue = digit) with the route's squares and
    Karatsuba moduli; it is pairwise coprime, covers twice the bound, and the oracle's chain gives the same
    C from it as from the route's own set."""
    M = N = 16
    K = 16384
    a, b = oz.eval_inputs(4, 2.0, M * K, K * N)
    A, B = a.reshape(M, K), b.reshape(K, N)
    p = oz.plan2(A, B, M, N, K, oz.Format.FP8)
    ms = [p.m[i] for i in range(p.S)]
    assert p.fp8_digits and p.S_window == p.rS and p.nprod < p.rnprod
    assert all(math.gcd(x, y) == 1 for i, x in enumerate(ms) for y in ms[i + 1:])
    assert any(x <= 33 for x in ms) and p.log2M > p.bound_log2 + 1.0
    assert abs(sum(math.log2(x) for x in ms) - p.log2M) < 1e-9
    c_small = oz2_chain(oracle, A, B, ms, p.b, p.nd)
    c_full = oz2_chain(oracle, A, B, [p.rm[i] for i in range(p.rS)], p.b, p.nd)
    np.testing.assert_array_equal(c_small.view(np.uint64), c_full.view(np.uint64))


def parallel_operands(phi: float, n: int = 64, K: int = 8192, seed: int = 5):
    """Rows of A and columns of B that are the same heavy-tailed vector v up to signs, A_i = s_i v and
    B_j = s_j v: C'_ii = ||A'_i||^2 makes Cauchy-Schwarz tight, so max |C'| reaches the bound, while the
    heavy tail keeps the bound bits below the window K 2^(2b)."""
    rng = np.random.default_rng(seed)
    v = (rng.random(K) - 0.5) * np.exp(phi * rng.standard_normal(K))
    s = rng.choice([-1.0, 1.0], size=(n, K))
    return s * v, (s * v).T.copy()


def test_tight_bound_near_the_smaller_modulus(oracle):
    """phi 0.5: max |C'| equals the bound to 1/100 bit and lies within 1/8 bit of M/2 of the smaller set
    that computes (15 moduli where the window needs 16); the oracle's chain gives the same C from that set
    as from the window's."""
    A, B = parallel_operands(0.5)
    n, K = A.shape
    p = oz.plan2(A, B, n, n, K, oz.Format.INT8)
    Ai, Bi = exact_operands(oracle, A, B, p.b, p.nd)
    c = math.log2(max_abs_product(Ai, Bi))
    assert p.S_window == p.rS > p.S
    assert c < p.bound_log2 < c + 0.01
    assert c < p.log2M - 1.0 < c + 0.125
    ms = [p.m[i] for i in range(p.S)]
    c_small = oz2_chain(oracle, A, B, ms, p.b, p.nd)
    c_full = oz2_chain(oracle, A, B, [p.rm[i] for i in range(p.rS)], p.b, p.nd)
    np.testing.assert_array_equal(c_small.view(np.uint64), c_full.view(np.uint64))
