"""The CPU oracle pinned against what the reference itself holds and against closed forms.

- inputs: the reference's recorded input hashes ahash/bhash (dgemm_ref.log:6,12);
- end to end: the reference's published output hash of II INT8 at 128^3 (tools/validated/quick.csv:13);
- ModRound: the reference's worked examples (sfpu_tf_proc.h:271, :303, :312);
- digits: the reference's example x = 2^-55 + 2^-80 -> A' = 0 (digits.h:44) and |A' - X| <= 1;
- split_f64: exactness hi + mid + lo == x*2^d (checked in exact rational arithmetic);
- residues: r == A' (mod m) and |r| <= floor(m/2), A' recomposed from the digits;
- exact CRT: against Python integers; Dot2 and binary128 references against exact rationals.
"""
import math
import random
from fractions import Fraction

import numpy as np
import pytest

from tests.oracle_lib import load_oracle


@pytest.fixture(scope="module")
def orc():
    return load_oracle()


@pytest.mark.parametrize("phi,ahash,bhash", [(0.0, 0x1d42484422793a1f, 0xd122911129734494),
                                             (0.5, 0xef34b292fe872ee4, 0xdf4dbd7b81b31c40)])
def test_inputs_match_reference_hashes(orc, phi, ahash, bhash):
    n = 4096
    a, b = orc.inputs(7, phi, n * n, n * n)
    assert orc.hash(a) == ahash and orc.hash(b) == bhash


INT8_K128 = [255, 254, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 83, 139]  # moduli at K=128, b=54


def test_end_to_end_reference_hash_quick_int8(orc):
    n, b, nd = 128, 54, 3
    a, bb = orc.inputs(7, -1.0, n * n, n * n)
    A, B = a.reshape(n, n), bb.reshape(n, n)
    shift = b - 40
    dA, fa = orc.scale(A, n, n, 0, 1, shift)
    dB, fb = orc.scale(B, n, n, 1, 1, shift)
    assert fa == fb == 0
    pa = orc.residues(A, n, n, 0, dA, nd, INT8_K128)
    pb = orc.residues(B, n, n, 1, dB, nd, INT8_K128)
    C = np.stack([orc.gemm_i8(pa[s], pb[s])[0] for s in range(len(INT8_K128))])
    out = orc.crt_ref(C, n, n, INT8_K128, b, nd, False, dA, dB)
    assert orc.hash(out) == 0xfe063f5214e93e2e
    # the exact reconstruction is at least as accurate (long-double reference)
    R = A.astype(np.longdouble) @ B.astype(np.longdouble)
    ex = orc.crt_exact(C, n, n, INT8_K128, b, nd, dA, dB)
    e_ref = float(np.sqrt(np.sum((out.reshape(n, n) - R) ** 2) / np.sum(R ** 2)))
    e_ex = float(np.sqrt(np.sum((ex.reshape(n, n) - R) ** 2) / np.sum(R ** 2)))
    assert e_ex <= e_ref < 8 * np.finfo(float).eps


def f32(x):
    return float(np.float32(x))


@pytest.mark.parametrize("d,m,expect", [(2.0 ** 24, 29, -8), (-16425964.0, 2005, -1004)])
def test_modround_reference_examples(orc, d, m, expect):
    assert orc.modround(d, float(m), f32(1.0 / m)) == expect


def test_modround_crt_example(orc):
    # sfpu_tf_proc.h:303: m = 3475, r = 1737, y = 3474 gives k = 1738 (one beyond floor(m/2))
    m = 3475
    assert orc.modround(f32(1737 * 3474), float(m), f32(1.0 / m)) == 1738


def test_modround_symmetric_below_2_22(orc):
    rng = np.random.default_rng(5)
    for m in [255, 254, 253, 199, 47, 3]:
        ri = f32(1.0 / m)
        for d in rng.integers(-(2 ** 22) + 1, 2 ** 22, 2000):
            r = orc.modround(float(d), float(m), ri)
            assert (int(d) - int(r)) % m == 0 and abs(r) <= m // 2


def test_split_f64_exact(orc):
    rng = random.Random(11)
    xs = [1.0, -1.0, 0.5, 2.0 ** -30, 1.0 + 2.0 ** -52, -(1.0 + 2.0 ** -23 + 2.0 ** -52)]
    xs += [rng.uniform(-1, 1) * 2.0 ** rng.randint(-60, 0) for _ in range(3000)]
    # tails around the rounding point of the 23-bit head: low 30 bits = 2^29 exactly and 2^29 + c
    for _ in range(200):
        x = rng.uniform(0.5, 1.0)
        u = np.frombuffer(np.float64(x).tobytes(), np.uint64)[0]
        for low in (0x20000000, 0x20000000 + rng.randint(1, 127), 0x1FFFFFFF):
            v = (int(u) & ~0x3FFFFFFF) | low
            xs.append(float(np.frombuffer(np.uint64(v).tobytes(), np.float64)[0]))
    for x in xs:
        d = rng.randint(-5, 20)
        hi, mid, lo = (float(v) for v in orc.load_triple(x, d))
        if abs(x) * 2.0 ** d >= 2.0 ** -72:
            assert Fraction(hi) + Fraction(mid) + Fraction(lo) == Fraction(x) * Fraction(2) ** d, (x, d)


def digits_to_int(dig):
    nd = len(dig)
    return sum(int(dig[j]) * (1 << (20 * (nd - 1 - j))) for j in range(nd))


def test_digits_reference_example_and_bound(orc):
    b, nd = 54, 3
    shift = b - 20 * (nd - 1)
    rng = np.random.default_rng(3)
    X = rng.uniform(-1, 1, (4, 300)) * np.exp2(rng.integers(-40, 0, (4, 300)))
    X[:, 0] = 1.0
    X[0, 1] = 2.0 ** -55 + 2.0 ** -80
    delta, _ = orc.scale(X, 4, 300, 0, 1, shift)
    dig = orc.digits(X, 4, 300, 0, delta, nd)
    assert digits_to_int(dig[0, 1]) == 0  # digits.h:44
    for r in range(4):
        e = shift - int(delta[r])
        for c in range(300):
            Xv = Fraction(float(X[r, c])) / Fraction(2) ** e * Fraction(2) ** b
            assert abs(digits_to_int(dig[r, c]) - Xv) <= 1
            assert abs(dig[r, c, 0]) <= 2 ** (b - 40) and all(abs(dig[r, c, j]) <= 2 ** 19 + 2 ** 16 + 1 for j in (1, 2))


@pytest.mark.parametrize("b,nd", [(54, 3), (72, 4), (96, 5)])
def test_residue_classes(orc, b, nd):
    rng = np.random.default_rng(b)
    X = (rng.uniform(0, 1, (8, 200)) - 0.5) * np.exp(3.0 * rng.standard_normal((8, 200)))
    shift = b - 20 * (nd - 1)
    delta, _ = orc.scale(X, 8, 200, 0, 1, shift)
    moduli = [255, 254, 253, 251, 247, 241, 199, 173, 151, 47, 3]
    dig = orc.digits(X, 8, 200, 0, delta, nd)
    res = orc.residues(X, 8, 200, 0, delta, nd, moduli)
    for r in range(8):
        for c in range(200):
            Ap = digits_to_int(dig[r, c])
            for s, m in enumerate(moduli):
                v = int(res[s, r, c])
                assert (Ap - v) % m == 0 and abs(v) <= m // 2


def test_exact_crt_against_python_integers(orc):
    moduli = [255, 254, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199, 47, 79]
    M = math.prod(moduli)
    rng = random.Random(9)
    for _ in range(300):
        v = rng.randint(-(M - 1) // 2, (M - 1) // 2) >> rng.randint(0, 120)
        r = [v % m - m * rng.randint(-1000, 1000) for m in moduli]
        assert orc.crt_exact_int(np.array(r, np.int32), moduli) == v


def test_quad_and_dot2_references(orc):
    rng = np.random.default_rng(2)
    M, N, K = 7, 9, 300
    A = rng.standard_normal((M, K)) * np.exp2(rng.integers(-20, 20, (M, K)))
    B = rng.standard_normal((K, N))
    rows, cols = np.repeat(np.arange(M), N), np.tile(np.arange(N), M)
    q = orc.quad_sample(A, B, M, N, K, rows, cols)
    hi, lo = orc.dot2(A, B, M, N, K, 0, M)
    for t in range(M * N):
        exact = sum(Fraction(float(A[rows[t], k])) * Fraction(float(B[k, cols[t]])) for k in range(K))
        assert q[t] == float(exact)
        absab = sum(abs(Fraction(float(A[rows[t], k])) * Fraction(float(B[k, cols[t]]))) for k in range(K))
        # Dot2: hi + lo carries the sum to about twice the working precision (gamma_K^2 sum|ab|)
        assert abs(Fraction(float(hi[t])) + Fraction(float(lo[t])) - exact) <= absab * Fraction(2) ** -85


# ---- Scheme I ----------------------------------------------------------------------------------

def test_scheme1_int8_reference_hash(orc):
    """tools/validated/quick.csv:12: I INT8 128^3, uniform seed 7, p = 8 -> hash 6c9693442bfc11b0. The
    oracle's slicer (tfMulR, radix 254), exact diagonal products, triple-float Horner and FP64
    assembly reproduce the reference's output bit for bit."""
    n = 128
    a, b = orc.inputs(7, -1.0, n * n, n * n)
    out, big = orc.oz1_int8_gemm(a, b, n, n, n, 8)
    assert orc.hash(out) == 0x6C9693442BFC11B0
    assert 0 < big < 2 ** 31


def test_scheme1_bf16_reference_hash(orc):
    """quick.csv:2 (and :4, :6, :8): I BF16 128^3, uniform seed 7, p = 10 -> be6558fa9f435fa0. Radix 64
    (tfMulP2), digits +-32, maxima truncated to BF16, all ten diagonals read whole (nsmall = 10)."""
    n, p = 128, 10
    a, b = orc.inputs(7, -1.0, n * n, n * n)
    A, B = a.reshape(n, n), b.reshape(n, n)
    dA, _ = orc.scale(A, n, n, 0, 0, -1)
    dB, _ = orc.scale(B, n, n, 1, 0, -1)
    sa = orc.oz1_slices(A, n, n, 0, dA, p, 64, 32)
    sb = orc.oz1_slices(B, n, n, 1, dB, p, 64, 32)
    Pd, _ = orc.oz1_gemm_diag(sa, sb, p)
    out = orc.oz1_recon(Pd, 64, 0, 10, dA, dB)
    assert orc.hash(out) == 0xBE6558FA9F435FA0


@pytest.mark.parametrize("radix,dmax", [(254, 127), (64, 32)])
def test_scheme1_slices_expand_the_element(orc, radix, dmax):
    """The digits are a balanced radix expansion of x*2^delta: |digit| <= dmax and, with R = dmax/(radix-1),
    |x*2^delta - sum_i d_i radix^-(i+1)| <= R radix^-p (slice_tf_body.h:60-75), checked in exact
    rational arithmetic; rows cover zeros, exact powers of two, tiny and full-range values."""
    rng = np.random.default_rng(radix)
    rows, cols, p = 6, 40, 9
    X = rng.uniform(-1, 1, (rows, cols)) * np.exp2(rng.integers(-40, 40, (rows, 1)))
    X[0] = 0.0
    X[1, :] = 0.25
    X[1, 3] = -0.5
    X[2, 5] = 1.0
    X[2, 6] = 1e-30
    X[3, 7] = -np.nextafter(1.0, 0.0)
    ceil = 1 if radix == 254 else 0
    dA, fl = orc.scale(X, rows, cols, 0, ceil, -1)
    assert fl == 0
    d = orc.oz1_slices(X, rows, cols, 0, dA, p, radix, dmax)
    assert np.abs(d.astype(np.int32)).max() <= dmax
    R = Fraction(dmax, radix - 1)
    for r in range(rows):
        for c in range(cols):
            x = Fraction(float(X[r, c])) * Fraction(2) ** int(dA[r])
            s = sum(Fraction(int(d[i, r, c])) / Fraction(radix) ** (i + 1) for i in range(p))
            assert abs(x) <= Fraction(1, 2) * (1 + Fraction(1, 128))
            assert abs(x - s) <= R / Fraction(radix) ** p * (1 + Fraction(1, 2 ** 20)), (r, c)


def test_scheme1_block_recon_agrees_with_one_block(orc):
    """orc_oz1_recon_blocks (the reconstruction K block by K block) against the one-block reconstruction
    of the summed diagonals: with one block it is the same sequence of operations (bit-identical to
    orc_oz1_recon reading every diagonal whole); with several blocks Horner is linear in P_d, so the
    results agree up to the final rounding (one unit in the last place)."""
    rng = np.random.default_rng(4)
    nkb, ndiag, M, N = 5, 7, 6, 9
    Pb = rng.integers(-(1 << 22), 1 << 22, (nkb, ndiag, M, N)).astype(np.int32)
    dA = rng.integers(-3, 4, M).astype(np.int32)
    dB = rng.integers(-3, 4, N).astype(np.int32)
    one = orc.oz1_recon_blocks(Pb[:1], 64, dA, dB)
    np.testing.assert_array_equal(one.view(np.uint64), orc.oz1_recon(Pb[0], 64, 0, ndiag, dA, dB).view(np.uint64))
    blocks = orc.oz1_recon_blocks(Pb, 64, dA, dB)
    whole = orc.oz1_recon(Pb.astype(np.int64).sum(axis=0).astype(np.int32), 64, 0, 0, dA, dB)
    assert np.all(np.abs(blocks - whole) <= np.spacing(np.abs(whole)))
    assert np.mean(blocks == whole) > 0.9


def test_scheme1_recon_scale_constant(orc):
    """radix^-(L+2) as W 2^qw: W has its top bit set and W 2^qw is within 2^-60 of the exact value; a
    power-of-two radix gives W = 2^63 exactly (plan.hpp:446-460)."""
    for radix, L in [(254, 7), (254, 12), (64, 9), (14, 15)]:
        whi, wlo, qw = orc.oz1_scale_w(radix, L)
        W = (whi << 32) | wlo
        assert W >> 63 == 1
        exact = Fraction(1, radix ** (L + 2))
        assert abs(Fraction(W) * Fraction(2) ** qw - exact) <= exact * Fraction(2) ** -60
    assert orc.oz1_scale_w(64, 9)[:2] == (1 << 31, 0)


def test_scheme1_recon_against_exact_horner(orc):
    """For random diagonal sums the oracle's reconstruction is the exact S radix^-(L+2) 2^-(dA+dB) to within
    the triple-float working precision (~2^-66 of the largest term) plus the final rounding."""
    rng = np.random.default_rng(11)
    ndiag, M, N = 8, 3, 50
    Pd = rng.integers(-(2 ** 30), 2 ** 30, (ndiag, M, N)).astype(np.int32)
    dA = rng.integers(-3, 3, M).astype(np.int32)
    dB = rng.integers(-3, 3, N).astype(np.int32)
    out = orc.oz1_recon(Pd, 254, 1, 0, dA, dB).reshape(M, N)
    for i in range(M):
        for j in range(N):
            S = sum(Fraction(int(Pd[d, i, j])) * 254 ** (ndiag - 1 - d) for d in range(ndiag))
            v = S / Fraction(254) ** (ndiag + 1) * Fraction(2) ** -(int(dA[i]) + int(dB[j]))
            top = Fraction(2 ** 30) * Fraction(254) ** (ndiag - 1) / Fraction(254) ** (ndiag + 1)
            assert abs(Fraction(float(out[i, j])) - v) <= abs(v) * Fraction(2) ** -52 + top * Fraction(2) ** -60


@pytest.mark.parametrize("radix,dmax,ceil,nshift,p,h", [(32, 16, 0, -1, 12, 0x4D24ADD106258287),
                                                        (14, 7, 0, -1, 16, 0xF353DBD6B57F8B99)])
def test_scheme1_other_formats_reference_hash(orc, radix, dmax, ceil, nshift, p, h):
    """quick.csv:10 (I FP8, p = 12) and :14 (I BFP4, p = 16) at 128^3, uniform seed 7: digits within +-dmax,
    int32 sums S_d of the deferred reconstruction, all diagonals read whole (nsmall = p)."""
    n = 128
    a, b = orc.inputs(7, -1.0, n * n, n * n)
    A, B = a.reshape(n, n), b.reshape(n, n)
    dA, _ = orc.scale(A, n, n, 0, ceil, nshift)
    dB, _ = orc.scale(B, n, n, 1, ceil, nshift)
    sa = orc.oz1_slices(A, n, n, 0, dA, p, radix, dmax)
    sb = orc.oz1_slices(B, n, n, 1, dB, p, radix, dmax)
    Pd, _ = orc.oz1_gemm_diag(sa, sb, p)
    assert orc.hash(orc.oz1_recon(Pd, radix, 0, min((1 << 24) // (n * dmax * dmax), p), dA, dB)) == h


def test_fp8_reference_hash_from_exact_residues(orc):
    """quick.csv:11: II FP8 128^3, uniform seed 7, b = 54, one pass -> 20046e5bb3816cbb. The FP8 route's set
    at K = 128 (the library planner), residues of the exact product A'B' modulo those moduli, and the oracle's
    restatement of the reference reconstruction reproduce the reference's output: its digit split, products
    and composition deliver exactly the residue classes of A'B', which is what this build computes."""
    import oztt_amd as oz
    n, b, nd = 128, 54, 3
    a, bb = orc.inputs(7, -1.0, n * n, n * n)
    A, B = a.reshape(n, n), bb.reshape(n, n)
    fp8 = oz.choose_moduli_fp8(n, 14, b)
    ms = [fp8.rm[i] for i in range(fp8.rS)]
    assert fp8.ok and len(ms) == 12
    shift = b - 20 * (nd - 1)
    dA, _ = orc.scale(A, n, n, 0, 1, shift)
    dB, _ = orc.scale(B, n, n, 1, 1, shift)
    dgA = orc.digits(A, n, n, 0, dA, nd).reshape(n, n, nd).astype(np.int64)
    dgB = orc.digits(B, n, n, 1, dB, nd).reshape(n, n, nd).astype(np.int64)
    w = [1 << 40, 1 << 20, 1]
    Ap = [[sum(int(dgA[i, k, j]) * w[j] for j in range(nd)) for k in range(n)] for i in range(n)]
    Bp = [[sum(int(dgB[k, c, j]) * w[j] for j in range(nd)) for c in range(n)] for k in range(n)]
    C = np.zeros((len(ms), n, n), dtype=np.int32)
    for i in range(n):
        for c in range(n):
            v = sum(Ap[i][k] * Bp[k][c] for k in range(n))
            for s, m in enumerate(ms):
                r = v % m
                C[s, i, c] = r - m if r > m // 2 else r
    assert orc.hash(orc.crt_ref(C, n, n, ms, b, nd, 0, dA, dB)) == 0x20046E5BB3816CBB


def _fp8_quick_plan():
    import oztt_amd as oz
    n, b = 128, 54
    a, bb = oz.eval_inputs(7, -1.0, n * n, n * n)
    dd, gd, crt, tm = oz.plan2_fp8_device(a, bb, n, n, n, max_moduli=14, reconstruction=oz.Reconstruction.OnePass,
                                          fixed_bits=b)
    S = dd.mo.S
    ms = [int(crt.m[s]) for s in range(S)]
    qs = [int(dd.q[s]) for s in range(S)]
    xm = [int(dd.xmode[s]) for s in range(S)]
    return n, b, dd.mo.nd, a.reshape(n, n), bb.reshape(n, n), dd, gd, crt, tm, ms, qs, xm


def _sparse_split(r, q):
    """sparse_fix.h:12-18 in integer arithmetic: rounded digits, then the odd ones >= 17 moved by q."""
    num = 2 * r + (q if r >= 0 else -q)  # round half away from zero (q odd: no ties)
    h = (abs(num) // (2 * q)) * (1 if num >= 0 else -1)
    t = r - q * h
    if t % 2 and abs(t) >= 17:
        s = 1 if t > 0 else -1
        t -= s * q
        h += s
    if h % 2 and abs(h) >= 17:
        h -= (1 if h > 0 else -1) * q
    return t, h


def test_fp8_digit_planes_closed_forms(orc):
    """The FP8-route digits of every element (quick case: six sparse squares, five dense squares and a
    Karatsuba modulus) equal the closed forms of split.hpp:157-279 applied to a residue of A'."""
    n, b, nd, A, B, dd, gd, crt, tm, ms, qs, xm = _fp8_quick_plan()
    assert sorted(set(xm)) == [0, 1, 2]
    shift = b - 20 * (nd - 1)
    for X, mode in ((A, 0), (B, 1)):
        dl, _ = orc.scale(X, n, n, mode, 1, shift)
        pl = orc.digit_planes(X, n, n, mode, dl, nd, ms, qs, xm).astype(np.int64)
        dig = orc.digits(X, n, n, mode, dl, nd).reshape(n, n, nd).astype(np.int64)
        Ap = sum(dig[:, :, j] << (20 * (nd - 1 - j)) for j in range(nd))  # exact A' (|A'| < 2^55)
        p = 0
        for m, q, x in zip(ms, qs, xm):
            l, h = pl[p], pl[p + 1]
            r = l + (16 if x == 1 else q) * h
            assert np.all((r - Ap) % m == 0), m
            if x == 2:  # the sparse moves change l + q h by multiples of q^2 = m: back to |r| <= m/2 + 1
                r = (r + m // 2) % m - m // 2
            assert np.all(np.abs(r) <= m // 2 + 1), m
            if x == 1:  # Karatsuba: h = sgn(r) ceil(|r|/16), s = h + l, all within 16
                assert np.all(h == np.sign(r) * (-(-np.abs(r) // 16))) and np.all(pl[p + 2] == h + l)
                assert np.abs(pl[p:p + 3]).max() <= 16
                p += 3
                continue
            if x == 0:  # rounded: h = round-half-even(r/q), |l| <= q/2, digits within 16
                hh = np.rint(r / q).astype(np.int64)
                assert np.all(h == hh) and np.all(l == r - q * hh) and np.abs(pl[p:p + 2]).max() <= 16
            else:  # sparse square: the integer restatement, digits in the exact e4m3 integers
                # r is one of the representatives within m/2 + 1 (both ends exist only for +-(m+1)/2)
                for v, lv, hv in zip(r.ravel(), l.ravel(), h.ravel()):
                    cands = [int(v)] + ([int(v) - m] if abs(int(v) - m) <= m // 2 + 1 else [])
                    assert (int(lv), int(hv)) in [_sparse_split(c, q) for c in cands], (m, v, lv, hv)
                for d in (l, h):
                    a_ = np.abs(d)
                    assert np.all((a_ <= 16) | ((a_ <= 32) & (a_ % 2 == 0)))
            p += 2
        assert p == gd.nplanes


def test_fp8_reference_hash_from_digit_products(orc):
    """quick.csv:11 end to end through the digit path: oracle digit planes, the planned product outputs
    (int64), their CRT terms w_o = coef_o P_o mod m, k_s = sum of the terms of modulus s, the residue
    k_s y_s^-1 mod m_s, and the reference reconstruction give the reference's output hash."""
    n, b, nd, A, B, dd, gd, crt, tm, ms, qs, xm = _fp8_quick_plan()
    shift = b - 20 * (nd - 1)
    dA, _ = orc.scale(A, n, n, 0, 1, shift)
    dB, _ = orc.scale(B, n, n, 1, 1, shift)
    pa = orc.digit_planes(A, n, n, 0, dA, nd, ms, qs, xm)
    pb = orc.digit_planes(B, n, n, 1, dB, nd, ms, qs, xm)
    k = [np.zeros((n, n), dtype=np.int64) for _ in ms]
    for o in range(gd.nout):
        g = gd.g[o]
        P = sum(orc.gemm_i8(pa[g.a[t]], pb[g.b[t]])[0].astype(np.int64) for t in range(g.npairs))
        assert np.abs(P).max() <= g.bound and g.bound + g.m <= 2 ** 24
        s = tm[o]
        assert g.modulus == s and g.m == ms[s]
        k[s] = (k[s] + (g.coef * (P % g.m)) % g.m) % g.m
    C = np.zeros((len(ms), n, n), dtype=np.int32)
    for s, m in enumerate(ms):
        r = (k[s] * pow(int(crt.y[s]), -1, m)) % m
        C[s] = np.where(r > m // 2, r - m, r)
    assert orc.hash(orc.crt_ref(C, n, n, ms, b, nd, 0, dA, dB)) == 0x20046E5BB3816CBB


@pytest.mark.parametrize("radix,dmax", [(254, 127), (14, 7)])
def test_tf_mul_r_forms_agree_where_the_slicer_takes_twoproduct(orc, radix, dmax):
    """The GPU's Scheme I slicer multiplies by a general radix with tfMulR in its TwoProduct form
    (one multiply and one FMA per limb product) for waves whose elements meet its condition: every
    limb a multiple of 2^e with e >= -126, and |hi| r <= dmax + 1/2. Under that condition the digits
    equal those of Dekker's form (the reference's) over 24 planes, in the FP32 model with flush to
    zero, for elements near their row maximum and elements 50-100 binades below it."""
    import ctypes
    cov = ctypes.c_int64()
    n = 300000
    bad = orc.lib.orc_check_tf_mul_r_forms(0, n, 7, radix, dmax, 24, ctypes.byref(cov))
    assert bad == 0
    assert cov.value > n // 2


@pytest.mark.parametrize("radix,pmax", [(254, 11), (14, 23)])
def test_tf_mul_r_forms_agree_in_the_reconstruction(orc, radix, pmax):
    """The reconstruction's Horner values are integers, so no intermediate is subnormal; with p at
    most the bound the GPU applies (2^31 r^(p-1) r/(r-1) 4097 < 2^127: 11 diagonals for radix 254,
    23 for radix 14) the two forms of tfMulR give identical triples, int32 extremes included."""
    import ctypes
    cov = ctypes.c_int64()
    n = 200000
    bad = orc.lib.orc_check_tf_mul_r_forms(1, n, 9, radix, 0, pmax, ctypes.byref(cov))
    assert bad == 0 and cov.value == n


@pytest.mark.parametrize("radix,dmax", [(254, 127), (14, 7), (32, 16), (12, 6)])
def test_tf_mul_r_fast_form_agrees_and_its_order_holds(orc, radix, dmax):
    """The GPU's slicer also takes two of tfMulR's TwoSums as FastTwoSums (TwoProduct form): on the slicer
    chains it covers its digits equal Dekker's form, and the FastTwoSum order (|a| >= |b| or a = 0) holds
    at every call, so the substitution is exact there rather than merely lucky."""
    mode, planes = 0, 24
    import ctypes
    f = orc.lib.orc_check_tf_mul_r_fast
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                  ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]
    cov, viol = ctypes.c_int64(), ctypes.c_int64()
    n = 300000
    bad = f(mode, n, 13, radix, dmax, planes, ctypes.byref(cov), ctypes.byref(viol))
    assert bad == 0 and viol.value == 0
    assert cov.value > n // 2


def _pow2_fast(orc):
    import ctypes
    f = orc.lib.orc_check_tf_mul_pow2_fast
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                  ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]

    def run(mode, n, seed, radix, dmax, planes):
        cov, viol = ctypes.c_int64(), ctypes.c_int64()
        bad = f(mode, n, seed, radix, dmax, planes, ctypes.byref(cov), ctypes.byref(viol))
        return bad, cov.value, viol.value
    return run


@pytest.mark.parametrize("radix,dmax", [(64, 32), (2, 1), (1 << 20, 1 << 30)])
def test_tf_mul_pow2_fast_form_agrees_and_its_order_holds(orc, radix, dmax):
    """For a power-of-two radix the slicer takes both TwoSums of tfMulP2 as FastTwoSums: on the slicer
    chains of every element, near its row maximum or 50-100 binades below it (subnormal limbs
    included), the digits equal the reference form's and the FastTwoSum order holds at every call."""
    bad, cov, viol = _pow2_fast(orc)(0, 300000, 17, radix, dmax, 24)
    assert bad == 0 and viol == 0 and cov == 300000


@pytest.mark.parametrize("nd", [3, 4, 5])
def test_tf_mul_pow2_fast_form_agrees_on_scheme2_digit_chains(orc, nd):
    """Scheme II's digit extraction (digits.h:80-112: a digit Rnd(hi) without clamp, then tfMulP2 by 2^20
    before each further digit) also takes the FastTwoSum form on the GPU: for elements up to 2^24 after
    scaling and 50-100 binades below their row maximum, every exponent, the nd digits equal the
    reference form's and the order holds at every call."""
    bad, cov, viol = _pow2_fast(orc)(2, 300000, 19 + nd, 1 << 20, 0, nd - 1)
    assert bad == 0 and viol == 0 and cov == 300000


def test_tf_mul_pow2_fast_checker_counts_order_violations(orc):
    """The order count can fire: on the reconstruction's Horner chains (integers added between the
    multiplications) radix 64 leaves states where |mid| < |lo|, which is why only the slicer takes
    the fast form."""
    bad, cov, viol = _pow2_fast(orc)(1, 300000, 5, 64, 0, 12)
    assert viol > 0


def test_tf_mul_r_forms_checker_sees_overflow_beyond_the_bound(orc):
    """The check can fail: past the bound (radix 14 with up to 30 diagonals) Dekker's split
    overflows where the TwoProduct form does not, and the checker counts those chains."""
    import ctypes
    cov = ctypes.c_int64()
    bad = orc.lib.orc_check_tf_mul_r_forms(1, 100000, 9, 14, 0, 30, ctypes.byref(cov))
    assert bad > 0


def test_one_digit_planes_are_the_residues(orc):
    """Mode 3 (one digit, split.hpp:202-205): the single plane of a modulus of at most 33 is the symmetric
    residue of A' itself, within 16 in magnitude (exact in e4m3), next to the planes of other modes."""
    n, nd, b = 64, 3, 56
    a, _ = orc.inputs(4, 2.0, n * n, n * n)
    X = a.reshape(n, n)
    shift = b - 20 * (nd - 1)
    dl, _ = orc.scale(X, n, n, 0, 1, shift)
    ms, qs, xm = [32, 31, 29, 27, 25, 509, 23], [1, 1, 1, 1, 1, 16, 1], [3, 3, 3, 3, 3, 1, 3]
    pl = orc.digit_planes(X, n, n, 0, dl, nd, ms, qs, xm).astype(np.int64)
    res = orc.residues(X, n, n, 0, dl, nd, ms).astype(np.int64)
    assert pl.shape[0] == 6 + 3
    p = 0
    for s, (m, x) in enumerate(zip(ms, xm)):
        if x == 3:
            np.testing.assert_array_equal(pl[p], res[s])
            assert np.abs(pl[p]).max() <= 16
            p += 1
        else:
            np.testing.assert_array_equal((pl[p] + 16 * pl[p + 1] - res[s]) % m, 0)
            p += 3
