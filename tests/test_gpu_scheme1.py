"""Scheme I INT8 on the GPU, through the C ABI and the public API.

1. Stages against the oracle, bit-exact: digit planes (radix 254 and 64, OZ_BLOCK layouts 2 and 3),
   the int32 diagonal products, and the Horner reconstruction (both input encodings).
2. The whole call reproduces the reference's published outputs bit for bit: the I-INT8 128^3 hash
   (tools/validated/quick.csv:12) and the 4096^3 output hashes of the phi sweep
   (experiments/paper_logs/accuracy_logs/phi_sweep.log, CONFIG chash, seed 7), with the slice
   count given and chosen automatically.
3. C2 itself (4096^3, seed 2, phi 1, automatic p): slices and int32 diagonal products bit-exact
   against the oracle, C within the error model against binary128.
"""
import numpy as np
import pytest

import oztt_amd as oz
from oztt_amd.device import Oz1ReconDesc, from_blocks, to_blocks

pytestmark = pytest.mark.gpu

I_INT8 = oz.Options(scheme=oz.Scheme.I, format=oz.Format.INT8)


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


def edge_rows(rows, cols, rng):
    X = rng.uniform(-1, 1, (rows, cols)) * np.exp2(rng.integers(-40, 40, (rows, 1)))
    X[0] = 0.0
    X[1, :] = 0.25
    X[1, 3] = -0.5                                   # exact power-of-two maximum
    X[2, 5] = 1.0 + 2.0 ** -40                        # dropped bits below the BF16 significand
    X[3, :] = rng.uniform(-1, 1, cols) * 2.0 ** -60   # wide range inside one row
    X[3, 0] = 1.0
    X[4, 1] = 1e-300                                  # an element far below its row maximum
    return X


@pytest.mark.parametrize("layout", [2, 3])
@pytest.mark.parametrize("radix,dmax,ceil,p", [(254, 127, 1, 8), (254, 127, 1, 13), (64, 32, 0, 10)])
def test_slices_match_oracle(dev, oracle, layout, radix, dmax, ceil, p):
    rng = np.random.default_rng(radix + p + layout)
    tran = layout == 3
    rows, cols = (200, 96) if tran else (96, 200)
    X = edge_rows(cols, rows, rng).T.copy() if tran else edge_rows(rows, cols, rng)
    mode = 1 if tran else 0
    delta, fl = oracle.scale(X, rows, cols, mode, ceil, -1)
    want = oracle.oz1_slices(X, rows, cols, mode, delta, p, radix, dmax)  # [p][rows][cols]
    prow = ((cols if tran else rows) + 15) // 16 * 16 + 16
    pld = ((rows if tran else cols) + 63) // 64 * 64 + 64
    pstride = prow * pld + 1024
    bx, bd = dev.upload(X), dev.upload(delta)
    bp = dev.alloc(p * pstride)
    dev.oz1_split(bx, rows, cols, cols, mode, bd, p, radix, dmax, bp, layout, prow, pld, pstride)
    got = from_blocks(dev.download(bp, np.int8, p * pstride).reshape(p, pstride)[:, :prow * pld], prow, pld)
    if tran:
        np.testing.assert_array_equal(got[:, :cols, :rows], want.transpose(0, 2, 1))
        assert not got[:, cols:, :].any() and not got[:, :, rows:].any()
    else:
        np.testing.assert_array_equal(got[:, :rows, :cols], want)
        assert not got[:, rows:, :].any() and not got[:, :, cols:].any()


@pytest.mark.parametrize("radix,dmax", [(254, 127), (64, 32)])
def test_slices_near_the_subnormal_range(dev, oracle, radix, dmax):
    """Digits of elements whose last significand bit sits just above and just below 2^-126 after
    scaling (row maxima near 1/2, elements near 2^-73): deep planes reach them. For radix 254 a wave
    takes the TwoProduct form of tfMulR only when all its elements' limbs are normal, Dekker's
    otherwise; radix 64 takes tfMulP2 with FastTwoSums everywhere (limbs flushed to zero included);
    the digits equal the oracle's either way."""
    rng = np.random.default_rng(21)
    rows, cols = 64, 256
    p = 16 if radix == 254 else 20
    # |x| in [2^-k-1, 2^-k): the last bit weighs 2^(-k-53); rows 0-31 (two bands of blocks) keep
    # k <= 73, so every limb is normal there, rows 32-63 straddle the boundary
    k = np.where(np.arange(rows)[:, None] < 32, rng.integers(66, 74, (rows, cols)), rng.integers(70, 81, (rows, cols)))
    X = rng.choice([-1.0, 1.0], (rows, cols)) * rng.uniform(0.5, 1.0, (rows, cols)) * np.exp2(-k.astype(np.float64))
    X[:, 0] = 0.5
    X[40::3, 1] = 1e-300  # far below every normal limb
    delta, _ = oracle.scale(X, rows, cols, 0, 1, -1)
    assert not delta.any()
    want = oracle.oz1_slices(X, rows, cols, 0, delta, p, radix, dmax)
    assert np.count_nonzero(want[p // 2:, :32]) > 32 * cols  # the deep planes reach the small elements
    prow, pld = rows, cols
    bx, bd = dev.upload(X), dev.upload(delta)
    bp = dev.alloc(p * prow * pld)
    dev.oz1_split(bx, rows, cols, cols, 0, bd, p, radix, dmax, bp, 2, prow, pld, prow * pld)
    got = from_blocks(dev.download(bp, np.int8, p * prow * pld).reshape(p, -1), prow, pld)
    for x in (bx, bd, bp):
        x.free()
    dev.bufs.clear()
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("M,N,K,p,radix,dmax", [(300, 520, 700, 8, 254, 127), (17, 5, 33, 10, 64, 32),
                                                (256, 256, 64, 13, 14, 7)])
def test_split_pair_equals_single_splits(dev, oracle, M, N, K, p, radix, dmax):
    """oz1_split_pair_int8 writes exactly the planes of oz1_split_int8 on A (layout 2) and B (layout 3),
    padding zeros included, and they equal the oracle's slices."""
    rng = np.random.default_rng(M + K + p)
    A = edge_rows(M, K, rng) if M > 5 else rng.uniform(-1, 1, (M, K))
    B = rng.uniform(-1, 1, (K, N)) * np.exp2(rng.integers(-30, 30, (1, N)))
    dA, _ = oracle.scale(A, M, K, 0, 1, -1)
    dB, _ = oracle.scale(B, K, N, 1, 1, -1)
    Mg, Ng, Kg = -(-M // 16) * 16 + 16, -(-N // 16) * 16, -(-K // 64) * 64 + 64
    bA, bB, bdA, bdB = dev.upload(A), dev.upload(B), dev.upload(dA), dev.upload(dB)
    pA, pB = dev.alloc(p * Mg * Kg), dev.alloc(p * Ng * Kg)
    qA, qB = dev.alloc(p * Mg * Kg), dev.alloc(p * Ng * Kg)
    dev.fill_u32(pA, 0x5A5A5A5A, p * Mg * Kg // 4)
    dev.fill_u32(pB, 0x5A5A5A5A, p * Ng * Kg // 4)
    dev.oz1_split_pair(bA, M, K, K, bdA, bB, N, N, bdB, p, radix, dmax, pA, pB, Mg, Ng, Kg)
    dev.oz1_split(bA, M, K, K, 0, bdA, p, radix, dmax, qA, 2, Mg, Kg, Mg * Kg)
    dev.oz1_split(bB, K, N, N, 1, bdB, p, radix, dmax, qB, 3, Ng, Kg, Ng * Kg)
    got = [dev.download(x, np.int8, p * r * Kg) for x, r in ((pA, Mg), (pB, Ng), (qA, Mg), (qB, Ng))]
    for x in (bA, bB, bdA, bdB, pA, pB, qA, qB):
        x.free()
    dev.bufs.clear()
    np.testing.assert_array_equal(got[0], got[2])
    np.testing.assert_array_equal(got[1], got[3])
    pa = from_blocks(got[0].reshape(p, -1), Mg, Kg)
    pb = from_blocks(got[1].reshape(p, -1), Ng, Kg)
    np.testing.assert_array_equal(pa[:, :M, :K], oracle.oz1_slices(A, M, K, 0, dA, p, radix, dmax))
    np.testing.assert_array_equal(pb[:, :N, :K], oracle.oz1_slices(B, K, N, 1, dB, p, radix, dmax).transpose(0, 2, 1))
    assert not pa[:, M:, :].any() and not pa[:, :, K:].any() and not pb[:, N:, :].any() and not pb[:, :, K:].any()


@pytest.mark.parametrize("M,N,K,p", [(256, 512, 192, 8), (512, 256, 1024, 13), (256, 256, 64, 1)])
def test_diagonal_products_exact(dev, M, N, K, p):
    """P_d = sum_{i<=d} A_i B_{d-i}^T with all d+1 pairs in one exact int32 accumulation; the all-127 rows
    reach the largest sums of the last diagonal."""
    rng = np.random.default_rng(M + K + p)
    A = rng.integers(-127, 128, (p, M, K), dtype=np.int8)
    Bt = rng.integers(-127, 128, (p, N, K), dtype=np.int8)
    A[:, 0, :] = 127
    Bt[:, 0, :] = 127
    A[:, 1, :] = -127
    bA, bB = dev.upload(to_blocks(A)), dev.upload(to_blocks(Bt))
    bC = dev.alloc(4 * p * M * N)
    dev.oz1_gemm_diag(bA, bB, bC, M, N, K, p, N, M * K, N * K, M * N)
    C = dev.download(bC, np.int32, p * M * N).reshape(p, M, N)
    Af, Bf = A.astype(np.float64), Bt.astype(np.float64)
    for d in range(p):
        want = sum(Af[i] @ Bf[d - i].T for i in range(d + 1))  # exact: |sum| < 2^53
        np.testing.assert_array_equal(C[d].astype(np.int64), want.astype(np.int64))


def test_diagonal_products_reject_overflow(dev):
    b = dev.alloc(1 << 20)
    with pytest.raises(RuntimeError):
        dev.oz1_gemm_diag(b, b, b, 256, 256, 16384, 9, 256, 256 * 16384, 256 * 16384, 256 * 256)  # 9*K*127^2 > 2^31


@pytest.mark.parametrize("radix,signmag,nsingle,ndiag", [(254, 1, 0, 8), (254, 1, 0, 13), (64, 0, 0, 8),
                                                         (64, 0, 5, 10)])
def test_recon_matches_oracle(dev, oracle, radix, signmag, nsingle, ndiag):
    """Partial sums up to the largest magnitude the planner admits: |S| < 2^116 (the FP32 exponent budget of
    the Horner evaluation, format.hpp:160-171), i.e. |P_d| < 2^(116 - (ndiag-1) log2 radix), and int32."""
    rng = np.random.default_rng(radix * ndiag + nsingle)
    M, N = 5, 777
    top = min(2 ** 31 - 1, int(2.0 ** (116 - (ndiag - 1) * np.log2(radix) - 1)))
    Pd = rng.integers(-top, top, (ndiag, M, N)).astype(np.int32)
    Pd[:nsingle] = rng.integers(-(2 ** 24), 2 ** 24, (nsingle, M, N))
    Pd[nsingle:, 0, :5] = [0, 1, -1, top, -top]
    Pd[:, 1, :] = 0
    Pd[1:, 2, :] = 0                                   # only the leading diagonal
    dA = rng.integers(-10, 40, M).astype(np.int32)
    dB = rng.integers(-10, 40, N).astype(np.int32)
    whi, wlo, qw = oracle.oz1_scale_w(radix, ndiag - 1)
    desc = Oz1ReconDesc(ndiag, radix, signmag, nsingle, whi, wlo, qw)
    ldp = N + 3
    Pp = np.zeros((ndiag, M, ldp), dtype=np.int32)
    Pp[:, :, :N] = Pd
    bP, bA, bB = dev.upload(Pp), dev.upload(dA), dev.upload(dB)
    bo = dev.alloc(8 * M * N)
    dev.oz1_recon(bP, M, N, ldp, M * ldp, desc, bA, bB, bo, N)
    got = dev.download(bo, np.float64, M * N)
    want = oracle.oz1_recon(Pd, radix, signmag, nsingle, dA, dB)
    np.testing.assert_array_equal(got.view(np.uint64), want.view(np.uint64))


def test_reference_hash_int8_128(ctx):
    """quick.csv:12: I INT8 128^3, uniform seed 7, p = 8 -> 6c9693442bfc11b0, from the GPU directly."""
    n = 128
    a, b = oz.eval_inputs(7, -1.0, n * n, n * n)
    c = np.empty(n * n)
    info = ctx.gemm(a, b, c, n, n, n, oz.Options(scheme=oz.Scheme.I, format=oz.Format.INT8, slices=8))
    assert (info.scheme, info.slices) == (oz.Scheme.I, 8)
    assert oz.eval_hash(c) == 0x6C9693442BFC11B0


# tools/validated/quick.csv, scheme I at 128^3, uniform seed 7 (format, slices, output hash): the four radix-64
# formats share the hash (lines 2, 4, 6, 8), FP8 line 10, BFP4 line 14, BFP2 line 16.
QUICK_I = [(oz.Format.BF16, 10, 0xBE6558FA9F435FA0), (oz.Format.FP16, 10, 0xBE6558FA9F435FA0),
           (oz.Format.TF32, 10, 0xBE6558FA9F435FA0), (oz.Format.BFP8, 10, 0xBE6558FA9F435FA0),
           (oz.Format.FP8, 12, 0x4D24ADD106258287), (oz.Format.BFP4, 16, 0xF353DBD6B57F8B99),
           (oz.Format.BFP2, 59, 0x13CD8E69EDCA2911)]


@pytest.mark.parametrize("fmt,slices,h", QUICK_I)
def test_reference_hashes_other_formats_128(ctx, fmt, slices, h):
    n = 128
    a, b = oz.eval_inputs(7, -1.0, n * n, n * n)
    c = np.empty(n * n)
    info = ctx.gemm(a, b, c, n, n, n, oz.Options(scheme=oz.Scheme.I, format=fmt, slices=slices))
    assert (info.format, info.slices) == (fmt, slices)
    assert oz.eval_hash(c) == h


# phi_sweep.log CONFIG lines of I-INT8 at 4096^3, seed 7: (phi, slices option, p used, chash)
PHI_HASHES = [(0.0, 8, 8, 0x2D5687AE78334480), (0.0, 0, 7, 0x16D398E7A7E7AB7E), (16.0, 0, 11, 0x53768BF42D24E8DE),
              (2.0, 8, 8, 0xB94DEA61BA62020B)]


@pytest.mark.parametrize("phi,slices,p,h", PHI_HASHES)
def test_reference_hashes_4096(ctx, phi, slices, p, h):
    n = 4096
    a, b = oz.eval_inputs(7, phi, n * n, n * n)
    c = np.empty(n * n)
    info = ctx.gemm(a, b, c, n, n, n, oz.Options(scheme=oz.Scheme.I, format=oz.Format.INT8, slices=slices))
    assert info.slices == p
    assert oz.eval_hash(c) == h


def test_c2_bit_exact_chain(ctx, dev, oracle):
    """BASELINE C2: 4096^3, seed 2, phi 1, automatic p. The slice planes of both operands and the int32
    diagonal products on a 64-row slab equal the oracle's; C is within the error model (binary128 sample)."""
    n = 4096
    a, b = oz.eval_inputs(2, 1.0, n * n, n * n)
    A, B = a.reshape(n, n), b.reshape(n, n)
    pl = oz.plan1(a, b, n, n, n)
    p = pl.p
    c = np.empty(n * n)
    info = ctx.gemm(a, b, c, n, n, n, I_INT8)
    assert info.slices == p
    # stages through the C ABI with the same p
    dA, _ = oracle.scale(A, n, n, 0, 1, -1)
    dB, _ = oracle.scale(B, n, n, 1, 1, -1)
    sa = oracle.oz1_slices(A, n, n, 0, dA, p, 254, 127)
    sb = oracle.oz1_slices(B, n, n, 1, dB, p, 254, 127)
    bA, bB, bdA, bdB = dev.upload(A), dev.upload(B), dev.upload(dA), dev.upload(dB)
    pA, pB = dev.alloc(p * n * n), dev.alloc(p * n * n)
    dev.oz1_split(bA, n, n, n, 0, bdA, p, 254, 127, pA, 2, n, n, n * n)
    dev.oz1_split(bB, n, n, n, 1, bdB, p, 254, 127, pB, 3, n, n, n * n)
    gA = from_blocks(dev.download(pA, np.int8, p * n * n).reshape(p, -1), n, n)
    np.testing.assert_array_equal(gA, sa)
    gB = from_blocks(dev.download(pB, np.int8, p * n * n).reshape(p, -1), n, n)
    np.testing.assert_array_equal(gB, sb.transpose(0, 2, 1))
    del gA, gB
    bP = dev.alloc(4 * p * n * n)
    dev.oz1_gemm_diag(pA, pB, bP, n, n, n, p, n, n * n, n * n, n * n)
    P = dev.download(bP, np.int32, p * n * n).reshape(p, n, n)
    rows = slice(1000, 1064)
    for d in range(p):
        want = sum(sa[i, rows].astype(np.float64) @ sb[d - i].astype(np.float64) for i in range(d + 1))
        np.testing.assert_array_equal(P[d, rows].astype(np.int64), want.astype(np.int64))
    for buf in (bA, bB, bdA, bdB, pA, pB, bP):
        buf.free()
    dev.bufs.clear()
    # accuracy on a sample against binary128, next to the FP64 error bound gamma_K |A||B|
    rng = np.random.default_rng(0)
    rs, cs = rng.choice(n, 48, replace=False), rng.choice(n, 48, replace=False)
    r_, c_ = np.repeat(rs, 48).astype(np.int32), np.tile(cs, 48).astype(np.int32)
    q = oz.eval_quad_sample(a, b, n, n, n, r_, c_)
    got = c.reshape(n, n)[r_, c_]
    absab = np.einsum("ij,ij->i", np.abs(A[r_]), np.abs(B[:, c_].T))
    assert np.all(np.abs(got - q) <= n * 2.0 ** -53 * absab)


def test_c5_shape_bit_exact(ctx, oracle):
    """The C5 class (BF16 format, 8 slices, k = 65536, seed 5, phi 4, rows i%100 == 0 of A and columns
    j%100 == 0 of B zero) at m = n = 512: the whole output of a row slab equals the oracle's chain (radix-64
    slices, exact int32 diagonal sums S_d, deferred reconstruction with no diagonal read whole)."""
    m = n = 512
    k = 65536
    a, b = oz.eval_inputs(5, 4.0, m * k, k * n)
    A, B = a.reshape(m, k), b.reshape(k, n)
    A[::100, :] = 0.0
    B[:, ::100] = 0.0
    c = np.empty(m * n)
    info = ctx.gemm(a, b, c, m, n, k, oz.Options(scheme=oz.Scheme.I, format=oz.Format.BF16, slices=8))
    assert (info.format, info.slices) == (oz.Format.BF16, 8)
    pl = oz.plan1(a, b, m, n, k, slices=8, fmt=oz.Format.BF16)
    assert (pl.pairwise, pl.defer, pl.nsmall) == (1, 1, 0)
    rows = slice(0, 64)
    dA, _ = oracle.scale(A, m, k, 0, 0, -1)
    dB, _ = oracle.scale(B, k, n, 1, 0, -1)
    sa = oracle.oz1_slices(np.ascontiguousarray(A[rows]), 64, k, 0, dA[rows], 8, 64, 32)
    sb = oracle.oz1_slices(B, k, n, 1, dB, 8, 64, 32)
    Pd = np.empty((8, 64, n), dtype=np.int32)
    for d in range(8):
        s = sum(sa[i].astype(np.float64) @ sb[d - i].astype(np.float64) for i in range(d + 1))  # exact: < 2^53
        Pd[d] = s.astype(np.int64)
    want = oracle.oz1_recon(Pd, 64, 0, 0, dA[rows], dB)
    np.testing.assert_array_equal(c.reshape(m, n)[rows].reshape(-1).view(np.uint64), want.view(np.uint64))
    assert not c.reshape(m, n)[::100, :].any() and not c.reshape(m, n)[:, ::100].any()


def _block_chain(oracle, A, B, rows, dA, dB, p, radix, dmax, Kc):
    """The oracle's block-by-block chain on the rows `rows` of C: slices, exact per-block diagonal sums,
    reconstruction with the limbs carried from block to block."""
    m, k = A.shape
    n = B.shape[1]
    sa = oracle.oz1_slices(np.ascontiguousarray(A[rows]), A[rows].shape[0], k, 0, dA[rows], p, radix, dmax)
    sb = oracle.oz1_slices(B, k, n, 1, dB, p, radix, dmax)
    nkb = k // Kc
    Pb = np.empty((nkb, p, sa.shape[1], n), dtype=np.int32)
    for kb in range(nkb):
        ks = slice(kb * Kc, (kb + 1) * Kc)
        ga = [sa[i][:, ks].astype(np.float64) for i in range(p)]
        gb = [sb[i][ks].astype(np.float64) for i in range(p)]
        for d in range(p):
            Pb[kb, d] = sum(ga[i] @ gb[d - i] for i in range(d + 1)).astype(np.int64)  # exact: < 2^24
    return oracle.oz1_recon_blocks(Pb, radix, dA[rows], dB)


@pytest.mark.parametrize("fmt,p,radix,dmax", [(oz.Format.BF16, 8, 64, 32), (oz.Format.FP8, 6, 32, 16)])
def test_block_reconstruction_forced_bit_exact(ctx, oracle, fmt, p, radix, dmax):
    """The reconstruction K block by K block (reference plan.hpp:104-109, recon_tf_f32in.cpp), forced with
    the evaluation hook force_kc at a size the oracle runs whole: C equals the oracle's block chain bit for
    bit, and differs from the one-block (deferred) reconstruction by at most one unit in the last place."""
    m, n, k, Kc = 256, 320, 2048, 512
    a, b = oz.eval_inputs(13, 2.0, m * k, k * n)
    A, B = a.reshape(m, k), b.reshape(k, n)
    opts = oz.Options(scheme=oz.Scheme.I, format=fmt, slices=p)
    c_blk, info, ev = ctx.evaluate(a, b, m, n, k, opts, force_kc=Kc)
    assert info.slices == p and ev.gemm_launches == k // Kc
    dA, _ = oracle.scale(A, m, k, 0, 0, -1)
    dB, _ = oracle.scale(B, k, n, 1, 0, -1)
    want = _block_chain(oracle, A, B, slice(0, m), dA, dB, p, radix, dmax, Kc)
    np.testing.assert_array_equal(c_blk.view(np.uint64), want.view(np.uint64))
    c_one = ctx.multiply(a, b, m, n, k, opts)
    ulp = np.abs(np.spacing(np.maximum(np.abs(c_one), np.abs(c_blk))))
    assert np.all(np.abs(c_blk - c_one) <= ulp)


def test_block_reconstruction_natural(ctx, oracle):
    """BF16 with 16 slices and k = 2^18: (L+1) k dmax^2 exceeds int32, so the plan reconstructs in K blocks
    of 1024 (the reference's recon_limbs plan, which this build runs instead of rejecting). Two rows of C
    equal the oracle's block chain bit for bit; a sample is within the FP64 error bound of binary128."""
    m = n = 64
    k = 1 << 18
    a, b = oz.eval_inputs(17, 0.5, m * k, k * n)
    A, B = a.reshape(m, k), b.reshape(k, n)
    opts = oz.Options(scheme=oz.Scheme.I, format=oz.Format.BF16, slices=16)
    pl = oz.plan1(a, b, m, n, k, slices=16, fmt=oz.Format.BF16)
    assert pl.defer == 0 and pl.nkb > 1
    c = np.empty(m * n)
    info = ctx.gemm(a, b, c, m, n, k, opts)
    assert info.slices == 16
    dA, _ = oracle.scale(A, m, k, 0, 0, -1)
    dB, _ = oracle.scale(B, k, n, 1, 0, -1)
    rows = slice(5, 7)
    want = _block_chain(oracle, A, B, rows, dA, dB, 16, 64, 32, pl.Kc)
    np.testing.assert_array_equal(c.reshape(m, n)[rows].reshape(-1).view(np.uint64), want.view(np.uint64))
    rng = np.random.default_rng(1)
    r_ = rng.integers(0, m, 32).astype(np.int32)
    c_ = rng.integers(0, n, 32).astype(np.int32)
    q = oz.eval_quad_sample(a, b, m, n, k, r_, c_)
    absab = np.einsum("ij,ij->i", np.abs(A[r_]), np.abs(B[:, c_].T))
    assert np.all(np.abs(c.reshape(m, n)[r_, c_] - q) <= k * 2.0 ** -53 * absab)
