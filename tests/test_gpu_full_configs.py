"""C4 and C5 at their full BASELINE shapes, through the public call, on the GPU.

The oracle cannot run these shapes whole, so each test checks what does not depend on the size:
* C4 (Scheme II FP8, m = n = k = 16384, phi 2): the library's default, the FP8 route's e4m3 digits
  on the FP8 matrix cores (42 digit products for the operands' own window, 45 for the reference's),
  and `Transport.Int8Residues` (the same plan on INT8 residues, other kernels, other moduli) give the
  same C bit for bit over the whole matrix: both are the exact CRT of the same integer product A'B'
  (reference ozaki2.cpp:228-318 and :333-350);
* C5 (Scheme I BF16 format, 8 slices, m = n = 8192, k = 65536, phi 4, rows i % 100 == 0 of A and
  columns j % 100 == 0 of B zero): those rows and columns of C are zero;
* in both, a 16 x 16 block of C whose rows and columns cross 256-tile boundaries (and, for C5, hold a
  zero row and column) equals the oracle's whole chain on those rows of A and columns of B: row and
  column deltas depend only on their own row or column, so the block's chain is the chain of the
  slabs, with the plan (width, moduli, slices) of the full problem.

The inputs follow the evaluation generator's distribution, (U(0,1) - 1/2) exp(phi N(0,1)), drawn with
numpy's generator: the reference's sequential mt19937 stream takes about 90 s per billion values on
the host, and these properties hold for any inputs.
"""
import numpy as np
import pytest

import oztt_amd as oz
from tests.oracle_chains import oz1_chain, oz2_chain

pytestmark = pytest.mark.gpu


def log(msg):
    print(f"[full configs] {msg}", flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


def synth(seed: int, phi: float, size: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    out = np.empty(size)
    step = 1 << 26
    for i in range(0, size, step):
        j = min(size, i + step)
        out[i:j] = (rng.random(j - i) - 0.5) * np.exp(phi * rng.standard_normal(j - i))
    return out


def test_c4_full_size_transports_agree_and_block_parity(ctx, oracle):
    n = 16384
    log("C4: inputs")
    a, b = synth(41, 2.0, n * n), synth(42, 2.0, n * n)
    log("C4: FP8 route on the FP8 matrix cores (default)")
    c8 = np.empty(n * n)
    i8 = ctx.gemm(a, b, c8, n, n, n, oz.Options(scheme=oz.Scheme.II, format=oz.Format.FP8))
    log("C4: the same plan on INT8 residues")
    ci = np.empty(n * n)
    ii = ctx.gemm(a, b, ci, n, n, n, oz.Options(scheme=oz.Scheme.II, format=oz.Format.FP8,
                                                transport=oz.Transport.Int8Residues))
    log(f"C4: FP8 route {i8.moduli} moduli, INT8 residues {ii.moduli} moduli, b = {i8.integer_bits}")
    assert (i8.integer_bits, i8.reconstruction_passes) == (ii.integer_bits, ii.reconstruction_passes)
    np.testing.assert_array_equal(c8.view(np.uint64), ci.view(np.uint64))
    del ci
    log("C4: plans")
    pr = oz.plan2(a, b, n, n, n, oz.Format.FP8)
    assert pr.fp8_digits and (pr.rS, pr.b) == (i8.moduli, i8.integer_bits)
    p = oz.plan2(a, b, n, n, n, oz.Format.FP8, transport=oz.Transport.Int8Residues)
    assert not p.fp8_digits and (p.S, p.b) == (ii.moduli, ii.integer_bits)
    log("C4: oracle chain on a 16 x 16 block")
    A, B = a.reshape(n, n), b.reshape(n, n)
    r0, c0 = 8184, 4088  # rows 8184..8199 and columns 4088..4103 cross the tiles at 8192 and 4096
    As, Bs = np.ascontiguousarray(A[r0:r0 + 16]), np.ascontiguousarray(B[:, c0:c0 + 16])
    got = np.ascontiguousarray(c8.reshape(n, n)[r0:r0 + 16, c0:c0 + 16])
    # with the INT8 set that computed under Int8Residues and with the FP8 route's own set for the window
    # K 2^(2b) (both calls computed with smaller sets, which the operands' bound on |C'| allows)
    assert p.S_window > p.S and pr.S_window == pr.rS and pr.nprod < pr.rnprod
    for ms in ([p.m[i] for i in range(p.S)], [pr.rm[i] for i in range(pr.rS)]):
        want = oz2_chain(oracle, As, Bs, ms, p.b, p.nd)
        np.testing.assert_array_equal(got.view(np.uint64), want.view(np.uint64))


def test_c5_full_size_zero_lines_and_block_parity(ctx, oracle):
    m = n = 8192
    k = 65536
    log("C5: inputs")
    a, b = synth(51, 4.0, m * k), synth(52, 4.0, k * n)
    A, B = a.reshape(m, k), b.reshape(k, n)
    A[::100, :] = 0.0
    B[:, ::100] = 0.0
    log("C5: public call")
    c = np.empty(m * n)
    info = ctx.gemm(a, b, c, m, n, k, oz.Options(scheme=oz.Scheme.I, format=oz.Format.BF16, slices=8))
    assert (info.format, info.slices) == (oz.Format.BF16, 8)
    C = c.reshape(m, n)
    assert not C[::100, :].any() and not C[:, ::100].any()
    log("C5: plan")
    pl = oz.plan1(a, b, m, n, k, slices=8, fmt=oz.Format.BF16)
    assert (pl.p, pl.pairwise, pl.defer, pl.nsmall) == (8, 1, 1, 0)
    log("C5: oracle chain on a 16 x 16 block")
    r0, c0 = 4090, 6390  # across the tiles at 4096 and 6400, with row 4100 and column 6400 zero
    want = oz1_chain(oracle, np.ascontiguousarray(A[r0:r0 + 16]), np.ascontiguousarray(B[:, c0:c0 + 16]), 8,
                     "BF16", nsmall=pl.nsmall)
    got = np.ascontiguousarray(C[r0:r0 + 16, c0:c0 + 16])
    np.testing.assert_array_equal(got.view(np.uint64), want.view(np.uint64))
