"""Scheme II with the operands' own CRT window, on the GPU, through the public call.

By default the plan computes with the smaller set that the operands' bound on |C'| allows (INT8
residues, or on the FP8 route a set of fewer e4m3 digit products). C must be bit for bit the C of the
set for the reference's window K 2^(2b) (the evaluation setting full_window) and the oracle's whole
chain with the reference's own set (moduli.hpp:338-344; the exact CRT makes C a function of b alone).
Info reports the reference's plan (under Transport.Int8Residues the moduli that computed); the
evaluation reports the products computed.
"""
import numpy as np
import pytest

import oztt_amd as oz
from tests.oracle_chains import oz2_chain

pytestmark = pytest.mark.gpu


def log(msg):
    print(f"[operand window] {msg}", flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


# (format, transport, M = N, K, seed, phi): the C3 distribution (a modulus saved), C4's (FP8 digit
# products saved; two INT8 moduli saved), uniform entries (a modulus saved at K = 1024), and entries of
# equal magnitude, whose bound lies within a bit of the window (phi None: nothing saved)
CASES = [
    ("INT8", "Automatic", 128, 8192, 3, 0.5),
    ("FP8", "Automatic", 64, 16384, 4, 2.0),
    ("FP8", "Int8Residues", 64, 16384, 4, 2.0),
    ("INT8", "Automatic", 64, 1024, 1, -1.0),
    ("INT8", "Automatic", 64, 1024, 1, None),
]


@pytest.mark.parametrize("fmt,tr,n,k,seed,phi", CASES, ids=[f"{c[0]}-{c[1]}-{c[3]}-{c[5]}" for c in CASES])
def test_operand_window_gives_the_full_window_c(ctx, oracle, fmt, tr, n, k, seed, phi):
    log(f"{fmt} {tr} {n}x{n}x{k} seed {seed} phi {phi}")
    a, b = oz.eval_inputs(seed, -1.0 if phi is None else phi, n * k, k * n)
    if phi is None:
        a, b = 0.75 * np.sign(a), 0.75 * np.sign(b)
    opts = oz.Options(scheme=oz.Scheme.II, format=oz.Format[fmt], transport=oz.Transport[tr])
    p = oz.plan2(a, b, n, n, k, oz.Format[fmt], transport=oz.Transport[tr])
    full = oz.plan2(a, b, n, n, k, oz.Format[fmt], transport=oz.Transport[tr], full_window=True)
    if phi is not None:
        assert p.S_window > 0 and p.nprod < full.nprod
    else:
        assert p.S_window == 0 and p.nprod == full.nprod
    c, info, ev = ctx.evaluate(a, b, n, n, k, opts, warmup=1, repeats=2)
    cf, infof, evf = ctx.evaluate(a, b, n, n, k, opts, warmup=1, repeats=2, full_window=True)
    log(f"products {ev.partial_products} (full window {evf.partial_products}), Info moduli {info.moduli}")
    assert ev.whole_checked and evf.whole_checked
    assert (ev.partial_products, evf.partial_products) == (p.nprod, full.nprod)
    assert (info.integer_bits, info.reconstruction_passes) == (infof.integer_bits, infof.reconstruction_passes)
    # Info: the reference's plan under Transport.Automatic, the moduli that computed under Int8Residues
    if tr == "Automatic":
        assert info.moduli == infof.moduli == p.rS
    else:
        assert (info.moduli, infof.moduli) == (p.S, full.S)
    np.testing.assert_array_equal(c.view(np.uint64), cf.view(np.uint64))
    # the plain call (no evaluation hooks) computes with the smaller set too
    c2 = np.empty(n * n)
    ctx.gemm(a, b, c2, n, n, k, opts)
    np.testing.assert_array_equal(c2.view(np.uint64), c.view(np.uint64))
    # the oracle's whole chain with the reference's set for its window (the route's moduli, up to 4096
    # on the FP8 route)
    want = oz2_chain(oracle, a.reshape(n, k), b.reshape(k, n), [p.rm[i] for i in range(p.rS)], p.b, p.nd)
    np.testing.assert_array_equal(c.reshape(n, n).view(np.uint64), want.view(np.uint64))


def test_resident_calls_keep_the_operand_window(ctx):
    """A resident pair plans once (with the operands' window) and reuses that plan: repeated calls give
    the host call's C."""
    n, k = 128, 8192
    a, b = oz.eval_inputs(3, 0.5, n * k, k * n)
    opts = oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8)
    c = np.empty(n * n)
    ctx.gemm(a, b, c, n, n, k, opts)
    ra, rb = ctx.upload(a, n, k), ctx.upload(b, k, n)
    try:
        for i in range(2):
            cr = np.empty(n * n)
            ev = oz.EvalStats()
            ctx.gemm_resident(ra, rb, cr, opts, evaluation=ev)
            assert ev.plan_reused == (i == 1)
            assert ev.partial_products == oz.plan2(a, b, n, n, k, oz.Format.INT8).S
            np.testing.assert_array_equal(cr.view(np.uint64), c.view(np.uint64))
    finally:
        ra.close()
        rb.close()


@pytest.mark.parametrize("fmt,phi,k", [("INT8", 0.5, 8192), ("INT8", 2.0, 8192), ("FP8", 2.0, 16384)])
def test_tight_bound_near_the_smaller_modulus(ctx, oracle, fmt, phi, k):
    """Rows of A and columns of B parallel up to signs (tests/test_operand_window.py parallel_operands):
    max |C'| reaches the operands' bound, which for INT8 at phi 0.5 lies within 1/8 bit of M/2 of the 15
    moduli that compute (16 for the window); on the FP8 route at K = 16384 the set of fewest products
    (one-digit moduli, sparse digits) computes. The public call, the full-window call and the oracle's
    chain with the reference's own set agree bit for bit."""
    from tests.test_operand_window import parallel_operands
    A, B = parallel_operands(phi, K=k)
    n = A.shape[0]
    log(f"parallel rows and columns, {fmt}, phi {phi}, K {k}")
    a, b = A.ravel(), B.ravel()
    opts = oz.Options(scheme=oz.Scheme.II, format=oz.Format[fmt])
    p = oz.plan2(a, b, n, n, k, oz.Format[fmt])
    full = oz.plan2(a, b, n, n, k, oz.Format[fmt], full_window=True)
    assert p.S_window == p.rS and p.nprod < full.nprod
    c, info, ev = ctx.evaluate(a, b, n, n, k, opts, warmup=1, repeats=2)
    cf, _, evf = ctx.evaluate(a, b, n, n, k, opts, warmup=1, repeats=2, full_window=True)
    assert ev.whole_checked and evf.whole_checked
    assert (ev.partial_products, evf.partial_products) == (p.nprod, full.nprod)
    np.testing.assert_array_equal(c.view(np.uint64), cf.view(np.uint64))
    want = oz2_chain(oracle, A, B, [p.rm[i] for i in range(p.rS)], p.b, p.nd)
    np.testing.assert_array_equal(c.reshape(n, n).view(np.uint64), want.view(np.uint64))
