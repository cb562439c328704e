"""Scheme II with the FP8 format on the GPU: e4m3 digit planes, digit products on the FP8 matrix
cores, composition in the product epilogue, exact CRT.

1. Stage parity against the oracle (reference modslice_digit.cpp / compose.cpp restated): the digit
   planes are bit-exact (decoded e4m3 values), every product output equals the int64 sum of its
   digit products, every uint16 term is coef * P mod m (a representative in [0, m]); the reference's published FP8 output hash
   (quick.csv:11, 20046e5bb3816cbb) follows from the GPU terms through the oracle's restatement of
   the reference reconstruction.
2. The public API: FP8 runs the e4m3 digits on the FP8 matrix cores by default and INT8 residues at
   the FP8 plan's width with Transport.Int8Residues. Both outputs are bit-identical to the INT8 output
   at the same width b (all reconstruct the exact C' = A'B'); Info reports the FP8 route by default
   and the INT8 moduli that computed otherwise; accuracy on the C4 generator.
"""
import numpy as np
import pytest

import oztt_amd as oz
from oztt_amd.device import E4M3, from_blocks
from tests.oracle_chains import oz2_chain
from tests.oracle_lib import assert_residues


pytestmark = pytest.mark.gpu


def log(msg):
    print(f"[fp8] {msg}", flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


def opts(fmt, **kw):
    o = oz.Options(scheme=oz.Scheme.II, format=fmt)
    for key, v in kw.items():
        setattr(o, key, v)
    return o


def test_fp8_quick_case_matches_int8_bits(ctx):
    """quick.csv:11 / :13 settings: 128^3, uniform seed 7, b = 54, one pass; S_req 14 (FP8), 16 (INT8)."""
    n = 128
    a, b = oz.eval_inputs(7, -1.0, n * n, n * n)
    one = oz.Reconstruction.OnePass
    o8 = opts(oz.Format.FP8, max_moduli=14, reconstruction=one)
    c8, i8, _ = ctx.evaluate(a, b, n, n, n, o8, fixed_bits=54)
    cr, ir, _ = ctx.evaluate(a, b, n, n, n, opts(oz.Format.FP8, max_moduli=14, reconstruction=one,
                                                  transport=oz.Transport.Int8Residues), fixed_bits=54)
    ci, ii, _ = ctx.evaluate(a, b, n, n, n, opts(oz.Format.INT8, max_moduli=16, reconstruction=one), fixed_bits=54)
    assert i8.format == oz.Format.FP8 and i8.moduli == 12 and i8.integer_bits == 54
    assert (ir.format, ir.integer_bits, ir.reconstruction_passes) == (oz.Format.FP8, 54, 1) and ir.moduli >= 15
    assert ii.moduli == 15 and ii.integer_bits == 54
    np.testing.assert_array_equal(c8.view(np.uint64), ci.view(np.uint64))
    np.testing.assert_array_equal(cr.view(np.uint64), ci.view(np.uint64))


@pytest.mark.parametrize("n", [1024, 2048])
def test_fp8_wide_range_auto(ctx, oracle, n):
    """C4 generator (seed 4, phi 2) at reduced size: automatic b, FP8 route moduli, accuracy; the e4m3
    digits on the FP8 matrix cores (the default) and INT8 residues (Transport.Int8Residues) give the same
    bits."""
    a, b = oz.eval_inputs(4, 2.0, n * n, n * n)
    p = oz.plan2(a, b, n, n, n, oz.Format.FP8)
    assert p.fp8_digits
    c = np.empty(n * n)
    info = ctx.gemm(a, b, c, n, n, n, opts(oz.Format.FP8))
    assert info.format == oz.Format.FP8 and info.moduli == p.rS and info.integer_bits == p.b
    assert info.reconstruction_passes == (2 if p.two_pass else 1)
    q = oz.plan2(a, b, n, n, n, oz.Format.FP8, transport=oz.Transport.Int8Residues)
    cf = np.empty(n * n)
    inf = ctx.gemm(a, b, cf, n, n, n, opts(oz.Format.FP8, transport=oz.Transport.Int8Residues))
    assert not q.fp8_digits and inf.moduli == q.S and inf.integer_bits == info.integer_bits
    np.testing.assert_array_equal(c.view(np.uint64), cf.view(np.uint64))
    ci = np.empty(n * n)
    ii = ctx.gemm(a, b, ci, n, n, n, opts(oz.Format.INT8))
    if ii.integer_bits == info.integer_bits:
        np.testing.assert_array_equal(c.view(np.uint64), ci.view(np.uint64))
    rs = np.random.default_rng(0).integers(0, n, 256)
    cs = np.random.default_rng(1).integers(0, n, 256)
    q = oracle.quad_sample(a, b, n, n, n, rs, cs)
    got = c.reshape(n, n)[rs, cs]
    absab = (np.abs(a.reshape(n, n)[rs]) * np.abs(b.reshape(n, n)[:, cs].T)).sum(axis=1)
    assert np.all(np.abs(got - q) <= absab * n * 2.0 ** -53)


def run_fp8_stages(dev, a, b, n, max_moduli=0, fixed_bits=0, one_pass=True, m=None, k=None, execution_set=False):
    """scale -> digit planes -> product outputs (int32 and uint16 terms) -> CRT on the GPU, for
    A (m x k) and B (k x n) (m = k = n unless given)."""
    m = n if m is None else m
    k = n if k is None else k
    rec = oz.Reconstruction.OnePass if one_pass else oz.Reconstruction.Automatic
    dd, gd, crt, tm = oz.plan2_fp8_device(a, b, m, n, k, max_moduli=max_moduli, reconstruction=rec,
                                          fixed_bits=fixed_bits, execution_set=execution_set)
    nd, b_ = dd.mo.nd, crt.b
    shift = b_ - 20 * (nd - 1)
    Mg, Ng = -(-m // 256) * 256, -(-n // 256) * 256
    Kg = -(-k // 64) * 64
    P, O = gd.nplanes, gd.nout
    bA, bB = dev.upload(a), dev.upload(b)
    bdA, bdB, bfl = dev.alloc(4 * m), dev.alloc(4 * n), dev.alloc(8)
    dev.fill_u32(bfl, 0, 2)
    dev.scale(bA, m, k, k, 0, 1, shift, bdA, bfl, 0)
    dev.scale(bB, k, n, n, 1, 1, shift, bdB, bfl, 1)
    pA, pB = dev.alloc(P * Mg * Kg), dev.alloc(P * Ng * Kg)
    dev.split_digits(bA, m, k, k, 0, bdA, dd, pA, 2, Mg, Kg, Mg * Kg)
    dev.split_digits(bB, k, n, n, 1, bdB, dd, pB, 3, Ng, Kg, Ng * Kg)
    bP = dev.alloc(4 * O * Mg * Ng)
    dev.gemm_groups_f8(pA, pB, bP, Mg, Ng, Kg, gd, 0, Ng, Mg * Kg, Ng * Kg, Mg * Ng)
    bW = dev.alloc(2 * O * Mg * Ng)
    dev.gemm_groups_f8(pA, pB, bW, Mg, Ng, Kg, gd, 1, Ng, Mg * Kg, Ng * Kg, Mg * Ng)
    bo = dev.alloc(8 * m * n)
    dev.crt_terms(bW, m, n, Ng, Mg * Ng, O, tm, crt, bdA, bdB, bo, n)
    r = dict(dd=dd, gd=gd, crt=crt, tm=tm, nd=nd, b=b_, shape=(m, n, k),
             dA=dev.download(bdA, np.int32, m), dB=dev.download(bdB, np.int32, n),
             flags=dev.download(bfl, np.uint32, 2),
             planesA=E4M3[from_blocks(dev.download(pA, np.uint8, P * Mg * Kg).reshape(P, -1), Mg, Kg)[:, :m, :k]],
             planesB=E4M3[from_blocks(dev.download(pB, np.uint8, P * Ng * Kg).reshape(P, -1), Ng, Kg)[:, :n, :k]],
             P=dev.download(bP, np.int32, O * Mg * Ng).reshape(O, Mg, Ng)[:, :m, :n],
             W=dev.download(bW, np.uint16, O * Mg * Ng).reshape(O, Mg, Ng)[:, :m, :n],
             out=dev.download(bo, np.float64, m * n))
    for buf in (bA, bB, bdA, bdB, bfl, pA, pB, bP, bW, bo):
        buf.free()
    dev.bufs.clear()
    return r


def check_fp8_chain(oracle, r, a, b, n):
    """Every stage of run_fp8_stages against the oracle; returns the composed residues (S, m, n)."""
    dd, gd, crt, tm, nd, b_ = r["dd"], r["gd"], r["crt"], r["tm"], r["nd"], r["b"]
    m_, n, kk = r["shape"]
    S = dd.mo.S
    ms = [int(crt.m[s]) for s in range(S)]
    qs = [int(dd.q[s]) for s in range(S)]
    xm = [int(dd.xmode[s]) for s in range(S)]
    A, B = a.reshape(m_, kk), b.reshape(kk, n)
    shift = b_ - 20 * (nd - 1)
    dA, fA = oracle.scale(A, m_, kk, 0, 1, shift)
    dB, fB = oracle.scale(B, kk, n, 1, 1, shift)
    np.testing.assert_array_equal(r["dA"], dA)
    np.testing.assert_array_equal(r["dB"], dB)
    assert fA == fB == 0 and not r["flags"].any()
    pa = oracle.digit_planes(A, m_, kk, 0, dA, nd, ms, qs, xm)
    pb = oracle.digit_planes(B, kk, n, 1, dB, nd, ms, qs, xm)
    np.testing.assert_array_equal(r["planesA"], pa.astype(np.float64))
    np.testing.assert_array_equal(r["planesB"], pb.transpose(0, 2, 1).astype(np.float64))
    k = [np.zeros((m_, n), dtype=np.int64) for _ in ms]
    for o in range(gd.nout):
        g = gd.g[o]
        P = sum(oracle.gemm_i8(pa[g.a[t]], pb[g.b[t]])[0].astype(np.int64) for t in range(g.npairs))
        np.testing.assert_array_equal(r["P"][o].astype(np.int64), P)
        w = (g.coef * (P % g.m)) % g.m
        assert_residues(r["W"][o], w, g.m, f"output {o}")
        k[tm[o]] = (k[tm[o]] + w) % g.m
    C = np.zeros((S, m_, n), dtype=np.int32)
    for s, m in enumerate(ms):
        res = (k[s] * pow(int(crt.y[s]), -1, m)) % m
        C[s] = np.where(res > m // 2, res - m, res)
    ex = oracle.crt_exact(C, m_, n, ms, b_, nd, dA, dB)
    np.testing.assert_array_equal(r["out"].view(np.uint64), ex.view(np.uint64))
    return C, ms, dA, dB


@pytest.mark.parametrize("m,n,k,encoding", [(300, 200, 700, 1), (64, 520, 130, 1), (17, 5, 33, 0)])
def test_split_digits_pair_equals_single_splits(dev, m, n, k, encoding):
    """oz2_split_digits_pair writes exactly the planes of oz2_split_digits on A (layout 2) and B
    (layout 3), padding zeros included, for both encodings."""
    a, b = oz.eval_inputs(9, 2.0, m * k, k * n)
    dd, gd, crt, tm = oz.plan2_fp8_device(a, b, m, n, k)
    dd.encoding = encoding
    nd, b_ = dd.mo.nd, crt.b
    shift = b_ - 20 * (nd - 1)
    Mg, Ng, Kg = -(-m // 16) * 16 + 16, -(-n // 16) * 16, -(-k // 64) * 64 + 64
    P = gd.nplanes
    bA, bB = dev.upload(a), dev.upload(b)
    bdA, bdB, bfl = dev.alloc(4 * m), dev.alloc(4 * n), dev.alloc(8)
    dev.fill_u32(bfl, 0, 2)
    dev.scale(bA, m, k, k, 0, 1, shift, bdA, bfl, 0)
    dev.scale(bB, k, n, n, 1, 1, shift, bdB, bfl, 1)
    pA, pB, qA, qB = (dev.alloc(P * r * Kg) for r in (Mg, Ng, Mg, Ng))
    dev.fill_u32(pA, 0x5A5A5A5A, P * Mg * Kg // 4)
    dev.fill_u32(pB, 0x5A5A5A5A, P * Ng * Kg // 4)
    dev.split_digits_pair(bA, m, k, k, bdA, bB, n, n, bdB, dd, pA, pB, Mg, Ng, Kg)
    dev.split_digits(bA, m, k, k, 0, bdA, dd, qA, 2, Mg, Kg, Mg * Kg)
    dev.split_digits(bB, k, n, n, 1, bdB, dd, qB, 3, Ng, Kg, Ng * Kg)
    got = [dev.download(x, np.uint8, P * r * Kg) for x, r in ((pA, Mg), (pB, Ng), (qA, Mg), (qB, Ng))]
    for x in (bA, bB, bdA, bdB, bfl, pA, pB, qA, qB):
        x.free()
    dev.bufs.clear()
    np.testing.assert_array_equal(got[0], got[2])
    np.testing.assert_array_equal(got[1], got[3])
    assert got[0].any() and got[1].any()


@pytest.mark.parametrize("k,phi", [(16384, 2.0), (4096, 0.5)])
def test_fp8_stages_fewest_products_set(dev, oracle, k, phi):
    """The FP8 set the public call computes with (the operands' window, fewest digit products): moduli
    of at most 33 carried as one digit (the residue itself, one plane and one product) next to the
    route's squares, Karatsuba and (K = 4096) sparse squares; every stage equals the oracle, and C the
    oracle's chain with the route's own set."""
    m = n = 64
    a, b = oz.eval_inputs(4, phi, m * k, k * n)
    p = oz.plan2(a, b, m, n, k, oz.Format.FP8)
    r = run_fp8_stages(dev, a, b, n, one_pass=False, m=m, k=k, execution_set=True)
    S = r["dd"].mo.S
    xm = [int(r["dd"].xmode[s]) for s in range(S)]
    log(f"K {k}: {S} moduli, modes {xm}, {p.nprod} products against the route's {p.rnprod}")
    assert S == p.S and 3 in xm and p.nprod < p.rnprod
    assert all(int(r["crt"].m[s]) <= 33 for s in range(S) if xm[s] == 3)
    check_fp8_chain(oracle, r, a, b, n)
    want = oz2_chain(oracle, a.reshape(m, k), b.reshape(k, n), [p.rm[i] for i in range(p.rS)], p.b, p.nd)
    np.testing.assert_array_equal(r["out"].reshape(m, n).view(np.uint64), want.view(np.uint64))


def test_fp8_stages_quick_case_reference_hash(dev, oracle):
    """quick.csv:11: II FP8 128^3, uniform seed 7, b = 54, 14 moduli requested, one pass."""
    n = 128
    a, b = oz.eval_inputs(7, -1.0, n * n, n * n)
    r = run_fp8_stages(dev, a, b, n, max_moduli=14, fixed_bits=54)
    assert r["dd"].mo.S == 12 and r["b"] == 54 and sorted(set(r["dd"].xmode[s] for s in range(12))) == [0, 1, 2]
    C, ms, dA, dB = check_fp8_chain(oracle, r, a, b, n)
    assert oracle.hash(oracle.crt_ref(C, n, n, ms, 54, r["nd"], 0, dA, dB)) == 0x20046E5BB3816CBB


@pytest.mark.parametrize("n,seed,phi,fixed", [(1024, 4, 2.0, 60), (256, 4, 2.0, 0), (320, 9, 1.0, 0)])
def test_fp8_stages_bit_exact(dev, oracle, n, seed, phi, fixed):
    """C4 generator; b = 60 at K = 1024 brings a wide (non-square, 4-product) modulus, 803."""
    a, b = oz.eval_inputs(seed, phi, n * n, n * n)
    r = run_fp8_stages(dev, a, b, n, fixed_bits=fixed, one_pass=False)
    if fixed == 60:
        assert 803 in [r["crt"].m[s] for s in range(r["dd"].mo.S)]
        assert any(r["gd"].g[o].m == 803 for o in range(r["gd"].nout))
    check_fp8_chain(oracle, r, a, b, n)


def test_fp8_gemm_rejects_inexact_bound(dev):
    """An output bound above 2^24 (the next float, 2^24 + 2) is refused before any launch; 2^24 itself
    is exact (test_fp8_products_exact_at_2_24)."""
    _, gd, _, _ = oz.plan2_fp8_device(*oz.eval_inputs(7, -1.0, 64 * 64, 64 * 64), 64, 64, 64)
    gd.g[0].bound = 2.0 ** 24 + 2.0
    A = dev.alloc(gd.nplanes * 256 * 64)
    P = dev.alloc(4 * gd.nout * 256 * 256)
    with pytest.raises(RuntimeError, match="exact FP32"):
        dev.gemm_groups_f8(A, A, P, 256, 256, 64, gd, 0, 256, 256 * 64, 256 * 64, 256 * 256)
    A.free()
    P.free()
    dev.bufs.clear()


@pytest.mark.parametrize("fmt", [oz.Format.BFP8, oz.Format.BF16, oz.Format.FP16, oz.Format.TF32, oz.Format.BFP4,
                                 oz.Format.BFP2, oz.Format.FP8])
def test_other_formats_run_int8_residues(ctx, oracle, fmt):
    """Scheme II with BF16, FP16, TF32, BFP8, BFP4, BFP2 and FP8: the format's own route plans (Info reports
    its moduli, width and passes, as the reference's), INT8 residues at that width compute (FP8: its own
    e4m3 digits), so the output is bit-identical to Format::INT8 at the same width, and to the oracle's
    whole chain at the route's width b with the route's own moduli (up to 4096; residues, exact products
    and the exact CRT on the CPU from the FP64 inputs)."""
    n = 256
    a, b = oz.eval_inputs(5, 1.0, n * n, n * n)
    p = oz.plan2(a, b, n, n, n, fmt, transport=oz.Transport.Int8Residues)
    c = np.empty(n * n)
    info = ctx.gemm(a, b, c, n, n, n, opts(fmt))  # FP8: its own digits
    assert info.format == fmt and info.scheme == oz.Scheme.II
    assert (info.moduli, info.integer_bits, info.reconstruction_passes) == (p.rS, p.b, 2 if p.two_pass else 1)
    ci, ii, ev = ctx.evaluate(a, b, n, n, n, opts(oz.Format.INT8, max_moduli=24), fixed_bits=info.integer_bits)
    assert ii.integer_bits == info.integer_bits and ev.partial_products == p.S
    np.testing.assert_array_equal(c.view(np.uint64), ci.view(np.uint64))
    rm = [p.rm[i] for i in range(p.rS)]
    want = oz2_chain(oracle, a.reshape(n, n), b.reshape(n, n), rm, p.b, p.nd).reshape(-1)
    np.testing.assert_array_equal(c.view(np.uint64), want.view(np.uint64))


def test_digit_route_beyond_the_int8_width_on_fp8_digits(ctx, oracle):
    """BFP8 at a fixed width of 90 bits at K = 4096, beyond the 85 that 24 INT8 moduli hold: the call keeps
    b = 90 (five digits of A') on the FP8 route's e4m3 digits, Info reports BFP8's route (17 moduli), and C
    equals the oracle's chain at b = 90 with BFP8's own moduli."""
    m = n = 64
    k = 4096
    a, b = oz.eval_inputs(4, 2.0, m * k, k * n)
    p = oz.plan2(a, b, m, n, k, oz.Format.BFP8, fixed_bits=90, max_moduli=24)
    assert p.fp8_digits and p.b == 90 and p.nd == 5
    c, info, ev = ctx.evaluate(a, b, m, n, k, opts(oz.Format.BFP8, max_moduli=24), fixed_bits=90)
    assert (info.moduli, info.integer_bits) == (17, 90)
    rm = [p.rm[i] for i in range(p.rS)]
    want = oz2_chain(oracle, a.reshape(m, k), b.reshape(k, n), rm, 90, 5).reshape(-1)
    np.testing.assert_array_equal(c.view(np.uint64), want.view(np.uint64))


def test_default_options_run(ctx):
    """Options{} (Scheme II, BFP8, automatic) works as the reference's default."""
    n = 128
    a, b = oz.eval_inputs(7, -1.0, n * n, n * n)
    c = ctx.multiply(a, b, n, n, n, oz.Options())
    R = a.reshape(n, n).astype(np.longdouble) @ b.reshape(n, n).astype(np.longdouble)
    err = float(np.sqrt(np.sum((c.reshape(n, n) - R) ** 2) / np.sum(R ** 2)))
    assert err <= 8 * np.finfo(float).eps
