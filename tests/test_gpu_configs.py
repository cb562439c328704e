"""The BASELINE configurations whose own plans need their full shapes, on the GPU.

C3 (the headline): Scheme II INT8, m = n = k = 8192, the evaluation generator with seed 3 and
phi 0.5, automatic moduli, two passes forced. The planner's choice (b = 56, two passes, 17 moduli
for the reference's window K 2^(2b), of which the operands' own bound on |C'| needs 16) runs through
the public API and, stage by stage, through the production kernels of the C ABI (scale, OZ_BLOCK
residue split, products reduced to CRT digits in the GEMM epilogue, CRT from the digits). On a
64-row slab that crosses a tile boundary, every stage is checked against the oracle: the exponent
deltas, the residue planes of A, all residue planes of B, the epilogue digits (the exact products
mod m_s times y_s, from float64 products of the oracle's residues, which are exact below 2^53), and
C (the oracle's exact CRT of the same products, and its whole chain with the reference's 17 moduli);
the public call gives the same bits as the staged chain for the whole matrix; a binary128 sample lies
within the FP64 bound k 2^-53 |A||B|. (Reference ozaki2.cpp:439-478; BASELINE.json configs[2].)

C4's K: Scheme II FP8 at k = 16384 (seed 4, phi 2) with m = n = 256. At this K the reference's
planner cannot use its sparse e4m3 digits (K 32^2 + m > 2^24) and falls back to dense digits with
moduli up to 33^2 = 1089 (moduli.hpp:724-731). The plan is asserted to be that route, and every
stage (digit planes, each output's digit products, its uint16 CRT term, C) is checked against the
oracle.

The FP8 product at its exactness bound: outputs that sum three products of K = 16384 digits +-16
reach 3 K 16^2 = 12582912, just below 2^24, where FP32 accumulation is still exact
(split.hpp:676-688; the reference's probe experiments/paper_logs/measure_logs/probe_gemm_exact.log);
and single products of sparse digits up to 32 reach 2^24 itself, which FP32 still holds.
"""
import numpy as np
import pytest

import oztt_amd as oz
from oztt_amd.device import E4M3, GroupsDesc, crt_desc, from_blocks, moduli_desc, to_blocks
from tests.oracle_lib import assert_residues
from tests.oracle_chains import oz2_chain
from tests.test_gpu_scheme2_fp8 import check_fp8_chain, run_fp8_stages

pytestmark = pytest.mark.gpu


def log(msg):
    print(f"[configs] {msg}", flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


def test_c3_headline_plan_and_slab_parity(ctx, dev, oracle):
    n, seed, phi = 8192, 3, 0.5
    r0, rows = 3000, 64  # the slab: rows 3000..3063, across the tile boundary at row 3072
    log("C3: inputs")
    a, b = oz.eval_inputs(seed, phi, n * n, n * n)
    A, B = a.reshape(n, n), b.reshape(n, n)
    two = oz.Reconstruction.TwoPass
    p = oz.plan2(a, b, n, n, n, oz.Format.INT8, reconstruction=two)
    moduli = [p.m[i] for i in range(p.S)]
    S, bw, nd = p.S, p.b, p.nd
    # the reference's plan: 17 moduli for the window K 2^(2b); the operands' own bound on |C'| needs 16
    assert (p.rS, p.S_window, S, bw, nd, p.two_pass) == (17, 17, 16, 56, 3, 1)
    log("C3: public call")
    c = np.empty(n * n)
    info = ctx.gemm(a, b, c, n, n, n, oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8, reconstruction=two))
    assert (info.moduli, info.integer_bits, info.reconstruction_passes) == (17, 56, 2)

    log("C3: staged production kernels")
    shift = bw - 20 * (nd - 1)
    Kg = n
    bA, bB = dev.upload(a), dev.upload(b)
    bdA, bdB, bfl = dev.alloc(4 * n), dev.alloc(4 * n), dev.alloc(8)
    dev.fill_u32(bfl, 0, 2)
    dev.scale(bA, n, n, n, 0, 1, shift, bdA, bfl, 0)
    dev.scale(bB, n, n, n, 1, 1, shift, bdB, bfl, 1)
    md, cd = moduli_desc(moduli, nd), crt_desc(moduli, bw, nd)
    plane = n * Kg
    pA, pB = dev.alloc(S * plane), dev.alloc(S * plane)
    dev.split_int8(bA, n, n, n, 0, bdA, md, pA, 2, n, Kg, plane)
    dev.split_int8(bB, n, n, n, 1, bdB, md, pB, 3, n, Kg, plane)
    bD = dev.alloc(S * n * n)
    dev.gemm_digits(pA, pB, bD, n, n, Kg, S, n, plane, plane, n * n, cd)
    bo = dev.alloc(8 * n * n)
    dev.crt_digits(bD, n, n, n, n * n, cd, bdA, bdB, bo, n)
    out = dev.download(bo, np.float64, n * n)
    np.testing.assert_array_equal(c.view(np.uint64), out.view(np.uint64))
    dA, dB = dev.download(bdA, np.int32, n), dev.download(bdB, np.int32, n)
    assert not dev.download(bfl, np.uint32, 2).any()
    # A's planes of the slab's 16-row bands, B's planes whole (OZ_BLOCK tiles, Kg/64 blocks per band)
    band0, band1 = r0 // 16, (r0 + rows + 15) // 16
    band_bytes = (Kg // 64) * 1024
    gA = np.stack([from_blocks(dev.download(pA, np.int8, (band1 - band0) * band_bytes,
                                            s * plane + band0 * band_bytes), 16 * (band1 - band0), Kg)
                   for s in range(S)])[:, r0 - 16 * band0:r0 - 16 * band0 + rows]
    gB = from_blocks(dev.download(pB, np.int8, S * plane).reshape(S, -1), n, Kg)  # (S, N, K)
    gD = np.stack([dev.download(bD, np.uint8, rows * n, s * n * n + r0 * n).reshape(rows, n) for s in range(S)])
    for buf in (bA, bB, bdA, bdB, bfl, pA, pB, bD, bo):
        buf.free()
    dev.bufs.clear()

    log("C3: oracle")
    wA, fA = oracle.scale(A, n, n, 0, 1, shift)
    wB, fB = oracle.scale(B, n, n, 1, 1, shift)
    np.testing.assert_array_equal(dA, wA)
    np.testing.assert_array_equal(dB, wB)
    assert fA == fB == 0
    want_A = oracle.residues(A[r0:r0 + rows], rows, n, 0, wA[r0:r0 + rows], nd, moduli)  # (S, rows, K)
    np.testing.assert_array_equal(gA, want_A)
    want_B = oracle.residues(B, n, n, 1, wB, nd, moduli)  # (S, K, N)
    for s in range(S):
        np.testing.assert_array_equal(gB[s], want_B[s].T)
    del gB
    Cs = np.empty((S, rows, n), dtype=np.int32)
    for s, m in enumerate(moduli):
        # |C_s| <= 8192 * 127^2 < 2^27: the float64 product is the exact integer
        prod = want_A[s].astype(np.float64) @ want_B[s].astype(np.float64)
        Cs[s] = prod.astype(np.int64)
        assert_residues(gD[s], (prod.astype(np.int64) % m) * int(cd.y[s]), m, f"modulus {m}")
    ex = oracle.crt_exact(Cs, rows, n, moduli, bw, nd, wA[r0:r0 + rows], wB)
    np.testing.assert_array_equal(c.reshape(n, n)[r0:r0 + rows].ravel().view(np.uint64), ex.view(np.uint64))
    log("C3: oracle chain with the reference's 17 moduli")
    full = oz2_chain(oracle, np.ascontiguousarray(A[r0:r0 + rows]), B, [p.rm[i] for i in range(p.rS)], bw, nd)
    np.testing.assert_array_equal(c.reshape(n, n)[r0:r0 + rows].view(np.uint64), full.view(np.uint64))

    log("C3: binary128 sample")
    rng = np.random.default_rng(3)
    rs, cs = rng.integers(0, n, 512), rng.integers(0, n, 512)
    q = oracle.quad_sample(a, b, n, n, n, rs, cs)
    got = c.reshape(n, n)[rs, cs]
    absab = np.einsum("ij,ij->i", np.abs(A[rs]), np.abs(B[:, cs].T))
    assert np.all(np.abs(got - q) <= absab * n * 2.0 ** -53)
    assert np.max(np.abs(got - q) / np.abs(q)) < 1e-12


def test_c4_inner_dimension_dense_fp8_route(dev, oracle):
    m = n = 256
    k = 16384
    a, b = oz.eval_inputs(4, 2.0, m * k, k * n)
    p = oz.plan2(a, b, m, n, k, oz.Format.FP8)
    # the dense-digit fallback: no sparse squares, every modulus at most 33^2
    route = [p.rm[i] for i in range(p.rS)]
    assert p.rsparse == 0 and max(route) <= 1089 and 1089 in route
    assert all(p.rmode[i] != 2 for i in range(p.rS))
    log(f"C4 K: {p.rS} moduli, b={p.b}, {p.rnprod} products, {p.rnout} outputs")
    r = run_fp8_stages(dev, a, b, n, one_pass=False, m=m, k=k)
    assert r["dd"].mo.S == p.rS and r["b"] == p.b
    assert all(r["dd"].xmode[s] != 2 for s in range(p.rS))
    # the concatenated outputs reach 2 K 16^2 = 2^23, half the FP32 limit
    bounds = [r["gd"].g[o].bound for o in range(r["gd"].nout)]
    assert max(bounds) < 2.0 ** 24 and max(bounds) >= 2.0 ** 23
    check_fp8_chain(oracle, r, a, b, n)


def test_c4_inner_dimension_public_call_equals_int8(ctx):
    """The public FP8 call on C4's inner dimension, by default on the FP8 matrix cores (dense-digit route,
    both operands split in one launch) and with Transport.Int8Residues (INT8 residues at the FP8 plan's
    width), gives C bit for bit equal to the INT8 format at the same width, with the same plan both ways
    (Info: the FP8 route's moduli by default, the INT8 moduli that computed otherwise) and checked
    whole-pass replays."""
    m = n = 256
    k = 16384
    a, b = oz.eval_inputs(4, 2.0, m * k, k * n)
    o8 = oz.Options(scheme=oz.Scheme.II, format=oz.Format.FP8)
    c8, info8, ev8 = ctx.evaluate(a, b, m, n, k, o8, warmup=0, repeats=1)
    assert ev8.whole_checked
    od = oz.Options(scheme=oz.Scheme.II, format=oz.Format.FP8, transport=oz.Transport.Int8Residues)
    cd, infod, evd = ctx.evaluate(a, b, m, n, k, od, warmup=0, repeats=1)
    assert evd.whole_checked
    assert (infod.integer_bits, infod.reconstruction_passes) == (info8.integer_bits, info8.reconstruction_passes)
    # products per pass: the FP8 route's digit products, or one per INT8 modulus
    oi = oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8, max_moduli=24)
    ci, infoi, evi = ctx.evaluate(a, b, m, n, k, oi, fixed_bits=info8.integer_bits)
    assert infoi.integer_bits == info8.integer_bits and evd.partial_products == evi.partial_products == infod.moduli
    # the operands' own window: fewer FP8 digit products than the route's, fewer INT8 moduli than the window's
    p = oz.plan2(a, b, m, n, k, oz.Format.FP8)
    assert ev8.partial_products == p.nprod < p.rnprod and info8.moduli == p.rS
    assert infoi.moduli > infod.moduli
    log(f"C4 K: FP8 {info8.moduli} moduli ({ev8.partial_products} digit products), INT8 {infoi.moduli} moduli, "
        f"b={info8.integer_bits}")
    np.testing.assert_array_equal(c8.view(np.uint64), ci.view(np.uint64))
    np.testing.assert_array_equal(cd.view(np.uint64), ci.view(np.uint64))


def test_fp8_products_exact_at_the_fp32_bound(dev):
    """Digit planes of +-16 (e4m3 0x58 / 0xD8), K = 16384, outputs of three concatenated products:
    all-positive digits give 3 K 256 = 12582912 < 2^24 exactly; random signs give every smaller sum.
    Compared with int64 products, as int32 outputs and as uint16 terms coef * P mod m (representatives in [0, m])."""
    M = N = 256
    K = 16384
    code = {16: int(np.flatnonzero(E4M3 == 16.0)[0]), -16: int(np.flatnonzero(E4M3 == -16.0)[0])}
    rng = np.random.default_rng(11)
    planes = 6
    sa = np.ones((planes, M, K), dtype=np.int64) * 16
    sb = np.ones((planes, N, K), dtype=np.int64) * 16
    sa[3:] *= rng.choice([-1, 1], size=(3, M, K))
    sb[3:] *= rng.choice([-1, 1], size=(3, N, K))
    enc = lambda v: np.where(v > 0, code[16], code[-16]).astype(np.uint8)
    bA = dev.upload(to_blocks(enc(sa)).ravel())
    bB = dev.upload(to_blocks(enc(sb)).ravel())
    gd = GroupsDesc()
    gd.nout, gd.nplanes = 2, planes
    for o, first in enumerate((0, 3)):
        g = gd.g[o]
        g.npairs, g.modulus, g.m, g.coef = 3, o, 1089, 5 + o
        for t in range(3):
            g.a[t] = g.b[t] = first + t
        g.bound = 3.0 * K * 16 * 16
    assert gd.g[0].bound == 12582912.0 < 2.0 ** 24
    bP, bW = dev.alloc(4 * 2 * M * N), dev.alloc(2 * 2 * M * N)
    dev.gemm_groups_f8(bA, bB, bP, M, N, K, gd, 0, N, M * K, N * K, M * N)
    dev.gemm_groups_f8(bA, bB, bW, M, N, K, gd, 1, N, M * K, N * K, M * N)
    P = dev.download(bP, np.int32, 2 * M * N).reshape(2, M, N).astype(np.int64)
    W = dev.download(bW, np.uint16, 2 * M * N).reshape(2, M, N).astype(np.int64)
    for buf in (bA, bB, bP, bW):
        buf.free()
    dev.bufs.clear()
    assert np.all(P[0] == 12582912)
    want = sum(sa[3 + t].astype(np.float64) @ sb[3 + t].astype(np.float64).T for t in range(3)).astype(np.int64)
    np.testing.assert_array_equal(P[1], want)
    for o in range(2):
        assert_residues(W[o], (5 + o) * (P[o] % 1089), 1089, f"output {o}")


def test_fp8_products_exact_at_2_24(dev):
    """Sparse e4m3 digits (|d| <= 16, and even up to 32) at K = 16384, one product per output: digits
    of 32 (e4m3 0x60) reach K 32^2 = 2^24 exactly, the largest integer up to which FP32 holds every
    integer; random sparse digits with random signs give every smaller sum. The FP8 set of fewest
    products uses such outputs at C4's K, whose epilogue reduces them in FP64."""
    M = N = 256
    K = 16384
    sparse = np.array([v for v in range(0, 33) if v <= 16 or v % 2 == 0], dtype=np.int64)
    code = {int(v): int(np.flatnonzero(E4M3 == float(v))[0]) for v in np.concatenate([sparse, -sparse])}
    rng = np.random.default_rng(12)
    sa = np.empty((2, M, K), dtype=np.int64)
    sb = np.empty((2, N, K), dtype=np.int64)
    sa[0], sb[0] = 32, 32
    sa[1] = rng.choice(sparse, size=(M, K)) * rng.choice([-1, 1], size=(M, K))
    sb[1] = rng.choice(sparse, size=(N, K)) * rng.choice([-1, 1], size=(N, K))
    enc = np.vectorize(lambda v: code[int(v)], otypes=[np.uint8])
    bA = dev.upload(to_blocks(enc(sa)).ravel())
    bB = dev.upload(to_blocks(enc(sb)).ravel())
    gd = GroupsDesc()
    gd.nout, gd.nplanes = 2, 2
    for o in range(2):
        g = gd.g[o]
        g.npairs, g.modulus, g.m, g.coef = 1, o, 2401, 7 + o
        g.a[0] = g.b[0] = o
        g.bound = float(K * 32 * 32)
    assert gd.g[0].bound == 2.0 ** 24
    bP, bW = dev.alloc(4 * 2 * M * N), dev.alloc(2 * 2 * M * N)
    dev.gemm_groups_f8(bA, bB, bP, M, N, K, gd, 0, N, M * K, N * K, M * N)
    dev.gemm_groups_f8(bA, bB, bW, M, N, K, gd, 1, N, M * K, N * K, M * N)
    P = dev.download(bP, np.int32, 2 * M * N).reshape(2, M, N).astype(np.int64)
    W = dev.download(bW, np.uint16, 2 * M * N).reshape(2, M, N).astype(np.int64)
    for buf in (bA, bB, bP, bW):
        buf.free()
    dev.bufs.clear()
    assert np.all(P[0] == 2 ** 24)
    want = (sa[1].astype(np.float64) @ sb[1].astype(np.float64).T).astype(np.int64)
    np.testing.assert_array_equal(P[1], want)
    for o in range(2):
        assert_residues(W[o], (7 + o) * (P[o] % 2401), 2401, f"output {o}")


AUTO, I8 = oz.Transport.Automatic, oz.Transport.Int8Residues


@pytest.mark.parametrize("scheme,fmt,transport", [(oz.Scheme.II, oz.Format.INT8, AUTO),
                                                  (oz.Scheme.II, oz.Format.FP8, AUTO),
                                                  (oz.Scheme.II, oz.Format.FP8, I8),
                                                  (oz.Scheme.I, oz.Format.INT8, AUTO),
                                                  (oz.Scheme.I, oz.Format.BF16, AUTO)])
def test_whole_pass_replay_is_checked(ctx, scheme, fmt, transport):
    """The whole-pass check (reference evaluation_hooks.hpp:175-211): the replays of a sound pass are
    checked; a replay that leaves out one phase's steps fails the check and is not timed, whichever
    phase it is, and the returned C stays the first pass's."""
    n = 512
    a, b = oz.eval_inputs(3, 0.5, n * n, n * n)
    o = oz.Options(scheme=scheme, format=fmt, transport=transport)
    c0 = ctx.multiply(a, b, n, n, n, o)
    c, info, ev = ctx.evaluate(a, b, n, n, n, o, warmup=1, repeats=2)
    assert ev.whole_checked == 1 and ev.whole_sentinel == 1 and ev.whole_ms > 0
    assert list(ev.whole_steps) == list(ev.expected_steps) and ev.expected_steps[2] >= 1
    np.testing.assert_array_equal(c.view(np.uint64), c0.view(np.uint64))
    phases = [1, 2, 4] + ([0] if scheme == oz.Scheme.II else [])
    for drop in phases:
        c1, _, bad = ctx.evaluate(a, b, n, n, n, o, repeats=2, replay_drop_phase=drop)
        assert bad.whole_checked == 0 and bad.whole_ms == 0, drop
        assert bad.whole_steps[drop] == 0 and bad.expected_steps[drop] >= 1
        np.testing.assert_array_equal(c1.view(np.uint64), c0.view(np.uint64))
