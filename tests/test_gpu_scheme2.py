"""End-to-end Scheme II INT8 on the GPU.

1. The reference's own correctness cases (tests/correctness.cpp:188-308): relative Frobenius error
   <= 8 eps against a long-double reference, rejected configurations leave C untouched.
2. Bit-exact chain against the oracle: residue planes, int32 products (full K on sampled rows),
   and the reconstructed C (exact CRT), for the BASELINE config C1 and the reference's quick case.
3. The reference's published output hash (tools/validated/quick.csv:13, fe063f5214e93e2e): the
   GPU products fed to the oracle's restatement of the reference reconstruction reproduce it.
"""
import numpy as np
import pytest

import oztt_amd as oz
from oztt_amd.device import crt_desc, from_blocks, moduli_desc

pytestmark = pytest.mark.gpu

EPS = np.finfo(np.float64).eps
II_INT8 = oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8)


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


def ref_error(a, b, c, m, n, k):
    A = a.reshape(m, k).astype(np.longdouble)
    B = b.reshape(k, n).astype(np.longdouble)
    R = A @ B
    err = np.sqrt(np.sum((c.reshape(m, n) - R) ** 2))
    nrm = np.sqrt(np.sum(R ** 2))
    return float(err / nrm) if nrm > 0 else float(err)


def pattern(mode, m, n, k):
    """Inputs of the reference's check() (tests/correctness.cpp:191-236), seeded."""
    rng = np.random.default_rng(42)
    a = rng.uniform(-1, 1, m * k)
    b = rng.uniform(-1, 1, k * n)
    if mode == "zero-A":
        a[:] = 0
    if mode == "nonnegative":
        a, b = np.abs(a), np.abs(b)
    if mode == "scaled":
        a = (a.reshape(m, k) * np.exp2((np.arange(m) % 31 - 15))[:, None]).ravel()
        b = (b.reshape(k, n) * np.exp2((np.arange(n) % 27 - 13))[None, :]).ravel()
    if mode == "zero-row-column":
        a.reshape(m, k)[0, :] = 0
        b.reshape(k, n)[:, 0] = 0
    if mode == "smallest-maximum":
        a[:] = 2.0 ** -126
        b[:] = 1
    if mode == "largest-maximum":
        a[:] = float.fromhex("0x1.fep127")
        b[:] = 1
    if mode == "cancellation":
        a = np.tile(np.where(np.arange(k) % 2, -1.0, 1.0), m)
        b[:] = 1
    return a, b


CASES = [("uniform", 64, 64, 64), ("nonnegative", 3, 5, 7), ("scaled", 65, 67, 97), ("zero-A", 9, 11, 17),
         ("cancellation", 3, 5, 64), ("zero-row-column", 3, 5, 7), ("smallest-maximum", 1, 1, 1),
         ("largest-maximum", 1, 1, 1), ("uniform", 5056, 64, 32)]


@pytest.mark.parametrize("fmt,transport", [(oz.Format.INT8, oz.Transport.Automatic),
                                           (oz.Format.FP8, oz.Transport.Automatic),
                                           (oz.Format.FP8, oz.Transport.Int8Residues)],
                         ids=["INT8", "FP8", "FP8-int8"])
@pytest.mark.parametrize("mode,m,n,k", CASES)
def test_reference_correctness_cases(ctx, mode, m, n, k, fmt, transport):
    """FP8: the FP8 route's e4m3 digits on the FP8 matrix cores (the default); FP8-int8: the FP8 plan
    carried by INT8 residues at its width (Transport.Int8Residues)."""
    a, b = pattern(mode, m, n, k)
    o = oz.Options(scheme=oz.Scheme.II, format=fmt, transport=transport)
    c = np.full(m * n, 123.0)
    info = ctx.gemm(a, b, c, m, n, k, o)
    assert info.format == fmt
    assert np.all(np.isfinite(c))
    err = ref_error(a, b, c, m, n, k)
    assert err <= 8 * EPS, (mode, err)
    assert info.moduli >= 2 and info.integer_bits >= 53
    assert (info.padded_m, info.padded_n, info.padded_k) == (-(-m // 64) * 64, -(-n // 64) * 64, -(-k // 32) * 32)


def test_two_pass_and_overlap(ctx):
    a, b = pattern("uniform", 64, 64, 64)
    c = np.empty(64 * 64)
    info = ctx.gemm(a, b, c, 64, 64, 64, oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8,
                                                      reconstruction=oz.Reconstruction.TwoPass))
    assert info.reconstruction_passes == 2
    assert ref_error(a, b, c, 64, 64, 64) <= 8 * EPS
    # input and output may overlap (tests/correctness.cpp:285-288)
    ov = np.array([1.0, 2, 3, 4])
    ctx.gemm(ov, np.array([1.0, 0, 0, 1]), ov, 2, 2, 2, II_INT8)
    assert list(ov) == [1, 2, 3, 4]


def test_too_few_moduli_rejected_and_c_untouched(ctx):
    a = np.ones(64 * 64)
    c = np.full(64 * 64, 123.0)
    with pytest.raises(RuntimeError):
        ctx.gemm(a, a, c, 64, 64, 64, oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8, max_moduli=2))
    assert np.all(c == 123.0)


def run_stages(dev, A, B, M, N, K, moduli, b, nd):
    """scale -> split -> products -> CRT on the GPU through the C ABI; returns host copies."""
    S = len(moduli)
    Mg, Ng, Kg = -(-M // 256) * 256, -(-N // 256) * 256, -(-K // 64) * 64
    shift = b - 20 * (nd - 1)
    bA, bB = dev.upload(A), dev.upload(B)
    bdA, bdB = dev.alloc(4 * M), dev.alloc(4 * N)
    bfl = dev.alloc(8)
    dev.fill_u32(bfl, 0, 2)
    dev.scale(bA, M, K, K, 0, 1, shift, bdA, bfl, 0)
    dev.scale(bB, K, N, N, 1, 1, shift, bdB, bfl, 1)
    md = moduli_desc(moduli, nd)
    pA, pB = dev.alloc(S * Mg * Kg), dev.alloc(S * Ng * Kg)
    dev.split_int8(bA, M, K, K, 0, bdA, md, pA, 2, Mg, Kg, Mg * Kg)  # OZ_BLOCK tiles
    dev.split_int8(bB, K, N, N, 1, bdB, md, pB, 3, Ng, Kg, Ng * Kg)
    bC = dev.alloc(4 * S * Mg * Ng)
    dev.gemm_i8(pA, pB, bC, Mg, Ng, Kg, S, Ng, Mg * Kg, Ng * Kg, Mg * Ng)
    bo = dev.alloc(8 * M * N)
    dev.crt(bC, M, N, Ng, Mg * Ng, crt_desc(moduli, b, nd), bdA, bdB, bo, N)
    r = dict(dA=dev.download(bdA, np.int32, M), dB=dev.download(bdB, np.int32, N),
             flags=dev.download(bfl, np.uint32, 2),
             planesA=from_blocks(dev.download(pA, np.int8, S * Mg * Kg).reshape(S, -1), Mg, Kg)[:, :M, :K],
             planesB=from_blocks(dev.download(pB, np.int8, S * Ng * Kg).reshape(S, -1), Ng, Kg)[:, :N, :K],
             C=dev.download(bC, np.int32, S * Mg * Ng).reshape(S, Mg, Ng)[:, :M, :N],
             out=dev.download(bo, np.float64, M * N))
    for buf in (bA, bB, bdA, bdB, bfl, pA, pB, bC, bo):
        buf.free()
    dev.bufs.clear()
    return r


def test_reference_output_hash_quick_int8(dev, oracle):
    """tools/validated/quick.csv:13: II INT8 128^3, uniform seed 7, b=54, 15 moduli, one pass."""
    n = 128
    a, b = oz.eval_inputs(7, -1.0, n * n, n * n)
    p = oz.plan2_int8(a, b, n, n, n, max_moduli=16, reconstruction=oz.Reconstruction.OnePass, fixed_bits=54)
    moduli = [p.m[i] for i in range(p.S)]
    assert p.S == 15 and p.b == 54 and p.nd == 3
    r = run_stages(dev, a, b, n, n, n, moduli, 54, 3)
    ref_out = oracle.crt_ref(np.ascontiguousarray(r["C"]), n, n, moduli, 54, 3, False, r["dA"], r["dB"])
    assert oracle.hash(ref_out) == 0xfe063f5214e93e2e
    # and the product path's exact reconstruction equals the oracle's exact CRT of the same products
    ex = oracle.crt_exact(np.ascontiguousarray(r["C"]), n, n, moduli, 54, 3, r["dA"], r["dB"])
    np.testing.assert_array_equal(r["out"].view(np.uint64), ex.view(np.uint64))


def test_baseline_c1_bit_exact_chain(dev, oracle, ctx):
    """II INT8 1024^3, (U(0,1)-0.5)*exp(0.5 N(0,1)) seed 1, auto moduli, one pass."""
    n = 1024
    a, b = oz.eval_inputs(1, 0.5, n * n, n * n)
    p = oz.plan2_int8(a, b, n, n, n, reconstruction=oz.Reconstruction.OnePass)
    moduli = [p.m[i] for i in range(p.S)]
    b_, nd = p.b, p.nd
    r = run_stages(dev, a, b, n, n, n, moduli, b_, nd)
    shift = b_ - 20 * (nd - 1)
    dA, fA = oracle.scale(a.reshape(n, n), n, n, 0, 1, shift)
    dB, fB = oracle.scale(b.reshape(n, n), n, n, 1, 1, shift)
    np.testing.assert_array_equal(r["dA"], dA)
    np.testing.assert_array_equal(r["dB"], dB)
    assert fA == fB == 0 and not r["flags"].any()
    want_A = oracle.residues(a.reshape(n, n), n, n, 0, dA, nd, moduli)
    want_B = oracle.residues(b.reshape(n, n), n, n, 1, dB, nd, moduli)
    np.testing.assert_array_equal(r["planesA"], want_A)
    np.testing.assert_array_equal(r["planesB"], want_B.transpose(0, 2, 1))
    rows = np.arange(0, n, 61)
    for s in range(len(moduli)):
        want_C = want_A[s, rows].astype(np.int64) @ want_B[s].astype(np.int64)
        np.testing.assert_array_equal(r["C"][s, rows].astype(np.int64), want_C)
    ex = oracle.crt_exact(np.ascontiguousarray(r["C"]), n, n, moduli, b_, nd, r["dA"], r["dB"])
    np.testing.assert_array_equal(r["out"].view(np.uint64), ex.view(np.uint64))
    # the public API gives the same bits
    c = np.empty(n * n)
    info = ctx.gemm(a, b, c, n, n, n, oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8,
                                                   reconstruction=oz.Reconstruction.OnePass))
    assert info.moduli == p.rS == (p.S_window or len(moduli)) and info.integer_bits == b_
    assert info.reconstruction_passes == 1
    np.testing.assert_array_equal(c.view(np.uint64), r["out"].view(np.uint64))
    # accuracy against binary128 on a sample: within the FP64 bound |A||B| k 2^-53 and close to C
    rs = np.random.default_rng(0).integers(0, n, 256)
    cs = np.random.default_rng(1).integers(0, n, 256)
    q = oracle.quad_sample(a, b, n, n, n, rs, cs)
    got = c.reshape(n, n)[rs, cs]
    absab = (np.abs(a.reshape(n, n)[rs]) * np.abs(b.reshape(n, n)[:, cs].T)).sum(axis=1)
    assert np.all(np.abs(got - q) <= absab * n * 2.0 ** -53)
    assert np.max(np.abs(got - q) / np.abs(q)) < 1e-13


def test_evaluation_hooks_bit_identical(ctx):
    """Whole-pass replays reproduce the first pass bit for bit (tests/correctness.cpp:88-172)."""
    n = 256
    a, b = oz.eval_inputs(3, 0.5, n * n, n * n)
    c0 = ctx.multiply(a, b, n, n, n, II_INT8)
    c1, info, ev = ctx.evaluate(a, b, n, n, n, II_INT8, warmup=1, repeats=3)
    assert ev.whole_checked == 1 and ev.whole_ms > 0 and ev.gemm_launch_ms > 0
    assert all(ev.phase_ms[i] > 0 for i in (0, 1, 2, 4))
    np.testing.assert_array_equal(c0.view(np.uint64), c1.view(np.uint64))
