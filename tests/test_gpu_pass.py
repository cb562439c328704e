"""The whole Scheme II INT8 pass in one C-ABI call (oz2_gemm_f64) on device-resident operands.

1. With the plan of the public API (dimensions that need no padding), the pass gives the public
   call's C bit for bit, and the range flags are clear.
2. With extents that are not multiples of the tile grid and leading dimensions larger than the
   extents, C equals the oracle's chain (scale, residues, exact products, exact CRT) bit for bit,
   and nothing outside the M x N window of C is written.
3. Bad arguments are refused before anything is launched: too small or misaligned a workspace,
   descriptors of different plans, a K too large for exact int32 products.
"""
import ctypes

import numpy as np
import pytest

import oztt_amd as oz
from oztt_amd.device import crt_desc, moduli_desc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


def plan_descs(a, b, M, N, K, **kw):
    p = oz.plan2_int8(a, b, M, N, K, **kw)
    moduli = [p.m[i] for i in range(p.S)]
    return moduli, p.b, p.nd, moduli_desc(moduli, p.nd), crt_desc(moduli, p.b, p.nd)


def run_pass(dev, a, lda, b, ldb, M, N, K, ldc, md, cd, fill=np.nan):
    bA, bB = dev.upload(a), dev.upload(b)
    c0 = np.full(M * ldc, fill)
    bC = dev.upload(c0)
    fl = dev.alloc(8)
    nbytes = dev.gemm_f64_workspace(M, N, K, md.S)
    work = dev.alloc(nbytes)
    dev.gemm_f64(bA, lda, bB, ldb, bC, ldc, M, N, K, md, cd, fl, work, nbytes)
    c = dev.download(bC, np.float64, M * ldc).reshape(M, ldc)
    flags = dev.download(fl, np.uint32, 2)
    for x in (bA, bB, bC, fl, work):
        x.free()
    dev.bufs.clear()
    return c, flags


@pytest.mark.parametrize("n,seed,phi", [(1024, 1, 0.5), (512, 3, 2.0)])
def test_pass_equals_public_call(ctx, dev, n, seed, phi):
    a, b = oz.eval_inputs(seed, phi, n * n, n * n)
    moduli, bw, nd, md, cd = plan_descs(a, b, n, n, n)
    c, flags = run_pass(dev, a, n, b, n, n, n, n, n, md, cd)
    want = np.empty(n * n)
    info = ctx.gemm(a, b, want, n, n, n, oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8))
    # Info reports the reference's plan (the set for the window K 2^(2b)); the pass computes with the
    # execution set, which the operands' own window may make smaller (512^3 at phi 2: 16 of 17)
    p = oz.plan2_int8(a, b, n, n, n)
    assert info.moduli == p.rS == (p.S_window or len(moduli)) and info.integer_bits == bw
    assert not flags.any()
    np.testing.assert_array_equal(c.ravel().view(np.uint64), want.view(np.uint64))


def test_pass_ragged_shape_and_leading_dimensions(dev, oracle):
    M, N, K = 1000, 700, 1500
    lda, ldb, ldc = K + 8, N + 20, N + 10
    rng = np.random.default_rng(5)
    A = (rng.uniform(-0.5, 0.5, (M, K)) * np.exp(rng.normal(0, 1.0, (M, K))))
    B = (rng.uniform(-0.5, 0.5, (K, N)) * np.exp(rng.normal(0, 1.0, (K, N))))
    a = np.zeros((M, lda))
    a[:, :K] = A
    b = np.zeros((K, ldb))
    b[:, :N] = B
    moduli, bw, nd, md, cd = plan_descs(A.ravel(), B.ravel(), M, N, K)
    c, flags = run_pass(dev, a, lda, b, ldb, M, N, K, ldc, md, cd, fill=-7.0)
    assert not flags.any()
    assert np.all(c[:, N:] == -7.0)  # only the M x N window is written
    shift = bw - 20 * (nd - 1)
    dA, _ = oracle.scale(A, M, K, 0, 1, shift)
    dB, _ = oracle.scale(B, K, N, 1, 1, shift)
    ra = oracle.residues(A, M, K, 0, dA, nd, moduli)
    rb = oracle.residues(B, K, N, 1, dB, nd, moduli)
    C = np.stack([(ra[s].astype(np.float64) @ rb[s].astype(np.float64)).astype(np.int32) for s in range(len(moduli))])
    want = oracle.crt_exact(C, M, N, moduli, bw, nd, dA, dB)
    np.testing.assert_array_equal(c[:, :N].ravel().view(np.uint64), want.view(np.uint64))


def test_pass_refuses_bad_arguments(dev):
    n = 256
    a, b = oz.eval_inputs(1, 0.5, n * n, n * n)
    moduli, bw, nd, md, cd = plan_descs(a, b, n, n, n)
    bA, bB, bC, fl = dev.upload(a), dev.upload(b), dev.alloc(8 * n * n), dev.alloc(8)
    need = dev.gemm_f64_workspace(n, n, n, md.S)
    work = dev.alloc(need + 256)
    with pytest.raises(RuntimeError, match="workspace needs"):
        dev.gemm_f64(bA, n, bB, n, bC, n, n, n, n, md, cd, fl, work, need - 1)

    class NoBuffer:
        ptr = ctypes.c_void_p()

    with pytest.raises(RuntimeError, match="workspace needs"):
        dev.gemm_f64(bA, n, bB, n, bC, n, n, n, n, md, cd, fl, NoBuffer(), need)
    with pytest.raises(RuntimeError, match="exact int32"):
        dev.gemm_f64(bA, 140000, bB, n, bC, n, n, n, 140000, md, cd, fl, work, need)
    other = crt_desc(moduli, bw, nd)
    other.m[0] -= 1
    with pytest.raises(RuntimeError, match="same INT8 moduli"):
        dev.gemm_f64(bA, n, bB, n, bC, n, n, n, n, md, other, fl, work, need)
    other = crt_desc(moduli, bw, nd)
    other.shift += 1
    with pytest.raises(RuntimeError, match="shift"):
        dev.gemm_f64(bA, n, bB, n, bC, n, n, n, n, md, other, fl, work, need)
    with pytest.raises(RuntimeError, match="leading"):
        dev.gemm_f64(bA, n - 1, bB, n, bC, n, n, n, n, md, cd, fl, work, need)
    for x in (bA, bB, bC, fl, work):
        x.free()
    dev.bufs.clear()
