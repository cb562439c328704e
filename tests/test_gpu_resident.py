"""Resident operands (ozTTgemm::Matrix, an extension of the reference interface; the "persistent
device matrices and cached plan" item beyond the reference, whose README.md:81-85 rebuilds
everything per call).

The contract: gemm on resident a, b gives the same C bit for bit, and the same Info, as gemm on
their host copies, because the device copies use the same zero-padded layouts, and the planner
reads the same padded host data or reuses the plan it made for the pair. The plan of a pair is
kept: the second call reports plan_reused and gives the same C. A result kept on the GPU chains
into later products, and a previous result's device memory is lent to the next one. The resident C
is also compared with the oracle's whole chain on the padded operands (tests/oracle_chains.py), so a
mistake in the padded role copies or the kept plan that the host-span path shares is caught too.
"""
import numpy as np
import pytest

import oztt_amd as oz
from tests.test_gpu_bands import oracle_c

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


CASES = [
    ("II-INT8", oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8)),
    ("II-FP8", oz.Options(scheme=oz.Scheme.II, format=oz.Format.FP8)),
    ("II-BFP8-2pass", oz.Options(scheme=oz.Scheme.II, format=oz.Format.BFP8,
                                 reconstruction=oz.Reconstruction.TwoPass)),
    ("I-INT8", oz.Options(scheme=oz.Scheme.I, format=oz.Format.INT8)),
    ("I-BF16", oz.Options(scheme=oz.Scheme.I, format=oz.Format.BF16, slices=6)),
    ("II-FP8-int8", oz.Options(scheme=oz.Scheme.II, format=oz.Format.FP8, transport=oz.Transport.Int8Residues)),
]


def bits(x):
    return np.ascontiguousarray(x).view(np.uint64)


@pytest.mark.parametrize("name,opts", CASES, ids=[c[0] for c in CASES])
def test_resident_matches_host_call(ctx, oracle, name, opts):
    m, n, k = 300, 200, 130  # every dimension padded
    a, b = oz.eval_inputs(21, 1.0, m * k, k * n)
    want = np.empty(m * n)
    i0 = ctx.gemm(a, b, want, m, n, k, opts)
    A, B = ctx.upload(a, m, k), ctx.upload(b, k, n)
    assert A.shape == (m, k) and B.shape == (k, n)
    got = np.empty(m * n)
    ev1 = oz.EvalStats()
    i1 = ctx.gemm_resident(A, B, got, opts, evaluation=ev1)
    np.testing.assert_array_equal(bits(got), bits(want))
    assert i1 == i0 and not ev1.plan_reused
    np.testing.assert_array_equal(bits(got), bits(oracle_c(oracle, a, b, m, n, k, opts, False, i1)))
    # second call: the kept plan, the same C
    got2 = np.empty(m * n)
    ev2 = oz.EvalStats()
    i2 = ctx.gemm_resident(A, B, got2, opts, evaluation=ev2)
    assert ev2.plan_reused and i2 == i0
    np.testing.assert_array_equal(bits(got2), bits(want))
    # result on the GPU, downloaded
    C = oz.Matrix()
    i3 = ctx.gemm_resident(A, B, C, opts)
    assert C.shape == (m, n) and i3 == i0
    np.testing.assert_array_equal(bits(ctx.download(C)), bits(want))


def test_resident_chain_and_roles(ctx):
    """A result used as the next left operand, and one matrix used as A and as B (A*A)."""
    opts = oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8)
    n = 192
    a, b = oz.eval_inputs(5, 0.5, n * n, n * n)
    A, B = ctx.upload(a, n, n), ctx.upload(b, n, n)
    C = oz.Matrix()
    ctx.gemm_resident(A, B, C, opts)
    D = oz.Matrix()
    ctx.gemm_resident(C, B, D, opts)
    c_host = ctx.multiply(a, b, n, n, n, opts)
    d_host = ctx.multiply(c_host, b, n, n, n, opts)
    np.testing.assert_array_equal(bits(ctx.download(D)), bits(d_host))
    sq = np.empty(n * n)
    ctx.gemm_resident(A, A, sq, opts)
    np.testing.assert_array_equal(bits(sq), bits(ctx.multiply(a, a, n, n, n, opts)))


def test_resident_result_memory_is_reused(ctx):
    """c's previous matrix lends its device memory when nobody else holds it; results stay correct,
    and a result that is also an operand (C = C*B) is computed before the old C is released."""
    opts = oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8)
    n = 256
    a, b = oz.eval_inputs(8, 0.5, n * n, n * n)
    A, B = ctx.upload(a, n, n), ctx.upload(b, n, n)
    C = oz.Matrix()
    ctx.gemm_resident(A, B, C, opts)
    first = ctx.download(C)
    ctx.gemm_resident(A, B, C, opts)  # reuses C's memory
    np.testing.assert_array_equal(bits(ctx.download(C)), bits(first))
    ctx.gemm_resident(C, B, C, opts)  # C is an operand: new memory, then the old C goes
    np.testing.assert_array_equal(bits(ctx.download(C)), bits(ctx.multiply(first, b, n, n, n, opts)))


def test_resident_checks(ctx):
    opts = oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8)
    A = ctx.upload(np.ones(6), 2, 3)
    B = ctx.upload(np.ones(6), 2, 3)
    with pytest.raises(ValueError):  # 2x3 times 2x3
        ctx.gemm_resident(A, B, np.empty(9), opts)
    Bt = ctx.upload(np.ones(6), 3, 2)
    with pytest.raises(ValueError):  # c has the wrong size
        ctx.gemm_resident(A, Bt, np.empty(5), opts)
    small = ctx.upload(np.full(4, 2.0 ** -130), 2, 2)  # row maximum below 2^-126
    with pytest.raises(ValueError):
        ctx.gemm_resident(small, ctx.upload(np.ones(4), 2, 2), np.empty(4), opts)
    other = oz.Context()
    X = other.upload(np.ones(4), 2, 2)
    with pytest.raises(ValueError):  # a Matrix of another Context
        ctx.gemm_resident(X, ctx.upload(np.ones(4), 2, 2), np.empty(4), opts)
    other.close()
    X.close()  # a Matrix may outlive its Context: it holds the GPU open until it is freed


@pytest.mark.parametrize("name,opts,fp8_cores", [c + (False,) for c in CASES[:2] + CASES[3:4] + CASES[5:6]] +
                         [("II-FP8-int8-cores", CASES[5][1], True)],
                         ids=["II-INT8", "II-FP8", "I-INT8", "II-FP8-int8", "II-FP8-int8-cores"])
def test_resident_row_bands(ctx, oracle, name, opts, fp8_cores):
    """Resident operands through row bands (forced by the evaluation hook max_band_rows): the band
    loop reads A's rows from the resident copy and writes C's rows into the result. II-FP8-int8-cores:
    the FP8 route's e4m3 digits on the FP8 matrix cores under Transport.Int8Residues (the evaluation
    setting), against the default call's C."""
    m, n, k = 1000, 384, 512
    a, b = oz.eval_inputs(11, 1.0, m * k, k * n)
    want = np.empty(m * n)
    ctx.gemm(a, b, want, m, n, k, opts)
    A, B = ctx.upload(a, m, k), ctx.upload(b, k, n)
    ev = oz.EvalStats()
    ev.max_band_rows = 256
    ev.fp8_matrix_cores = int(fp8_cores)
    got = np.empty(m * n)
    info = ctx.gemm_resident(A, B, got, opts, evaluation=ev)
    assert ev.gemm_launches == 4
    np.testing.assert_array_equal(bits(got), bits(want))
    np.testing.assert_array_equal(bits(got), bits(oracle_c(oracle, a, b, m, n, k, opts, fp8_cores, info)))
    C = oz.Matrix()
    ev2 = oz.EvalStats()
    ev2.max_band_rows = 256
    ev2.fp8_matrix_cores = int(fp8_cores)
    ctx.gemm_resident(A, B, C, opts, evaluation=ev2)
    assert ev2.gemm_launches == 4
    np.testing.assert_array_equal(bits(ctx.download(C)), bits(want))
