"""Row bands on the GPU (the reference's row bands when device memory runs short,
ozaki2/plan.hpp:386-444).

A band recomputes nothing that depends on the other rows: the row maxima of A are per row, the
column maxima and the planes of B are computed once, and the plan comes from the whole operands.
So C must be bit-identical whether the rows run in one band or in many. The evaluation hook
max_band_rows forces bands of 256 rows (the band logic otherwise only engages when the workspace
exceeds the device memory); M = 1000 leaves a ragged last band of 232 rows.

The banded C is also compared with the oracle's whole chain (tests/oracle_chains.py: scale, residues
or slices, exact products, reconstruction, all on the CPU from the FP64 inputs) on the padded operands
the library plans on, so a mistake shared by the one-band and banded paths (the padded copies, the
plan, the band offsets) is caught too.
"""
import numpy as np
import pytest

import oztt_amd as oz
from tests.oracle_chains import oz1_chain, oz2_chain, pad_dims, padded

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


CASES = [
    ("II-INT8", oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8), False),
    ("II-FP8", oz.Options(scheme=oz.Scheme.II, format=oz.Format.FP8), False),
    ("II-FP8-int8", oz.Options(scheme=oz.Scheme.II, format=oz.Format.FP8, transport=oz.Transport.Int8Residues),
     False),
    ("II-FP8-int8-cores", oz.Options(scheme=oz.Scheme.II, format=oz.Format.FP8, transport=oz.Transport.Int8Residues),
     True),
    ("I-INT8", oz.Options(scheme=oz.Scheme.I, format=oz.Format.INT8), False),
    ("I-BF16", oz.Options(scheme=oz.Scheme.I, format=oz.Format.BF16, slices=6), False),
]


def oracle_c(oracle, a, b, m, n, k, opts, fp8_cores, info):
    """C of the oracle's chain for the call's plan, on the zero-padded operands, cropped to m x n."""
    mp, np_, kp = pad_dims(m, n, k)
    A, B = padded(a.reshape(m, k), mp, kp), padded(b.reshape(k, n), kp, np_)
    if opts.scheme == oz.Scheme.II:
        p = oz.plan2(A, B, mp, np_, kp, opts.format, transport=opts.transport, fp8_matrix_cores=fp8_cores)
        # Info: the route's moduli under Transport.Automatic, the moduli that computed under Int8Residues
        computed = opts.transport == oz.Transport.Int8Residues
        assert (p.S if computed else p.rS, p.b) == (info.moduli, info.integer_bits)
        # the set the device computes with (FP8 digits: the route's, or the FP8 set for the operands' own
        # window when that has fewer digit products)
        ms = [p.m[i] for i in range(p.S)]
        if opts.format == oz.Format.FP8:
            assert p.fp8_digits == (fp8_cores or opts.transport == oz.Transport.Automatic)
        if p.fp8_digits:
            assert (p.S_window or p.S) == p.rS and p.nprod <= p.rnprod
        want = oz2_chain(oracle, A, B, ms, p.b, p.nd)
        if p.S_window:  # the same C from the route's own set
            full = oz2_chain(oracle, A, B, [p.rm[i] for i in range(p.rS)], p.b, p.nd)
            np.testing.assert_array_equal(full.view(np.uint64), want.view(np.uint64))
    else:
        pl = oz.plan1(A, B, mp, np_, kp, slices=opts.slices, fmt=opts.format)
        assert pl.p == info.slices and pl.nkb == 1
        want = oz1_chain(oracle, A, B, pl.p, opts.format.name, nsmall=pl.nsmall)
    return np.ascontiguousarray(want[:m, :n]).reshape(-1)


@pytest.mark.parametrize("name,opts,fp8_cores", CASES, ids=[c[0] for c in CASES])
def test_bands_bit_identical(ctx, oracle, name, opts, fp8_cores):
    """II-FP8 and II-FP8-int8-cores: the FP8 route's e4m3 digits on the FP8 matrix cores (A's digit planes
    per band); II-FP8-int8: the FP8 plan on INT8 residues."""
    m, n, k = 1000, 384, 512
    a, b = oz.eval_inputs(11, 1.0, m * k, k * n)
    c1, i1, e1 = ctx.evaluate(a, b, m, n, k, opts, warmup=1, repeats=2, fp8_matrix_cores=fp8_cores)
    c4, i4, e4 = ctx.evaluate(a, b, m, n, k, opts, warmup=1, repeats=2, max_band_rows=256,
                              fp8_matrix_cores=fp8_cores)
    assert e1.gemm_launches == 1
    assert e4.gemm_launches == 4  # 1024 padded rows: 256 + 256 + 256 + 232
    assert e1.whole_checked and e4.whole_checked
    assert (i1.moduli, i1.slices, i1.integer_bits) == (i4.moduli, i4.slices, i4.integer_bits)
    np.testing.assert_array_equal(c4.view(np.uint64), c1.view(np.uint64))
    # both equal the oracle's chain
    want = oracle_c(oracle, a, b, m, n, k, opts, fp8_cores, i4)
    np.testing.assert_array_equal(c4.view(np.uint64), want.view(np.uint64))
    # and the plain call (no evaluation hooks) gives the same C
    c0 = ctx.multiply(a, b, m, n, k, opts)
    np.testing.assert_array_equal(c0.view(np.uint64), c1.view(np.uint64))
