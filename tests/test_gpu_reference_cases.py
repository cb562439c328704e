"""The reference's own device correctness cases (tests/correctness.cpp:259-308) for both schemes and
every format, through the public API: relative Frobenius error at most 8 eps against a long-double
product, C finite, Info consistent. Scheme II INT8 and FP8 run the full pattern set in
test_gpu_scheme2.py; here are the rest:
  * every format with both schemes on 64^3 uniform and 3x5x7 nonnegative inputs (:266-274);
  * Scaled, ZeroA, Cancellation, ZeroRowAndColumn, SmallestMaximum, LargestMaximum with scheme I
    and the reference's first format, BF16 (:275-283);
  * fixed slices (10 for BF16, :284-286), and BF16 64x64x32768, which crosses the exact FP32
    accumulator's K block (:301-306).
"""
import numpy as np
import pytest

import oztt_amd as oz
from tests.test_gpu_scheme2 import EPS, pattern, ref_error

pytestmark = pytest.mark.gpu

FORMATS = [oz.Format.BF16, oz.Format.FP16, oz.Format.TF32, oz.Format.BFP8, oz.Format.FP8, oz.Format.INT8,
           oz.Format.BFP4, oz.Format.BFP2]


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


def run_case(ctx, opts, mode, m, n, k):
    a, b = pattern(mode, m, n, k)
    c = np.full(m * n, 123.0)
    info = ctx.gemm(a, b, c, m, n, k, opts)
    assert np.all(np.isfinite(c))
    err = ref_error(a, b, c, m, n, k)
    assert err <= 8 * EPS, (opts.scheme, opts.format, mode, err)
    assert info.scheme == opts.scheme and info.format == opts.format
    assert (info.padded_m, info.padded_n, info.padded_k) == (-(-m // 64) * 64, -(-n // 64) * 64, -(-k // 32) * 32)
    return info


@pytest.mark.parametrize("scheme", [oz.Scheme.I, oz.Scheme.II])
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("mode,m,n,k", [("uniform", 64, 64, 64), ("nonnegative", 3, 5, 7)])
def test_every_format_both_schemes(ctx, scheme, fmt, mode, m, n, k):
    info = run_case(ctx, oz.Options(scheme=scheme, format=fmt), mode, m, n, k)
    if scheme == oz.Scheme.I:
        assert info.slices >= 1 and info.moduli == 0
    else:
        assert info.moduli >= 2 and info.integer_bits >= 53


@pytest.mark.parametrize("mode,m,n,k", [("scaled", 65, 67, 97), ("zero-A", 9, 11, 17), ("cancellation", 3, 5, 64),
                                        ("zero-row-column", 3, 5, 7), ("smallest-maximum", 1, 1, 1),
                                        ("largest-maximum", 1, 1, 1)])
def test_scheme1_edge_patterns(ctx, mode, m, n, k):
    run_case(ctx, oz.Options(scheme=oz.Scheme.I, format=oz.Format.BF16), mode, m, n, k)


def test_scheme1_fixed_slices(ctx):
    info = run_case(ctx, oz.Options(scheme=oz.Scheme.I, format=oz.Format.BF16, slices=10), "uniform", 3, 5, 7)
    assert info.slices == 10


def test_scheme1_bf16_beyond_one_accumulator_block(ctx):
    info = run_case(ctx, oz.Options(scheme=oz.Scheme.I, format=oz.Format.BF16), "nonnegative", 64, 64, 32768)
    assert info.slices >= 1
