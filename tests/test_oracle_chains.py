"""The whole oracle chains of tests/oracle_chains.py, pinned on the CPU before the GPU tests trust them:
each reproduces the reference's published outputs (tools/validated/quick.csv) from the FP64 inputs, and
the exact reconstruction gives the same C from two different moduli sets of one width."""
import numpy as np
import pytest

import oztt_amd as oz
from tests.oracle_chains import oz1_chain, oz2_chain
from tests.test_planner import EVAL_LIMIT, ROUTE_HASHES

N = 128


@pytest.fixture(scope="module")
def quick_inputs():
    a, b = oz.eval_inputs(7, -1.0, N * N, N * N)
    return a.reshape(N, N), b.reshape(N, N)


def test_oz2_chain_reference_hash_int8(oracle, quick_inputs):
    """quick.csv:13: II INT8 128^3, b = 54, 16 moduli requested, one pass -> fe063f5214e93e2e."""
    A, B = quick_inputs
    p = oz.plan2(A, B, N, N, N, oz.Format.INT8, max_moduli=16, fixed_bits=54)
    ms = [p.m[i] for i in range(p.S)]
    assert len(ms) == 15
    assert oracle.hash(oz2_chain(oracle, A, B, ms, 54, 3, reference_passes=1)) == 0xFE063F5214E93E2E


@pytest.mark.parametrize("fmt", ["BF16", "TF32", "BFP4", "BFP2"])
def test_oz2_chain_reference_hash_routes(oracle, quick_inputs, fmt):
    """The digit routes' published outputs at 128^3 from the routes' own sets (moduli up to 4096)."""
    A, B = quick_inputs
    p = oz.plan2(A, B, N, N, N, oz.Format[fmt], max_moduli=EVAL_LIMIT.get(fmt, 24), fixed_bits=54,
                 reconstruction=oz.Reconstruction.OnePass)
    rm = [p.rm[i] for i in range(p.rS)]
    assert oracle.hash(oz2_chain(oracle, A, B, rm, 54, 3, reference_passes=1)) == ROUTE_HASHES[fmt]


def test_oz2_chain_exact_crt_is_a_function_of_the_width(oracle, quick_inputs):
    """Two sets of one width (BFP4's route, moduli up to 4096, and the INT8 set) give the same exact C; the
    reference's one-pass reconstruction of the same products differs from it only in rare last bits, by far
    less than the 2^-53 relative accuracy the plan targets."""
    A, B = quick_inputs
    p = oz.plan2(A, B, N, N, N, oz.Format.BFP4, fixed_bits=54)
    rm = [p.rm[i] for i in range(p.rS)]
    ms = [p.m[i] for i in range(p.S)]
    assert max(rm) > 255 and max(ms) <= 255 and rm != ms
    x = oz2_chain(oracle, A, B, rm, 54, 3)
    y = oz2_chain(oracle, A, B, ms, 54, 3)
    np.testing.assert_array_equal(x.view(np.uint64), y.view(np.uint64))
    ref = oz2_chain(oracle, A, B, ms, 54, 3, reference_passes=1)
    assert 0 < np.mean(ref != x) < 0.01
    assert np.abs(ref - x).max() <= 2.0 ** -53 * np.abs(x).max()


def test_oz1_chain_reference_hashes(oracle, quick_inputs):
    """quick.csv:12 (I INT8, p = 8 -> 6c9693442bfc11b0) and quick.csv:2 (I BF16, p = 10, every diagonal
    read whole -> be6558fa9f435fa0)."""
    A, B = quick_inputs
    assert oracle.hash(oz1_chain(oracle, A, B, 8, "INT8")) == 0x6C9693442BFC11B0
    assert oracle.hash(oz1_chain(oracle, A, B, 10, "BF16", nsmall=10)) == 0xBE6558FA9F435FA0
