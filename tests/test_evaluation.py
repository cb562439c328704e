"""The evaluator's numerics in the product library (reference evaluation/numerics.hpp): Dot2 reference
GEMM and the accuracy measure, pinned by the effective bits and relative Frobenius errors that the
reference's validated runs recorded (tools/validated/quick.csv:2, :12) for outputs this build
reproduces bit for bit (their hashes are pinned in test_oracle.py)."""
from pathlib import Path

import numpy as np
import pytest

import oztt_amd as oz


@pytest.fixture(scope="module")
def quick_inputs():
    n = 128
    a, b = oz.eval_inputs(7, -1.0, n * n, n * n)
    hi, lo = oz.eval_reference_gemm(a, b, n, n, n)
    return n, a, b, hi, lo


def test_dot2_reference_is_compensated(quick_inputs):
    n, a, b, hi, lo = quick_inputs
    exact = a.reshape(n, n).astype(np.longdouble) @ b.reshape(n, n).astype(np.longdouble)
    # head + tail agrees with the 64-bit-mantissa product to that product's own rounding (~1e-18),
    # a thousand times closer than the head alone
    err = np.abs((hi.astype(np.longdouble) + lo) - exact.ravel())
    err_hi = np.abs(hi.astype(np.longdouble) - exact.ravel())
    assert float(err.max()) < 1e-17 and float(err.max()) * 1000 < float(err_hi.max())
    # row ranges compute the same values
    h2, l2 = oz.eval_reference_gemm(a, b, n, n, n, 40, 70)
    np.testing.assert_array_equal(h2, hi[40 * n:70 * n])
    np.testing.assert_array_equal(l2, lo[40 * n:70 * n])


def test_accuracy_reproduces_reference_records(oracle, quick_inputs):
    n, a, b, hi, lo = quick_inputs
    A, B = a.reshape(n, n), b.reshape(n, n)
    # I-INT8, p = 8 (quick.csv:12)
    out, _ = oracle.oz1_int8_gemm(a, b, n, n, n, 8)
    assert oracle.hash(out) == 0x6C9693442BFC11B0
    rel, eb = oz.eval_accuracy(out, hi, lo)
    assert f"{eb:.12g}" == "54.243846521" and f"{rel:.12g}" == "4.68786522126e-17"
    # I-BF16, p = 10 (quick.csv:2)
    dA, _ = oracle.scale(A, n, n, 0, 0, -1)
    dB, _ = oracle.scale(B, n, n, 1, 0, -1)
    sa = oracle.oz1_slices(A, n, n, 0, dA, 10, 64, 32)
    sb = oracle.oz1_slices(B, n, n, 1, dB, 10, 64, 32)
    Pd, _ = oracle.oz1_gemm_diag(sa, sb, 10)
    out = oracle.oz1_recon(Pd, 64, 0, 10, dA, dB)
    assert oracle.hash(out) == 0xBE6558FA9F435FA0
    rel, eb = oz.eval_accuracy(out, hi, lo)
    assert f"{eb:.12g}" == "54.2420686589" and f"{rel:.12g}" == "4.69364573273e-17"


def test_accuracy_edge_cases():
    z = np.zeros(4)
    assert oz.eval_accuracy(z, z, z) == (0.0, 99.0)
    assert oz.eval_accuracy(np.ones(4), z, z)[0] == np.inf


def test_bench_traffic_figures_come_from_their_profiles():
    """bench.py prints roofline.traffic for every configuration from its committed counter profile: the
    figure (bytes per launch of the product kernel) is the one that profile's table derives from its
    FETCH_SIZE and WRITE_SIZE counters, and the profile names the command that made it."""
    import re
    import bench
    root = Path(__file__).resolve().parent.parent
    for cfg, (traffic, prof, products) in bench.TRAFFIC.items():
        assert traffic is not None and traffic > 0, cfg
        text = (root / prof).read_text()
        assert "rocprofv3 --pmc FETCH_SIZE" in text and "rocprofv3 --pmc WRITE_SIZE" in text, prof
        kernel = "gemm_f8_groups_kernel" if cfg == "C4" else "gemm_i8_kernel"
        rows = [ln for ln in text.splitlines() if ln.startswith(f"| `{kernel}") and "(GB)" not in ln]
        gb = float(rows[0].split("|")[4])  # the traffic column of the per-kernel table
        # the table prints GB to three decimals
        assert abs(gb * 1e9 - traffic) <= max(0.5e6, 0.005 * traffic), (cfg, gb, traffic)
        assert products > 0 and re.search(rf"--config {cfg}\b", text), cfg
