"""Public-API behaviour that needs no GPU (reference tests/correctness.cpp:49-85 host validation), and
the C ABI library: it loads and exports every function include/oz_hip.h declares."""
import re
from pathlib import Path

import numpy as np
import pytest

import oztt_amd as oz

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def ctx():
    c = oz.Context()
    yield c
    c.close()


def test_c_abi_exports_every_declared_symbol():
    hdr = (ROOT / "include" / "oz_hip.h").read_text()
    names = re.findall(r"^\s*(?:int|void|const char\*)\s+(oz\w+)\s*\(", hdr, re.M)
    assert len(names) >= 16
    lib = oz.hip()
    for n in names:
        assert hasattr(lib, n), n


def test_formats():
    assert oz.format_name(oz.Format.INT8) == "INT8" and oz.format_name(oz.Format.BFP2) == "BFP2"
    # both schemes run every format (Scheme I digits and Scheme II residues are int8 values, FP8 digits e4m3)
    assert all(oz.is_available(f) for f in oz.Format)


def test_context_rejects_bad_device_options():
    with pytest.raises(ValueError):
        oz.Context(device_id=-1)
    with pytest.raises(ValueError):
        oz.Context(kernel_directory="/nonexistent/kernel/dir")


OPT = oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8)


def test_host_validation_leaves_c_untouched(ctx):
    a, b, c = np.ones(4), np.ones(4), np.full(4, 123.0)
    cases = [
        lambda: ctx.gemm(a, b, c, 0, 2, 2, OPT),                     # zero dimension
        lambda: ctx.gemm(a, b, c, 2, 3, 2, OPT),                     # span sizes
        lambda: ctx.gemm(a, b, c, 2, 2, 2, oz.Options(scheme=100, format=oz.Format.INT8)),
        lambda: ctx.gemm(a, b, c, 2, 2, 2, oz.Options(scheme=oz.Scheme.II, format=100)),
        lambda: ctx.gemm(a, b, c, 2, 2, 2, oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8, slices=10)),
        lambda: ctx.gemm(a, b, c, 2, 2, 2, oz.Options(scheme=oz.Scheme.I, format=oz.Format.INT8,
                                                      reconstruction=oz.Reconstruction.TwoPass)),
        lambda: ctx.gemm(a, b, c, 2, 2, 2, oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8, max_moduli=25)),
        lambda: ctx.gemm(a, b, c, 2, 2, 2, oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8,
                                                      reconstruction=7)),
        # the transport (an extension) is a Scheme II setting with two values
        lambda: ctx.gemm(a, b, c, 2, 2, 2, oz.Options(scheme=oz.Scheme.II, format=oz.Format.FP8, transport=2)),
        lambda: ctx.gemm(a, b, c, 2, 2, 2, oz.Options(scheme=oz.Scheme.I, format=oz.Format.INT8,
                                                      transport=oz.Transport.Int8Residues)),
    ]
    for f in cases:
        with pytest.raises(ValueError):
            f()
    for bad in (np.nan, np.inf):
        with pytest.raises(ValueError):
            ctx.gemm(np.array([bad, 1, 1, 1]), b, c, 2, 2, 2, OPT)
        with pytest.raises(ValueError):
            ctx.gemm(a, np.array([1, 1, bad, 1]), c, 2, 2, 2, OPT)
    with pytest.raises(ValueError):
        ctx.gemm(np.full(4, 2.0 ** -130), b, c, 2, 2, 2, OPT)  # row maximum below 2^-126
    with pytest.raises(ValueError):
        ctx.gemm(np.full(4, 2.0 ** 128), b, c, 2, 2, 2, OPT)   # row maximum above the BF16 range
    assert np.all(c == 123.0)


def test_resident_upload_validation(ctx):
    """Context.upload (the resident-operand extension) rejects bad input before it touches the GPU."""
    with pytest.raises(ValueError):
        ctx.upload(np.ones(6), 2, 4)          # span size
    with pytest.raises(ValueError):
        ctx.upload(np.ones(4), 0, 4)          # zero dimension
    for bad in (np.nan, np.inf, -np.inf):
        with pytest.raises(ValueError):
            ctx.upload(np.array([1.0, bad, 0.0, 0.0]), 2, 2)
    empty = oz.Matrix()
    assert empty.shape == (0, 0)
    with pytest.raises(ValueError):
        ctx.gemm_resident(empty, empty, np.empty(1))  # empty operands
    with pytest.raises(ValueError):
        ctx.download(empty)
