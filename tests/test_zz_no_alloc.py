"""oz2_gemm_f64_noalloc, the whole Scheme II INT8 pass with its intermediates in the library's own
device array (no workspace argument, no allocation), against oz2_gemm_f64 with a caller workspace:
two calls in a row, the second with a smaller problem and another plan (the array then holds the
first call's contents), each bit-identical in C and in the range flags; and a problem beyond the
array's size refused with a clear error, before anything is launched."""
import ctypes

import numpy as np
import pytest

import oztt_amd as oz
from oztt_amd import hip
from oztt_amd.device import crt_desc, moduli_desc

pytestmark = pytest.mark.gpu


def descs(a, b, M, N, K):
    p = oz.plan2_int8(a, b, M, N, K)
    moduli = [p.m[i] for i in range(p.S)]
    return moduli_desc(moduli, p.nd), crt_desc(moduli, p.b, p.nd)


def noalloc(dev, bA, lda, bB, ldb, bC, ldc, M, N, K, md, cd, fl):
    return hip().oz2_gemm_f64_noalloc(dev.h, bA.ptr, lda, bB.ptr, ldb, bC.ptr, ldc, M, N, K, ctypes.byref(md),
                                      ctypes.byref(cd), fl.ptr)


@pytest.mark.parametrize("calls", [[(1024, 1024, 1024, 1, 0.5), (512, 384, 320, 4, 2.0)]])
def test_noalloc_matches_workspace_pass(dev, calls):
    for M, N, K, seed, phi in calls:
        print(f"no-alloc pass {M}x{N}x{K} seed {seed}", flush=True)
        a, b = oz.eval_inputs(seed, phi, M * K, K * N)
        md, cd = descs(a, b, M, N, K)
        bA, bB = dev.upload(a), dev.upload(b)
        bC1, bC2 = dev.upload(np.full(M * N, np.nan)), dev.upload(np.full(M * N, np.nan))
        fl1, fl2 = dev.alloc(8), dev.alloc(8)
        dev.fill_u32(fl2, 0xFFFFFFFF, 2)  # the pass must clear the flags itself
        need = dev.gemm_f64_workspace(M, N, K, md.S)
        assert need <= 256 << 20
        work = dev.alloc(need)
        dev.gemm_f64(bA, K, bB, N, bC1, N, M, N, K, md, cd, fl1, work, need)
        st = noalloc(dev, bA, K, bB, N, bC2, N, M, N, K, md, cd, fl2)
        assert st == 0, hip().oz_last_error(dev.h)
        want = dev.download(bC1, np.float64, M * N)
        got = dev.download(bC2, np.float64, M * N)
        np.testing.assert_array_equal(got.view(np.uint64), want.view(np.uint64))
        np.testing.assert_array_equal(dev.download(fl2, np.uint32, 2), dev.download(fl1, np.uint32, 2))
        assert not dev.download(fl2, np.uint32, 2).any()
        for x in (bA, bB, bC1, bC2, fl1, fl2, work):
            x.free()
        dev.bufs.clear()


def test_noalloc_refuses_problems_beyond_its_array(dev):
    n = 4096
    a, b = oz.eval_inputs(1, 0.5, 256 * 256, 256 * 256)
    md, cd = descs(a, b, 256, 256, 256)
    assert dev.gemm_f64_workspace(n, n, n, md.S) > 256 << 20
    small = dev.alloc(8)  # never touched: the size check comes first
    st = noalloc(dev, small, n, small, n, small, n, n, n, n, md, cd, small)
    assert st == -1
    msg = hip().oz_last_error(dev.h).decode()
    assert "bytes of scratch; the limit is 268435456" in msg
    small.free()
    dev.bufs.clear()
