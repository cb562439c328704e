"""Whole oracle chains for the public-call tests: the CPU restatement of every stage of a pass, from
the FP64 operands to C, with nothing taken from the GPU.

Scheme II (reference ozaki2.cpp:439-478): scale (BF16 maxima rounded up, ozaki2.cpp:143-146) ->
symmetric residues of A' and B' per modulus (digits.h:80-179) -> exact products, each reduced to its
symmetric residue -> exact CRT and rounding to FP64. The exact CRT makes C a function of the width b
alone, so any pairwise coprime set whose window holds b gives the same C: the execution set of the
plan, or the format route's own set (moduli up to 4096, residues as int16).

Scheme I (reference ozaki1.cpp run()): scale (the format's rounding) -> p slices of the format's
radix (slice_tf_body.h:86-131) -> diagonal sums of the slice products (stages.hpp:157) -> Horner
reconstruction (recon_tf_i32in.cpp:116-157).

The products are computed in float64 BLAS, which is exact here: every partial sum is an integer below
2^53 (asserted).
"""
from __future__ import annotations

import numpy as np

# Scheme I slicing parameters per format (ozaki1/param.hpp:43-100, ozaki1/format.hpp:85): radix of the
# slices, bound of a slice, BF16 rounding of the maxima (1: up), sign-magnitude int32 sums in the
# reconstruction (INT8 only)
OZ1_FORMAT = {
    "INT8": dict(radix=254, dmax=127, ceil=1, signmag=1),
    "BF16": dict(radix=64, dmax=32, ceil=0, signmag=0),
}


def padded(x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """x (r x c) zero-padded to rows x cols (the public API pads m, n to 64 and k to 32)."""
    out = np.zeros((rows, cols))
    out[: x.shape[0], : x.shape[1]] = x
    return out


def pad_dims(m: int, n: int, k: int):
    up = lambda v, q: (v + q - 1) // q * q
    return up(m, 64), up(n, 64), up(k, 32)


def exact_matmul(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """x @ y for integer-valued arrays whose sums stay below 2^53, as int64."""
    bound = np.abs(x).astype(np.float64).max(initial=0) * np.abs(y).astype(np.float64).max(initial=0) * x.shape[1]
    assert bound < 2.0 ** 53
    return (x.astype(np.float64) @ y.astype(np.float64)).astype(np.int64)


def oz2_chain(oracle, A: np.ndarray, B: np.ndarray, moduli, bw: int, nd: int, reference_passes: int = 0) -> np.ndarray:
    """C (M x N) of Scheme II at width bw with digits nd of A', from padded A (M x K) and B (K x N).
    reference_passes 1 or 2 reconstructs with the oracle's restatement of the reference's triple-float CRT
    (recon_crt.cpp, the reference's published outputs) instead of the exact CRT."""
    M, K = A.shape
    N = B.shape[1]
    shift = bw - 20 * (nd - 1)
    dA, fA = oracle.scale(A, M, K, 0, 1, shift)
    dB, fB = oracle.scale(B, K, N, 1, 1, shift)
    assert fA == 0 and fB == 0
    rA = oracle.residues(A, M, K, 0, dA, nd, moduli)
    rB = oracle.residues(B, K, N, 1, dB, nd, moduli)
    C = np.empty((len(moduli), M, N), dtype=np.int32)
    for s, m in enumerate(moduli):
        r = exact_matmul(rA[s], rB[s]) % m
        C[s] = np.where(r > m // 2, r - m, r)
    if reference_passes:
        return oracle.crt_ref(C, M, N, list(moduli), bw, nd, reference_passes == 2, dA, dB).reshape(M, N)
    return oracle.crt_exact(C, M, N, list(moduli), bw, nd, dA, dB).reshape(M, N)


def oz1_chain(oracle, A: np.ndarray, B: np.ndarray, p: int, fmt: str, nsmall: int = 0) -> np.ndarray:
    """C (M x N) of Scheme I with p slices in one K block, from padded A (M x K) and B (K x N)."""
    M, K = A.shape
    N = B.shape[1]
    f = OZ1_FORMAT[fmt]
    dA, _ = oracle.scale(A, M, K, 0, f["ceil"], -1)
    dB, _ = oracle.scale(B, K, N, 1, f["ceil"], -1)
    sa = oracle.oz1_slices(A, M, K, 0, dA, p, f["radix"], f["dmax"])
    sb = oracle.oz1_slices(B, K, N, 1, dB, p, f["radix"], f["dmax"])
    Pd = np.empty((p, M, N), dtype=np.int32)
    for d in range(p):
        s = sum(exact_matmul(sa[i], sb[d - i]) for i in range(d + 1))
        assert np.abs(s).max(initial=0) < 2**31
        Pd[d] = s
    return oracle.oz1_recon(Pd, f["radix"], f["signmag"], nsmall, dA, dB).reshape(M, N)
