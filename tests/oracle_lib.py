"""ctypes access to the CPU oracle (oracle/build/liboz_oracle.so). Tests only: the oracle is the
checker, never part of the product path."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "build" / "liboz_oracle.so"

_lib = None


def assert_residues(got, want, m, what: str = "") -> None:
    """The product kernels store (c * y) mod m as a representative in [0, m], m standing for 0
    (oz2::mod_mul_f64): `got` must lie in that range and agree with `want` modulo m."""
    got = np.asarray(got).astype(np.int64)
    m = np.asarray(m, dtype=np.int64)
    assert np.all((got >= 0) & (got <= m)), f"{what}: a representative outside [0, m]"
    np.testing.assert_array_equal(got % m, np.asarray(want).astype(np.int64) % m, err_msg=what)


def P(a: np.ndarray) -> ctypes.c_void_p:
    return a.ctypes.data_as(ctypes.c_void_p)


class Oracle:
    def __init__(self, lib: ctypes.CDLL):
        self.lib = lib
        lib.orc_hash_f64.restype = ctypes.c_uint64
        lib.orc_gemm_i8.restype = ctypes.c_int64
        lib.orc_modround.restype = ctypes.c_float
        lib.orc_modround.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_float]
        lib.orc_oz1_gemm_diag.restype = ctypes.c_int64
        lib.orc_oz1_int8_gemm.restype = ctypes.c_int64
        lib.orc_check_tf_mul_r_forms.restype = ctypes.c_int64
        lib.orc_check_tf_mul_r_forms.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int,
                                                 ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int64)]

    def inputs(self, seed, phi, na, nb):
        a = np.empty(na)
        b = np.empty(nb)
        self.lib.orc_inputs(ctypes.c_uint(seed), ctypes.c_double(phi), ctypes.c_size_t(na), ctypes.c_size_t(nb), P(a), P(b))
        return a, b

    def hash(self, c) -> int:
        c = np.ascontiguousarray(c, dtype=np.float64).reshape(-1)
        return int(self.lib.orc_hash_f64(P(c), ctypes.c_size_t(c.size)))

    def scale(self, X, rows, cols, mode, ceil_mode, shift):
        X = np.ascontiguousarray(X, dtype=np.float64)
        n = rows if mode == 0 else cols
        d = np.empty(n, dtype=np.int32)
        fl = np.zeros(1, dtype=np.uint32)
        self.lib.orc_scale(P(X), rows, cols, cols, mode, ceil_mode, shift, P(d), P(fl))
        return d, int(fl[0])

    def split_f64(self, x: float, d: int):
        u = np.frombuffer(np.float64(x).tobytes(), dtype=np.uint64)[0]
        out = np.zeros(4, dtype=np.uint32)
        self.lib.orc_split_f64(ctypes.c_uint32(int(u >> np.uint64(32))), ctypes.c_uint32(int(u & np.uint64(0xFFFFFFFF))),
                               ctypes.c_int32(d), P(out))
        return out

    def load_triple(self, x: float, d: int):
        out = np.zeros(3, dtype=np.float32)
        self.lib.orc_load_triple(ctypes.c_double(x), ctypes.c_int32(d), P(out))
        return out

    def digits(self, X, rows, cols, mode, delta, nd):
        X = np.ascontiguousarray(X, dtype=np.float64)
        out = np.empty(rows * cols * nd, dtype=np.float32)
        self.lib.orc_oz2_digits(P(X), rows, cols, cols, mode, P(np.ascontiguousarray(delta, np.int32)), nd, P(out))
        return out.reshape(rows, cols, nd)

    def residues(self, X, rows, cols, mode, delta, nd, moduli):
        """Symmetric residues of A' for INT8 moduli (<= 255), int8, shape (S, rows, cols); moduli above 255
        (the digit routes) come back as int16."""
        X = np.ascontiguousarray(X, dtype=np.float64)
        m = np.array(moduli, dtype=np.int32)
        wide = int(m.max()) > 255
        out = np.empty((len(moduli), rows, cols), dtype=np.int16 if wide else np.int8)
        fn = self.lib.orc_oz2_residues16 if wide else self.lib.orc_oz2_residues
        fn(P(X), rows, cols, cols, mode, P(np.ascontiguousarray(delta, np.int32)), nd, len(moduli), P(m), P(out))
        return out

    def digit_planes(self, X, rows, cols, mode, delta, nd, moduli, q, xmode):
        """FP8-route digit planes (l, h[, s] per modulus) as int8 values, shape (planes, rows, cols)."""
        X = np.ascontiguousarray(X, dtype=np.float64)
        m = np.array(moduli, dtype=np.int32)
        qa = np.array(q, dtype=np.int32)
        xa = np.array(xmode, dtype=np.int32)
        n = int(sum(3 if x == 1 else (1 if x == 3 else 2) for x in xmode))
        out = np.empty((n, rows, cols), dtype=np.int8)
        self.lib.orc_oz2_digit_planes(P(X), rows, cols, cols, mode, P(np.ascontiguousarray(delta, np.int32)), nd,
                                      len(moduli), P(m), P(qa), P(xa), P(out))
        return out

    def modround(self, d, m, rinv) -> float:
        return float(self.lib.orc_modround(d, m, rinv))

    def gemm_i8(self, A, B):
        M, K = A.shape
        K2, N = B.shape
        assert K == K2
        C = np.empty((M, N), dtype=np.int32)
        mx = self.lib.orc_gemm_i8(P(np.ascontiguousarray(A)), P(np.ascontiguousarray(B)), P(C), M, N, K)
        return C, int(mx)

    def crt_ref(self, C, M, N, moduli, b, nd, two_pass, dA, dB):
        m = np.array(moduli, dtype=np.int32)
        out = np.empty(M * N)
        self.lib.orc_oz2_crt_ref(P(np.ascontiguousarray(C, np.int32)), M, N, len(moduli), P(m), b, nd, int(two_pass),
                                 P(np.ascontiguousarray(dA, np.int32)), P(np.ascontiguousarray(dB, np.int32)), P(out))
        return out

    def crt_exact(self, C, M, N, moduli, b, nd, dA, dB):
        m = np.array(moduli, dtype=np.int32)
        out = np.empty(M * N)
        self.lib.orc_oz2_crt_exact(P(np.ascontiguousarray(C, np.int32)), M, N, len(moduli), P(m), b, nd,
                                   P(np.ascontiguousarray(dA, np.int32)), P(np.ascontiguousarray(dB, np.int32)), P(out))
        return out

    def crt_exact_int(self, r, moduli) -> int:
        r = np.ascontiguousarray(r, np.int32)
        m = np.array(moduli, dtype=np.int32)
        out = np.zeros(4, dtype=np.uint64)
        self.lib.orc_oz2_crt_exact_int(P(r), len(moduli), P(m), P(out))
        v = sum(int(out[i]) << (64 * i) for i in range(4))
        return v - (1 << 256) if v >> 255 else v

    def quad_sample(self, A, B, M, N, K, rows, cols):
        rows = np.ascontiguousarray(rows, np.int32)
        cols = np.ascontiguousarray(cols, np.int32)
        out = np.empty(rows.size)
        self.lib.orc_gemm_quad_sample(P(np.ascontiguousarray(A)), P(np.ascontiguousarray(B)), M, N, K, rows.size, P(rows),
                                      P(cols), P(out))
        return out

    def dot2(self, A, B, M, N, K, r0, r1):
        hi = np.empty(M * N)
        lo = np.empty(M * N)
        self.lib.orc_dot2_gemm(P(np.ascontiguousarray(A)), P(np.ascontiguousarray(B)), M, N, K, r0, r1, P(hi), P(lo))
        return hi, lo


def _oz1_slices(self, X, rows, cols, mode, delta, p, radix, dmax):
    """Scheme I digit planes [p][rows][cols] (int8)."""
    X = np.ascontiguousarray(X, dtype=np.float64)
    out = np.empty((p, rows, cols), dtype=np.int8)
    self.lib.orc_oz1_slices(P(X), rows, cols, cols, mode, P(np.ascontiguousarray(delta, dtype=np.int32)), p, radix,
                            dmax, P(out))
    return out


def _oz1_gemm_diag(self, A, B, ndiag):
    """A: [p][M][K] int8, B: [p][K][N] int8 -> P_d [ndiag][M][N] int32 (and the largest |P|)."""
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    p, M, K = A.shape
    N = B.shape[2]
    out = np.empty((ndiag, M, N), dtype=np.int32)
    big = self.lib.orc_oz1_gemm_diag(P(A), P(B), P(out), M, N, K, p, ndiag)
    return out, int(big)


def _oz1_recon(self, Pd, radix, signmag, nsingle, dA, dB):
    Pd = np.ascontiguousarray(Pd, dtype=np.int32)
    ndiag, M, N = Pd.shape
    out = np.empty(M * N)
    self.lib.orc_oz1_recon(P(Pd), M, N, ndiag, radix, signmag, nsingle, P(np.ascontiguousarray(dA, dtype=np.int32)),
                           P(np.ascontiguousarray(dB, dtype=np.int32)), P(out))
    return out


def _oz1_recon_blocks(self, Pb, radix, dA, dB):
    """Block-by-block reconstruction: Pb [nkb][ndiag][M][N] int32 -> C (M*N)."""
    Pb = np.ascontiguousarray(Pb, dtype=np.int32)
    nkb, ndiag, M, N = Pb.shape
    out = np.empty(M * N)
    self.lib.orc_oz1_recon_blocks(P(Pb), M, N, ndiag, nkb, radix, P(np.ascontiguousarray(dA, dtype=np.int32)),
                                  P(np.ascontiguousarray(dB, dtype=np.int32)), P(out))
    return out


def _oz1_scale_w(self, radix, L):
    whi, wlo, qw = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_int32()
    self.lib.orc_oz1_scale_w(radix, L, ctypes.byref(whi), ctypes.byref(wlo), ctypes.byref(qw))
    return whi.value, wlo.value, qw.value


def _oz1_int8_gemm(self, A, B, M, N, K, p):
    A = np.ascontiguousarray(A, dtype=np.float64)
    B = np.ascontiguousarray(B, dtype=np.float64)
    out = np.empty(M * N)
    big = self.lib.orc_oz1_int8_gemm(P(A), P(B), M, N, K, p, P(out))
    return out, int(big)


Oracle.oz1_slices = _oz1_slices
Oracle.oz1_gemm_diag = _oz1_gemm_diag
Oracle.oz1_recon = _oz1_recon
Oracle.oz1_recon_blocks = _oz1_recon_blocks
Oracle.oz1_scale_w = _oz1_scale_w
Oracle.oz1_int8_gemm = _oz1_int8_gemm


def load_oracle() -> Oracle:
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
        _lib = Oracle(ctypes.CDLL(str(ORACLE_SO)))
    return _lib
