"""Thin Python access to the C ABI of include/oz_hip.h (liboz_hip.so): a device handle, device
buffers and the stage entry points, for tests and the evaluator. Every call checks the status and
raises RuntimeError with the device layer's message."""
from __future__ import annotations

import ctypes

import numpy as np

from . import hip

OZ2_MAXS = 24


class ModuliDesc(ctypes.Structure):
    _fields_ = [("S", ctypes.c_int), ("nd", ctypes.c_int), ("m", ctypes.c_float * OZ2_MAXS),
                ("rinv", ctypes.c_float * OZ2_MAXS), ("c", (ctypes.c_float * OZ2_MAXS) * 4)]


class Oz1ReconDesc(ctypes.Structure):
    _fields_ = [("ndiag", ctypes.c_int), ("radix", ctypes.c_int), ("signmag", ctypes.c_int), ("nsingle", ctypes.c_int),
                ("Whi", ctypes.c_uint32), ("Wlo", ctypes.c_uint32), ("qw", ctypes.c_int32)]


class CrtDesc(ctypes.Structure):
    _fields_ = [("S", ctypes.c_int), ("b", ctypes.c_int), ("shift", ctypes.c_int), ("nw", ctypes.c_int),
                ("m", ctypes.c_uint32 * OZ2_MAXS), ("y", ctypes.c_uint32 * OZ2_MAXS),
                ("Q", (ctypes.c_uint32 * 8) * OZ2_MAXS), ("Mw", ctypes.c_uint32 * 8), ("Mtop", ctypes.c_double)]


OZ2_MAXPLANES = 72
OZ2_MAXOUT = 96


class DigitDesc(ctypes.Structure):
    _fields_ = [("mo", ModuliDesc), ("xmode", ctypes.c_int * OZ2_MAXS), ("q", ctypes.c_float * OZ2_MAXS),
                ("qinv", ctypes.c_float * OZ2_MAXS), ("encoding", ctypes.c_int)]


class GroupDesc(ctypes.Structure):
    _fields_ = [("npairs", ctypes.c_int), ("modulus", ctypes.c_int), ("a", ctypes.c_ubyte * 4),
                ("b", ctypes.c_ubyte * 4), ("m", ctypes.c_uint32), ("coef", ctypes.c_uint32), ("bound", ctypes.c_float)]


class GroupsDesc(ctypes.Structure):
    _fields_ = [("nout", ctypes.c_int), ("nplanes", ctypes.c_int), ("g", GroupDesc * OZ2_MAXOUT)]


# OCP e4m3 (the gfx950 FP8 format): byte -> value
def _e4m3_table() -> np.ndarray:
    t = np.zeros(256)
    for u in range(256):
        s, e, f = u >> 7, (u >> 3) & 15, u & 7
        v = (f / 8.0) * 2.0 ** -6 if e == 0 else (1 + f / 8.0) * 2.0 ** (e - 7)
        t[u] = -v if s else v
    t[0x7F] = t[0xFF] = np.nan
    return t


E4M3 = _e4m3_table()


def moduli_desc(moduli, nd: int) -> ModuliDesc:
    d = ModuliDesc()
    d.S, d.nd = len(moduli), nd
    for s, m in enumerate(moduli):
        d.m[s] = float(m)
        d.rinv[s] = float(np.float32(1.0 / m))
        for j in range(4):
            d.c[j][s] = float(pow(2, 20 * (j + 1), m))
    return d


def crt_desc(moduli, b: int, nd: int) -> CrtDesc:
    d = CrtDesc()
    S = len(moduli)
    M = 1
    for m in moduli:
        M *= m
    d.S, d.b, d.shift = S, b, b - 20 * (nd - 1)
    bits = ((S + 1) * M).bit_length() + 1
    d.nw = max(3, (bits + 31) // 32)
    for w in range(8):
        d.Mw[w] = (M >> (32 * w)) & 0xFFFFFFFF
    d.Mtop = float(M)
    for s, m in enumerate(moduli):
        d.m[s] = m
        Q = M // m
        for w in range(8):
            d.Q[s][w] = (Q >> (32 * w)) & 0xFFFFFFFF
        d.y[s] = pow(Q % m, -1, m)
    return d


class Buffer:
    def __init__(self, dev: "Device", nbytes: int):
        self.dev, self.nbytes = dev, int(nbytes)
        self.ptr = ctypes.c_void_p()
        dev._check(hip().oz_dev_malloc(dev.h, ctypes.c_size_t(max(self.nbytes, 1)), ctypes.byref(self.ptr)),
                   "oz_dev_malloc")

    def free(self):
        if self.ptr:
            hip().oz_dev_free(self.dev.h, self.ptr)
            self.ptr = ctypes.c_void_p()

    def offset(self, nbytes: int) -> ctypes.c_void_p:
        return ctypes.c_void_p(self.ptr.value + int(nbytes))


class Device:
    def __init__(self, device_id: int = 0):
        self.h = ctypes.c_void_p()
        st = hip().oz_dev_open(device_id, ctypes.byref(self.h))
        if st != 0:
            raise RuntimeError(f"oz_dev_open({device_id}) failed with status {st}")
        self.bufs: list[Buffer] = []

    def _check(self, st: int, what: str):
        if st != 0:
            raise RuntimeError(f"{what}: status {st}: {hip().oz_last_error(self.h).decode(errors='replace')}")

    def close(self):
        for b in self.bufs:
            b.free()
        self.bufs.clear()
        if self.h:
            hip().oz_dev_close(self.h)
            self.h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def alloc(self, nbytes: int) -> Buffer:
        b = Buffer(self, nbytes)
        self.bufs.append(b)
        return b

    def upload(self, arr: np.ndarray) -> Buffer:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes)
        self._check(hip().oz_memcpy_h2d(self.h, b.ptr, arr.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(arr.nbytes)),
                    "oz_memcpy_h2d")
        return b

    def download(self, buf: Buffer, dtype, count: int, offset_bytes: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        src = buf.offset(offset_bytes)
        self._check(hip().oz_memcpy_d2h(self.h, out.ctypes.data_as(ctypes.c_void_p), src, ctypes.c_size_t(out.nbytes)),
                    "oz_memcpy_d2h")
        return out

    def fill_u32(self, buf: Buffer, value: int, count: int):
        self._check(hip().oz_fill_u32(self.h, buf.ptr, ctypes.c_uint32(value), ctypes.c_size_t(count)), "oz_fill_u32")

    def copy(self, dst: Buffer, src: Buffer, nbytes: int):
        self._check(hip().oz_memcpy_d2d(self.h, dst.ptr, src.ptr, ctypes.c_size_t(nbytes)), "oz_memcpy_d2d")

    def sync(self):
        self._check(hip().oz_sync(self.h), "oz_sync")

    # ---- timing --------------------------------------------------------------------------------
    def event_record(self, slot: int):
        self._check(hip().oz_event_record(self.h, slot), "oz_event_record")

    def elapsed_ms(self, begin: int, end: int) -> float:
        ms = ctypes.c_float()
        self._check(hip().oz_event_elapsed_ms(self.h, begin, end, ctypes.byref(ms)), "oz_event_elapsed_ms")
        return ms.value

    def time_products_begin(self, begin: int, end: int):
        self._check(hip().oz_time_products_begin(self.h, begin, end), "oz_time_products_begin")

    def time_products_end(self) -> bool:
        """Ends the request; True if a product kernel ran under it."""
        launched = ctypes.c_int()
        self._check(hip().oz_time_products_end(self.h, ctypes.byref(launched)), "oz_time_products_end")
        return bool(launched.value)

    # ---- stages --------------------------------------------------------------------------------
    def scale(self, X: Buffer, rows, cols, ld, mode, ceil_mode, shift, delta: Buffer, flags: Buffer, flag_index=0):
        self._check(hip().oz_scale_f64(self.h, X.ptr, rows, cols, ld, mode, ceil_mode, shift, delta.ptr,
                                       flags.offset(4 * flag_index)), "oz_scale_f64")

    def scale_pair(self, A: Buffer, M, K, lda, B: Buffer, N, ldb, ceil_mode, shift, dA: Buffer, dB: Buffer,
                   flags: Buffer, clear=None):
        """clear: a pointer (ctypes.c_void_p, e.g. Buffer.offset) to two words the launch zeroes, or None."""
        self._check(hip().oz_scale_pair_f64(self.h, A.ptr, M, K, lda, B.ptr, N, ldb, ceil_mode, shift, dA.ptr, dB.ptr,
                                            flags.ptr, clear), "oz_scale_pair_f64")

    def split_pair_int8(self, A: Buffer, M, K, lda, dA: Buffer, B: Buffer, N, ldb, dB: Buffer, desc: ModuliDesc,
                        pA: Buffer, pB: Buffer, Mg, Ng, Kg):
        self._check(hip().oz2_split_pair_int8(self.h, A.ptr, M, K, lda, dA.ptr, B.ptr, N, ldb, dB.ptr,
                                              ctypes.byref(desc), pA.ptr, pB.ptr, Mg, Ng, Kg), "oz2_split_pair_int8")

    def split_int8(self, X: Buffer, rows, cols, ld, mode, delta: Buffer, desc: ModuliDesc, planes: Buffer, layout, prow,
                   pld, pstride):
        self._check(hip().oz2_split_int8(self.h, X.ptr, rows, cols, ld, mode, delta.ptr, ctypes.byref(desc), planes.ptr,
                                         layout, prow, pld, ctypes.c_longlong(pstride)), "oz2_split_int8")

    def digits(self, X: Buffer, rows, cols, ld, mode, delta: Buffer, nd, out: Buffer):
        self._check(hip().oz2_digits_f32(self.h, X.ptr, rows, cols, ld, mode, delta.ptr, nd, out.ptr), "oz2_digits_f32")

    def gemm_i8(self, A: Buffer, Bt: Buffer, C: Buffer, M, N, K, batch, ldc, sA, sB, sC):
        """C[b] = A[b] Bt[b]^T with A, Bt in OZ_BLOCK tiles (see to_blocks)."""
        self._check(hip().oz_gemm_i8(self.h, A.ptr, Bt.ptr, C.ptr, M, N, K, batch, ldc, ctypes.c_longlong(sA),
                                     ctypes.c_longlong(sB), ctypes.c_longlong(sC)), "oz_gemm_i8")

    def gemm_digits(self, A: Buffer, Bt: Buffer, D: Buffer, M, N, K, S, ldd, sA, sB, sD, desc: CrtDesc):
        """D[s] = CRT digits ((A_s Bt_s^T) mod m_s) * y_s mod m_s as uint8 (operands as gemm_i8)."""
        self._check(hip().oz2_gemm_digits(self.h, A.ptr, Bt.ptr, D.ptr, M, N, K, S, ldd, ctypes.c_longlong(sA),
                                          ctypes.c_longlong(sB), ctypes.c_longlong(sD), ctypes.byref(desc)),
                    "oz2_gemm_digits")

    def gemm_f64_workspace(self, M, N, K, S) -> int:
        n = ctypes.c_size_t()
        self._check(hip().oz2_gemm_f64_workspace(M, N, K, S, ctypes.byref(n)), "oz2_gemm_f64_workspace")
        return n.value

    def gemm_f64(self, A: Buffer, lda, B: Buffer, ldb, C: Buffer, ldc, M, N, K, md: ModuliDesc, cd: CrtDesc,
                 flags: Buffer, work: Buffer, work_bytes):
        """The whole Scheme II INT8 pass C = A B on device-resident operands (oz2_gemm_f64)."""
        self._check(hip().oz2_gemm_f64(self.h, A.ptr, lda, B.ptr, ldb, C.ptr, ldc, M, N, K, ctypes.byref(md),
                                       ctypes.byref(cd), flags.ptr, work.ptr, ctypes.c_size_t(work_bytes)),
                    "oz2_gemm_f64")

    def crt_digits(self, D: Buffer, M, N, ldd, sD, desc: CrtDesc, dA: Buffer, dB: Buffer, out: Buffer, ldo):
        self._check(hip().oz2_crt_digits_f64(self.h, D.ptr, M, N, ldd, ctypes.c_longlong(sD), ctypes.byref(desc),
                                             dA.ptr, dB.ptr, out.ptr, ldo), "oz2_crt_digits_f64")

    # ---- scheme I ----
    def oz1_split(self, X: Buffer, rows, cols, ld, mode, delta: Buffer, p, radix, dmax, planes: Buffer, layout, prow,
                  pld, pstride):
        self._check(hip().oz1_split_int8(self.h, X.ptr, rows, cols, ld, mode, delta.ptr, p, radix, dmax, planes.ptr,
                                         layout, prow, pld, ctypes.c_longlong(pstride)), "oz1_split_int8")

    def oz1_split_pair(self, A: Buffer, M, K, lda, dA: Buffer, B: Buffer, N, ldb, dB: Buffer, p, radix, dmax,
                       pA: Buffer, pB: Buffer, Mg, Ng, Kg):
        """oz1_split of A (layout 2, planes Mg x Kg) and of B (layout 3, planes Ng x Kg) in one launch."""
        self._check(hip().oz1_split_pair_int8(self.h, A.ptr, M, K, lda, dA.ptr, B.ptr, N, ldb, dB.ptr, p, radix, dmax,
                                              pA.ptr, pB.ptr, Mg, Ng, Kg), "oz1_split_pair_int8")

    def oz1_gemm_diag(self, A: Buffer, Bt: Buffer, C: Buffer, M, N, K, ndiag, ldc, sA, sB, sC, dmax=127):
        self._check(hip().oz1_gemm_diag_i8(self.h, A.ptr, Bt.ptr, C.ptr, M, N, K, ndiag, dmax, ldc, ctypes.c_longlong(sA),
                                           ctypes.c_longlong(sB), ctypes.c_longlong(sC)), "oz1_gemm_diag_i8")

    def oz1_recon(self, P: Buffer, M, N, ldp, sP, desc: "Oz1ReconDesc", dA: Buffer, dB: Buffer, out: Buffer, ldo):
        self._check(hip().oz1_recon_f64(self.h, P.ptr, M, N, ldp, ctypes.c_longlong(sP), ctypes.byref(desc), dA.ptr,
                                        dB.ptr, out.ptr, ldo), "oz1_recon_f64")

    def split_digits(self, X: Buffer, rows, cols, ld, mode, delta: Buffer, desc: DigitDesc, planes: Buffer, layout,
                     prow, pld, pstride):
        self._check(hip().oz2_split_digits(self.h, X.ptr, rows, cols, ld, mode, delta.ptr, ctypes.byref(desc),
                                              planes.ptr, layout, prow, pld, ctypes.c_longlong(pstride)),
                    "oz2_split_digits")

    def split_digits_pair(self, A: Buffer, M, K, lda, dA: Buffer, B: Buffer, N, ldb, dB: Buffer, desc: DigitDesc,
                          pA: Buffer, pB: Buffer, Mg, Ng, Kg):
        """split_digits of A (layout 2, planes Mg x Kg) and of B (layout 3, planes Ng x Kg) in one launch."""
        self._check(hip().oz2_split_digits_pair(self.h, A.ptr, M, K, lda, dA.ptr, B.ptr, N, ldb, dB.ptr,
                                                ctypes.byref(desc), pA.ptr, pB.ptr, Mg, Ng, Kg), "oz2_split_digits_pair")

    def gemm_groups_f8(self, A: Buffer, Bt: Buffer, out: Buffer, M, N, K, desc: GroupsDesc, kind, ldo, sA, sB, sO):
        self._check(hip().oz2_gemm_groups_f8(self.h, A.ptr, Bt.ptr, out.ptr, M, N, K, ctypes.byref(desc), kind, ldo,
                                                ctypes.c_longlong(sA), ctypes.c_longlong(sB), ctypes.c_longlong(sO)),
                    "oz2_gemm_groups_f8")

    def crt_terms(self, W: Buffer, M, N, ldw, sW, nterms, term_modulus, desc: CrtDesc, dA: Buffer, dB: Buffer,
                  out: Buffer, ldo):
        tm = (ctypes.c_ubyte * OZ2_MAXOUT)(*[int(x) for x in term_modulus])
        self._check(hip().oz2_crt_terms_f64(self.h, W.ptr, M, N, ldw, ctypes.c_longlong(sW), nterms, tm,
                                               ctypes.byref(desc), dA.ptr, dB.ptr, out.ptr, ldo), "oz2_crt_terms_f64")

    def crt(self, C: Buffer, M, N, ldc, sC, desc: CrtDesc, dA: Buffer, dB: Buffer, out: Buffer, ldo):
        self._check(hip().oz2_crt_f64(self.h, C.ptr, M, N, ldc, ctypes.c_longlong(sC), ctypes.byref(desc), dA.ptr,
                                      dB.ptr, out.ptr, ldo), "oz2_crt_f64")



def block_swizzle(r):
    """Chunk swizzle of the OZ_BLOCK tiles: ((r >> 1) ^ (r >> 2)) & 3."""
    return ((r >> 1) ^ (r >> 2)) & 3


def block_offsets(R: int, C: int) -> np.ndarray:
    """Byte offset, in OZ_BLOCK tiles, of every element of a row-major R x C plane (R % 16 == 0,
    C % 64 == 0): block (i, j) of 16 rows x 64 columns at (i*(C/64) + j)*1024, element (r, c) of a
    block at 64*r + 16*((c/16) ^ block_swizzle(r)) + c%16."""
    if R % 16 or C % 64:
        raise ValueError("OZ_BLOCK planes need R % 16 == 0 and C % 64 == 0")
    r = np.arange(R, dtype=np.int64)[:, None]
    c = np.arange(C, dtype=np.int64)[None, :]
    rb, cb = r % 16, c % 64
    return ((r // 16) * (C // 64) + c // 64) * 1024 + 64 * rb + 16 * ((cb // 16) ^ block_swizzle(rb)) + cb % 16


def to_blocks(plane: np.ndarray) -> np.ndarray:
    """Row-major planes (..., R, C) -> the same bytes in OZ_BLOCK tiles, flat per plane (..., R*C)."""
    *lead, R, C = plane.shape
    src = plane.reshape(-1, R * C)
    out = np.empty_like(src)
    out[:, block_offsets(R, C).ravel()] = src
    return out.reshape(*lead, R * C)


def from_blocks(blocks: np.ndarray, R: int, C: int) -> np.ndarray:
    """Inverse of to_blocks: planes in OZ_BLOCK tiles (..., R*C) -> row-major (..., R, C)."""
    src = blocks.reshape(-1, R * C)
    return src[:, block_offsets(R, C).ravel()].reshape(*blocks.shape[:-1], R, C)
