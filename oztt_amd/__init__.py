"""oztt_amd — ozTTgemm for AMD Instinct MI355X (gfx950).

Python mirror of the reference's public C++ interface (reference include/ozTTgemm/ozTTgemm.hpp:21-123):
the same enums, Options, Info and Context.gemm/multiply, with the same validation and error
behaviour (ValueError for std::invalid_argument, RuntimeError for std::runtime_error, MemoryError
for std::bad_alloc). The computation runs in the native libraries built in oztt_amd/lib/:

  libozTTgemm.so  C++20 host library (planning, dispatch, drivers) — the drop-in C++ API
  liboz_hip.so    HIP kernels for gfx950 behind the C ABI of include/oz_hip.h

There is no CPU fallback: without the built libraries every entry point raises.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass
from pathlib import Path

import numpy as np

LIB_DIR = Path(__file__).resolve().parent / "lib"

__all__ = ["Scheme", "Format", "Reconstruction", "Transport", "Options", "Info", "Context", "is_available", "format_name",
           "hip", "host", "LIB_DIR"]


class Scheme(enum.IntEnum):
    I = 0
    II = 1


class Format(enum.IntEnum):
    BF16 = 0
    FP16 = 1
    TF32 = 2
    BFP8 = 3
    FP8 = 4
    INT8 = 5
    BFP4 = 6
    BFP2 = 7


class Reconstruction(enum.IntEnum):
    Automatic = 0
    OnePass = 1
    TwoPass = 2


class Transport(enum.IntEnum):
    """Scheme II (extension of the reference's Options): Automatic runs INT8 and FP8 on their own matrix
    instructions (FP8: the reference's e4m3 digits) and the other formats' plans on INT8 residues;
    Int8Residues carries every format's plan by INT8 residues at its width (the same C)."""
    Automatic = 0
    Int8Residues = 1


@dataclass
class Options:
    scheme: Scheme = Scheme.II
    format: Format = Format.BFP8
    slices: int = 0
    max_moduli: int = 0
    reconstruction: Reconstruction = Reconstruction.Automatic
    transport: Transport = Transport.Automatic


@dataclass
class Info:
    scheme: Scheme
    format: Format
    slices: int
    moduli: int
    integer_bits: int
    reconstruction_passes: int
    padded_m: int
    padded_n: int
    padded_k: int


class _Info(ctypes.Structure):
    _fields_ = [("scheme", ctypes.c_int), ("format", ctypes.c_int), ("slices", ctypes.c_uint),
                ("moduli", ctypes.c_uint), ("integer_bits", ctypes.c_uint),
                ("reconstruction_passes", ctypes.c_uint), ("padded_m", ctypes.c_ulonglong),
                ("padded_n", ctypes.c_ulonglong), ("padded_k", ctypes.c_ulonglong)]


class EvalStats(ctypes.Structure):
    _fields_ = [("fixed_bits", ctypes.c_uint), ("warmup", ctypes.c_int), ("repeats", ctypes.c_int),
                ("phase_ms", ctypes.c_double * 5), ("whole_ms", ctypes.c_double), ("whole_checked", ctypes.c_int),
                ("partial_products", ctypes.c_uint), ("product_ops", ctypes.c_double),
                ("gemm_launch_ms", ctypes.c_double), ("gemm_launches", ctypes.c_int),
                ("max_band_rows", ctypes.c_uint), ("plan_reused", ctypes.c_int), ("force_kc", ctypes.c_uint),
                ("replay_drop_phase", ctypes.c_int), ("whole_sentinel", ctypes.c_int),
                ("whole_steps", ctypes.c_uint * 5), ("expected_steps", ctypes.c_uint * 5),
                ("fp8_matrix_cores", ctypes.c_int), ("full_window", ctypes.c_int)]

    def __init__(self, *args, **kw):
        super().__init__(*args, **kw)
        if "replay_drop_phase" not in kw:
            self.replay_drop_phase = -1


class Plan2(ctypes.Structure):
    _fields_ = [("ok", ctypes.c_int), ("b", ctypes.c_int), ("S", ctypes.c_int), ("nd", ctypes.c_int),
                ("two_pass", ctypes.c_int), ("m_cap", ctypes.c_int), ("m", ctypes.c_int * 24),
                ("log2M", ctypes.c_double), ("recon1_log2", ctypes.c_double), ("TA", ctypes.c_double),
                ("TB", ctypes.c_double), ("nA", ctypes.c_double), ("nB", ctypes.c_double), ("nC", ctypes.c_double),
                ("wA", ctypes.c_double), ("wB", ctypes.c_double), ("b_cap", ctypes.c_int),
                ("rS", ctypes.c_int), ("rsparse", ctypes.c_int), ("rfold_first", ctypes.c_int), ("rmaxg", ctypes.c_int),
                ("rnprod", ctypes.c_int), ("rnplane", ctypes.c_int), ("rnout", ctypes.c_int),
                ("rm", ctypes.c_int * 24), ("rmode", ctypes.c_int * 24), ("rmaxg_m", ctypes.c_int * 24),
                ("rlog2M", ctypes.c_double), ("fp8_digits", ctypes.c_int), ("rmodel_set", ctypes.c_int),
                ("bound_log2", ctypes.c_double), ("S_window", ctypes.c_int), ("nprod", ctypes.c_int),
                ("nplane", ctypes.c_int)]


class Plan1(ctypes.Structure):
    _fields_ = [("p", ctypes.c_int), ("pmax", ctypes.c_int), ("nsmall", ctypes.c_int), ("Kc", ctypes.c_uint),
                ("nkb", ctypes.c_uint), ("pairloop", ctypes.c_int), ("pairwise", ctypes.c_int), ("fuse", ctypes.c_int),
                ("defer", ctypes.c_int), ("Whi", ctypes.c_uint), ("Wlo", ctypes.c_uint), ("qw", ctypes.c_int),
                ("bits_indep", ctypes.c_double), ("bits_sampled", ctypes.c_double)]


_host = None
_hip = None


def _load(name: str) -> ctypes.CDLL:
    path = LIB_DIR / name
    if not path.exists():
        raise RuntimeError(f"{path} is missing: build the native libraries first (python __graft_entry__.py build "
                           f"or python -c 'import __graft_entry__ as g; g.build()')")
    return ctypes.CDLL(str(path), mode=ctypes.RTLD_GLOBAL)


def hip() -> ctypes.CDLL:
    """The C ABI of include/oz_hip.h (liboz_hip.so)."""
    global _hip
    if _hip is None:
        _hip = _load("liboz_hip.so")
        _hip.oz_last_error.restype = ctypes.c_char_p
    return _hip


def host() -> ctypes.CDLL:
    """The C entry points of libozTTgemm.so."""
    global _host
    if _host is None:
        hip()
        h = _load("libozTTgemm.so")
        h.ozt_format_name.restype = ctypes.c_char_p
        h.ozt_eval_hash.restype = ctypes.c_ulonglong
        h.ozt_matrix_new.restype = ctypes.c_void_p
        _host = h
    return _host


def is_available(fmt: Format) -> bool:
    return bool(host().ozt_is_available(int(fmt)))


def format_name(fmt: Format) -> str:
    return host().ozt_format_name(int(fmt)).decode()


_ERRORS = {1: ValueError, 2: RuntimeError, 3: MemoryError, 4: RuntimeError}


def _raise(code: int, err: ctypes.Array) -> None:
    if code:
        raise _ERRORS.get(code, RuntimeError)(err.value.decode(errors="replace"))


def _f64(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float64).reshape(-1)


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return a.ctypes.data_as(ctypes.c_void_p)


class Matrix:
    """A matrix kept on the GPU of a Context between calls (ozTTgemm::Matrix, an extension of the
    reference's interface). Made by Context.upload, or filled as the result of Context.gemm_resident
    (pass an empty Matrix() as c)."""

    def __init__(self):
        self._m = ctypes.c_void_p(host().ozt_matrix_new())
        if not self._m:
            raise MemoryError("ozt_matrix_new")

    @property
    def shape(self) -> tuple[int, int]:
        r, c = ctypes.c_size_t(), ctypes.c_size_t()
        host().ozt_matrix_dims(self._m, ctypes.byref(r), ctypes.byref(c))
        return r.value, c.value

    def close(self) -> None:
        if self._m:
            host().ozt_matrix_free(self._m)
            self._m = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Context:
    """Owns one GPU (opened lazily by the first valid GEMM), like ozTTgemm::Context."""

    def __init__(self, device_id: int = 0, kernel_directory: str = ""):
        self._ctx = ctypes.c_void_p()
        err = ctypes.create_string_buffer(1024)
        kd = kernel_directory.encode() if kernel_directory else None
        _raise(host().ozt_context_new(int(device_id), kd, ctypes.byref(self._ctx), err, ctypes.c_size_t(1024)), err)

    def close(self) -> None:
        if self._ctx:
            host().ozt_context_free(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _call(self, a, b, c, m, n, k, options: Options, evaluation: EvalStats | None = None) -> Info:
        err = ctypes.create_string_buffer(4096)
        info = _Info()
        o = options
        args = [self._ctx, _ptr(a), ctypes.c_size_t(a.size), _ptr(b), ctypes.c_size_t(b.size), _ptr(c),
                ctypes.c_size_t(c.size), ctypes.c_size_t(m), ctypes.c_size_t(n), ctypes.c_size_t(k), int(o.scheme),
                int(o.format), ctypes.c_uint(o.slices), ctypes.c_uint(o.max_moduli), int(o.reconstruction),
                int(o.transport),
                ctypes.byref(info)]
        if evaluation is None:
            code = host().ozt_gemm(*args, err, ctypes.c_size_t(4096))
        else:
            code = host().ozt_eval_gemm(*args, ctypes.byref(evaluation), err, ctypes.c_size_t(4096))
        _raise(code, err)
        return Info(Scheme(info.scheme), Format(info.format), info.slices, info.moduli, info.integer_bits,
                    info.reconstruction_passes, info.padded_m, info.padded_n, info.padded_k)

    def gemm(self, a, b, c: np.ndarray, m: int, n: int, k: int, options: Options | None = None) -> Info:
        """C = A*B into the float64 array c (m*n elements, contiguous); returns Info."""
        if not (isinstance(c, np.ndarray) and c.dtype == np.float64 and c.flags.c_contiguous):
            raise ValueError("c must be a contiguous float64 numpy array")
        return self._call(_f64(a), _f64(b), c.reshape(-1), m, n, k, options or Options())

    def multiply(self, a, b, m: int, n: int, k: int, options: Options | None = None) -> np.ndarray:
        a, b = _f64(a), _f64(b)
        if a.size != m * k or b.size != k * n:
            raise ValueError("matrix span sizes do not match m, n, k")
        c = np.empty(m * n, dtype=np.float64)
        self.gemm(a, b, c, m, n, k, options)
        return c

    def evaluate(self, a, b, m: int, n: int, k: int, options: Options, fixed_bits: int = 0, warmup: int = 0,
                 repeats: int = 0, max_band_rows: int = 0, force_kc: int = 0, replay_drop_phase: int = -1,
                 fp8_matrix_cores: bool = False, full_window: bool = False):
        """GEMM under the evaluation hooks: returns (C, Info, EvalStats) with phase and whole-pass times.
        max_band_rows > 0 caps the rows of a band (row bands are otherwise used only when the problem
        does not fit in device memory); force_kc > 0 makes Scheme I with an FP32-product format
        reconstruct K block by K block with blocks of that length. replay_drop_phase >= 0 is the
        self-test of the whole-pass check: its checking replay leaves out that phase's steps, so
        whole_checked must be 0, and nothing is timed. fp8_matrix_cores runs Scheme II FP8 as the FP8
        route's e4m3 digit products on the FP8 matrix cores also under Transport.Int8Residues.
        full_window makes Scheme II INT8 residues compute with the set for the window K 2^(2b) rather
        than the smaller set the operands' own bound on |C'| allows (the same C)."""
        a, b = _f64(a), _f64(b)
        c = np.empty(m * n, dtype=np.float64)
        ev = EvalStats()
        ev.fixed_bits, ev.warmup, ev.repeats = fixed_bits, warmup, repeats
        ev.max_band_rows = max_band_rows
        ev.force_kc = force_kc
        ev.replay_drop_phase = replay_drop_phase
        ev.fp8_matrix_cores = int(bool(fp8_matrix_cores))
        ev.full_window = int(bool(full_window))
        info = self._call(a, b, c, m, n, k, options, ev)
        return c, info, ev


    # ---- resident operands (extension) --------------------------------------------------------
    def upload(self, x, rows: int, cols: int) -> Matrix:
        """Copies the row-major rows x cols float64 matrix x to the GPU (Context::upload)."""
        x = _f64(x)
        m = Matrix()
        err = ctypes.create_string_buffer(2048)
        _raise(host().ozt_upload(self._ctx, _ptr(x), ctypes.c_size_t(x.size), ctypes.c_size_t(rows),
                                 ctypes.c_size_t(cols), m._m, err, ctypes.c_size_t(2048)), err)
        return m

    def download(self, m: Matrix) -> np.ndarray:
        rows, cols = m.shape
        out = np.empty(rows * cols, dtype=np.float64)
        err = ctypes.create_string_buffer(2048)
        _raise(host().ozt_download(self._ctx, m._m, _ptr(out), ctypes.c_size_t(out.size), err,
                                   ctypes.c_size_t(2048)), err)
        return out

    def gemm_resident(self, a: Matrix, b: Matrix, c, options: Options | None = None,
                      evaluation: EvalStats | None = None) -> Info:
        """C = A*B for resident a, b (Context::gemm on Matrix operands): c is a contiguous float64 array
        of m*n elements (C read back) or a Matrix (C stays on the GPU; an empty Matrix() receives it).
        With an EvalStats the call runs under the evaluation hooks."""
        o = options or Options()
        err = ctypes.create_string_buffer(4096)
        info = _Info()
        if isinstance(c, Matrix):
            cptr, nc, cm = ctypes.c_void_p(), 0, c._m
        else:
            if not (isinstance(c, np.ndarray) and c.dtype == np.float64 and c.flags.c_contiguous):
                raise ValueError("c must be a Matrix or a contiguous float64 numpy array")
            cptr, nc, cm = _ptr(c), c.size, ctypes.c_void_p()
        _raise(host().ozt_gemm_resident(self._ctx, a._m, b._m, cptr, ctypes.c_size_t(nc), cm, int(o.scheme),
                                        int(o.format), ctypes.c_uint(o.slices), ctypes.c_uint(o.max_moduli),
                                        int(o.reconstruction), int(o.transport), ctypes.byref(info),
                                        ctypes.byref(evaluation) if evaluation is not None else None, err,
                                        ctypes.c_size_t(4096)), err)
        return Info(Scheme(info.scheme), Format(info.format), info.slices, info.moduli, info.integer_bits,
                    info.reconstruction_passes, info.padded_m, info.padded_n, info.padded_k)


def plan2(a, b, M: int, N: int, K: int, fmt: Format = Format.INT8, max_moduli: int = 0,
          reconstruction: Reconstruction = Reconstruction.Automatic, fixed_bits: int = 0,
          transport: Transport = Transport.Automatic, fp8_matrix_cores: bool = False,
          full_window: bool = False) -> Plan2:
    """Scheme II planner on padded row-major A (M x K) and B (K x N): the execution set (m, S, b, ...;
    fp8_digits when it is the FP8 route's digit set) and the route's plan of the format (rm, rS, rmode, ...).
    INT8 residues compute with the smallest set that covers the operands' bound on |C'| (bound_log2;
    S_window > 0 is the size of the set for the window K 2^(2b) that it replaced); full_window keeps
    that set, as the evaluation setting does. fp8_matrix_cores as the evaluation setting (FP8 keeps its
    digits also under Int8Residues)."""
    a, b = _f64(a), _f64(b)
    out = Plan2()
    err = ctypes.create_string_buffer(2048)
    int8_transport = transport == Transport.Int8Residues and not fp8_matrix_cores
    _raise(host().ozt_plan_scheme2(_ptr(a), _ptr(b), M, N, K, int(fmt), max_moduli, int(reconstruction), fixed_bits,
                                   int(int8_transport), int(bool(full_window)), ctypes.byref(out), err,
                                   ctypes.c_size_t(2048)), err)
    return out


def plan2_fp8_device(a, b, M: int, N: int, K: int, max_moduli: int = 0,
                     reconstruction: Reconstruction = Reconstruction.Automatic, fixed_bits: int = 0,
                     execution_set: bool = False):
    """Device descriptors of the Scheme II FP8 plan: (DigitDesc, GroupsDesc, CrtDesc, term moduli), for the
    route's own set, or with execution_set for the set the public call computes with."""
    from .device import CrtDesc, DigitDesc, GroupsDesc, OZ2_MAXOUT
    a, b = _f64(a), _f64(b)
    dd, gd, crt = DigitDesc(), GroupsDesc(), CrtDesc()
    tm = (ctypes.c_ubyte * OZ2_MAXOUT)()
    err = ctypes.create_string_buffer(2048)
    _raise(host().ozt_plan2_fp8_device(_ptr(a), _ptr(b), M, N, K, max_moduli, int(reconstruction), fixed_bits,
                                       int(bool(execution_set)), ctypes.byref(dd), ctypes.byref(gd), ctypes.byref(crt),
                                       tm, err, ctypes.c_size_t(2048)), err)
    return dd, gd, crt, [tm[i] for i in range(gd.nout)]


def plan2_int8(a, b, M: int, N: int, K: int, max_moduli: int = 0,
               reconstruction: Reconstruction = Reconstruction.Automatic, fixed_bits: int = 0) -> Plan2:
    """Scheme II INT8 planner on padded row-major A (M x K) and B (K x N)."""
    return plan2(a, b, M, N, K, Format.INT8, max_moduli, reconstruction, fixed_bits)


def choose_moduli_fp8(K: int, num_moduli: int, b_cap: int, window_log2: float = 0.0) -> Plan2:
    """FP8-route moduli selection (route fields r*); window_log2 > 0 replaces the CRT window log2 K."""
    out = Plan2()
    host().ozt_choose_moduli_fp8(K, num_moduli, b_cap, ctypes.c_double(window_log2), ctypes.byref(out))
    return out


def plan1(a, b, M: int, N: int, K: int, slices: int = 0, fmt: Format = Format.INT8) -> Plan1:
    """Scheme I planner (slices, issue, reconstruction constants) on padded row-major A (M x K), B (K x N)."""
    a, b = _f64(a), _f64(b)
    out = Plan1()
    err = ctypes.create_string_buffer(2048)
    _raise(host().ozt_plan1(_ptr(a), _ptr(b), M, N, K, slices, int(fmt), ctypes.byref(out), err,
                            ctypes.c_size_t(2048)), err)
    return out


def choose_moduli_int8(K: int, num_moduli: int, b_cap: int) -> Plan2:
    out = Plan2()
    host().ozt_choose_moduli_int8(K, num_moduli, b_cap, ctypes.byref(out))
    return out


def choose_moduli_route(fmt: Format, M: int, N: int, K: int, num_moduli: int, b_cap: int) -> Plan2:
    """Moduli selection on the digit route of a format other than INT8 (route fields r*; rmodel_set when the
    stage-time model chose the set). M and N feed only the model's memory estimate."""
    out = Plan2()
    err = ctypes.create_string_buffer(2048)
    _raise(host().ozt_choose_moduli_route(int(fmt), M, N, K, num_moduli, b_cap, ctypes.c_double(0.0),
                                          ctypes.byref(out), err, ctypes.c_size_t(2048)), err)
    return out


def eval_inputs(seed: int, phi: float, na: int, nb: int):
    """Evaluator inputs (reference evaluation/numerics.hpp:19-38 with a seed): A then B, float64."""
    a = np.empty(na, dtype=np.float64)
    b = np.empty(nb, dtype=np.float64)
    host().ozt_eval_inputs(ctypes.c_uint(seed), ctypes.c_double(phi), ctypes.c_size_t(na), ctypes.c_size_t(nb),
                           _ptr(a), _ptr(b))
    return a, b


def eval_hash(c) -> int:
    c = _f64(c)
    return int(host().ozt_eval_hash(_ptr(c), ctypes.c_size_t(c.size)))


def eval_reference_gemm(a, b, M: int, K: int, N: int, r0: int = 0, r1: int | None = None):
    """Dot2 reference GEMM of the evaluator (numerics.hpp:58-93) for rows [r0, r1): (hi, lo), each (r1-r0)*N."""
    a, b = _f64(a), _f64(b)
    r1 = M if r1 is None else min(r1, M)
    hi = np.empty((r1 - r0) * N)
    lo = np.empty((r1 - r0) * N)
    host().ozt_eval_reference_gemm(_ptr(a), _ptr(b), M, K, N, r0, r1, _ptr(hi), _ptr(lo))
    return hi, lo


def eval_accuracy(c, hi, lo):
    """(relative Frobenius error, effective bits) of C against the Dot2 reference (numerics.hpp:98-127)."""
    c, hi, lo = _f64(c), _f64(hi), _f64(lo)
    rel, eb = ctypes.c_double(), ctypes.c_double()
    host().ozt_eval_accuracy(_ptr(c), _ptr(hi), _ptr(lo), ctypes.c_size_t(c.size), ctypes.byref(rel), ctypes.byref(eb))
    return rel.value, eb.value


def eval_quad_sample(a, b, M: int, N: int, K: int, rows, cols) -> np.ndarray:
    a, b = _f64(a), _f64(b)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    cols = np.ascontiguousarray(cols, dtype=np.int32)
    out = np.empty(rows.size, dtype=np.float64)
    host().ozt_eval_quad_sample(_ptr(a), _ptr(b), M, N, K, int(rows.size), _ptr(rows), _ptr(cols), _ptr(out))
    return out
