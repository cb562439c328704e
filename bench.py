#!/usr/bin/env python3
"""Headline benchmark: Ozaki-II INT8 FP64 GEMM at m = n = k = 8192 on one MI355X.

`--config C1|C2|C4|C5` measures the other BASELINE configs the same way (C1: II-INT8 1024^3 one
pass; C2: I-INT8 4096^3 automatic slices; C4: II-FP8 16384^3, phi 2; C5: I-BF16 8192 x 8192 x 65536,
8 slices, 1% zero rows and columns); the default line is C3. C4's value is the FP8 format as the
config names it and the library runs it by default, the FP8 route's e4m3 digit products on the FP8
matrix cores; the same plan carried by INT8 residues at its width (Transport.Int8Residues, the same C)
is reported beside it (`int8_residues`).

Workload: row-major FP64 A, B with entries (U(0,1)-0.5)*exp(0.5*N(0,1)),
the reference's evaluation generator with seed 3; Scheme II, INT8 residues, automatic moduli (<= 24),
forced two-pass reconstruction (the reconstruction here is exact, which serves both pass modes).

A "step" is one whole pass of the device pipeline (scale -> slice -> products -> reconstruction)
with A and B already resident in HBM and C left in HBM: the evaluation hooks replay the recorded
device steps `warmup` times untimed and `steps` times between two HIP events on the library's
stream (the host synchronizes before and after). This is the reference's "Total" (its whole-pass
replay, evaluation_hooks.hpp:175-211); planning and PCIe transfers are outside, as there.

value = 2*m*n*k / (time of one whole pass)  [effective FP64 TFLOP/s]

Scheme II computes with the smallest set of moduli (on the FP8 route, of e4m3 digit products) that
covers the operands' own bound on the exact integer product |C'| (Cauchy-Schwarz on A' and B'); the
reference sizes its set for the worst case K 2^(2b). C is the same bit for bit: the pass with the
reference's set is timed beside the line (`full_window`) and must give the same C.

Also reported: accuracy against binary128 on a 64x64 sample of C at full K (and the same numbers
for a native FP64 dot product), the per-phase device times, the roofline of the product kernel
(algorithmic int8 operations per launch / its average launch time in whole-pass replays right
after the timed ones, each product launch timed by its own dispatch on the library stream
(oz_time_products_begin), kept out of the timed region; against 5.0 POP/s dense INT8, or FP8 for C4;
`traffic` = the memory bytes per launch from the config's committed counter profile),
the reference's host OpenMP Dot2 GEMM (the oracle's restatement) timed on this host on a row
slab of the same problem, the GPU's own FP64 GEMM (rocBLAS dgemm) on the same operands, and the
wall time of calls on resident operands (Context.upload once; later calls reuse the pair's plan
and move only C over PCIe, or nothing when C stays on the GPU).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "effective FP64 TFLOP/s (2mnk/t) + max rel err vs binary128, Ozaki-II INT8 8192³"
INT8_PEAK_TOPS = 5000.0  # MI355X dense INT8 MFMA, 5.0 POP/s
FP8_PEAK_TFLOPS = 5000.0  # MI355X dense FP8 MFMA, 5.0 PFLOP/s
# Memory traffic per launch of each config's product kernel: 2.000 x FETCH_SIZE + 1.000 x WRITE_SIZE (KiB
# per dispatch, from rocprofv3 --pmc passes over this script; the factors are what the same counters read
# for a plain 1 GiB copy, whose FETCH_SIZE counts half of the bytes it reads), in bytes, with the committed
# summary it comes from and the plan it was measured on (the figure is printed only for that plan).
TRAFFIC = {
    # config: (bytes per launch, profile, products per launch of the plan measured)
    "C1": (0.0506e9, "profiles/scheme2_int8_c1_1024_traffic.md", 16),
    "C2": (4.415e9, "profiles/scheme1_int8_c2_4096_traffic.md", 36),
    "C3": (15.319e9, "profiles/scheme2_int8_c3_8192_traffic.md", 16),
    "C4": (247.123e9, "profiles/scheme2_fp8_c4_16384_traffic.md", 34),
    "C5": (248.19e9, "profiles/scheme1_bf16_c5_8192x65536_traffic.md", 36),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(a, b, m: int, n: int, k: int, rows: int) -> dict:
    """Reference host path (evaluation/numerics.hpp:58-93 Dot2, OpenMP) on rows [0, rows) of C."""
    from tests.oracle_lib import load_oracle
    orc = load_oracle()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rows = min(rows, m)
    t0 = time.perf_counter()
    hi, lo = orc.dot2(a, b, m, n, k, 0, rows)
    dt = time.perf_counter() - t0
    return {"value": round(2.0 * rows * n * k / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "sample": f"Dot2 compensated FP64 GEMM (reference_gemm restated in oracle/) on rows "
                                     f"0..{rows - 1} of C (full N={n}, K={k}), {dt:.2f} s; value = 2*rows*N*K/t"}, \
        hi[:rows * n], lo[:rows * n]


def effective_bits(c, hi, lo) -> float:
    """The reference's accuracy measure (evaluation/numerics.hpp:98-127): -log2 ||C - Cref||_F / ||Cref||_F with
    Cref = hi + lo renormalized, sums scaled by the largest magnitude."""
    s = hi + lo
    bb = s - hi
    rlo = (hi - (s - bb)) + (lo - bb)
    d = (c - s) - rlo
    mx = max(float(np.max(np.abs(s))), float(np.max(np.abs(d))))
    sc = 2.0 ** -np.floor(np.log2(mx)) if mx > 0 and np.isfinite(mx) else 1.0
    num = float(np.sum((d * sc) ** 2))
    den = float(np.sum((s * sc) ** 2))
    rel = np.sqrt(num) / np.sqrt(den) if den > 0 else (np.inf if num > 0 else 0.0)
    return float(-np.log2(rel)) if rel > 0 and np.isfinite(rel) else (99.0 if rel == 0 else -1.0)


def copy_probe(nbytes: int) -> int:
    """Reference transfer for the traffic counters: copy16_kernel reads and writes nbytes once each."""
    from oztt_amd.device import Device
    dev = Device(0)
    src, dst = dev.alloc(nbytes), dev.alloc(nbytes)
    dev.fill_u32(src, 0x01020304, nbytes // 4)
    for _ in range(3):
        dev.copy(dst, src, nbytes)
    dev.sync()
    print(json.dumps({"copy_probe_bytes": nbytes, "launches": 3}), flush=True)
    return 0


def native_fp64_gemm(a, b, m: int, n: int, k: int, reps: int = 3) -> dict:
    """The GPU's own FP64 GEMM on the same operands, as a yardstick for `value`: rocBLAS dgemm (its
    kernels on the FP64 matrix cores) on device-resident operands, timed with HIP events over `reps`
    calls after one warm-up call. Row 0 of the result is checked against numpy."""
    import ctypes
    try:
        hiprt = ctypes.CDLL("libamdhip64.so")
        rb = ctypes.CDLL("librocblas.so")
    except OSError as e:
        return {"error": str(e)}
    from oztt_amd.device import Device
    dev = Device(0)
    h = ctypes.c_void_p()
    try:
        bA, bB, bC = dev.upload(a), dev.upload(b), dev.alloc(8 * m * n)
        if rb.rocblas_create_handle(ctypes.byref(h)) != 0:
            return {"error": "rocblas_create_handle failed"}
        alpha, beta = ctypes.c_double(1.0), ctypes.c_double(0.0)
        none = 111  # rocblas_operation_none
        # row-major C = A B is the column-major product C^T = B^T A^T: (n x k) times (k x m)
        call = lambda: rb.rocblas_dgemm(h, none, none, n, m, k, ctypes.byref(alpha), bB.ptr, n, bA.ptr, k,
                                        ctypes.byref(beta), bC.ptr, n)
        if call() != 0:
            return {"error": "rocblas_dgemm failed"}
        hiprt.hipDeviceSynchronize()
        e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
        hiprt.hipEventCreate(ctypes.byref(e0))
        hiprt.hipEventCreate(ctypes.byref(e1))
        hiprt.hipEventRecord(e0, None)
        for _ in range(reps):
            call()
        hiprt.hipEventRecord(e1, None)
        hiprt.hipEventSynchronize(e1)
        t = ctypes.c_float()
        hiprt.hipEventElapsedTime(ctypes.byref(t), e0, e1)
        hiprt.hipEventDestroy(e0)
        hiprt.hipEventDestroy(e1)
        ms = t.value / reps
        row0 = dev.download(bC, np.float64, n)
        ok = bool(np.allclose(row0, a[:k] @ b.reshape(k, n), rtol=1e-10, atol=1e-300))
        return {"library": "rocBLAS dgemm", "ms": round(ms, 4), "tflops": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 3),
                "row0_checked": ok}
    finally:
        if h:
            rb.rocblas_destroy_handle(h)
        dev.close()


def vendor_int8_gemm(m: int, n: int, k: int, reps: int = 5) -> dict:
    """The vendor's int8 GEMM (hipBLASLt, through torch._int_mm) on one modulus's product shape,
    m x k times k x n int8 -> int32, with operands drawn like residues (uniform on [-127, 127]), as
    a yardstick for the product kernel: both run on the same matrix cores under the same power limit.
    Timed with torch events on torch's current stream (where torch launches it) over `reps` calls
    after one warm-up call; one row is checked against an int64 product."""
    import torch
    try:
        g = torch.Generator(device="cuda:0").manual_seed(11)
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda:0", generator=g)
        b = torch.randint(-127, 128, (k, n), dtype=torch.int8, device="cuda:0", generator=g)
        c = torch._int_mm(a, b)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            c = torch._int_mm(a, b)
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1) / reps
        want = a[:1].cpu().to(torch.int64) @ b.cpu().to(torch.int64)
        ok = bool(torch.equal(c[:1].cpu().to(torch.int64), want))
        ops = 2.0 * m * n * k
        out = {"library": "hipBLASLt int8 GEMM (torch._int_mm)", "shape": [m, n, k], "ms": round(ms, 4),
               "tops": round(ops / (ms * 1e-3) / 1e12, 2), "frac": round(ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
               "row0_checked": ok}
        del a, b, c
        torch.cuda.empty_cache()
        return out
    except Exception as e:  # an unsupported shape or build: report, do not fail the bench
        return {"error": f"{type(e).__name__}: {e}"}


# name -> (scheme, format, m, n, k, seed, phi, options, peak of the product format, rows of
# the CPU baseline slab, sample edge of the binary128 check). C3 is the headline and the default.
CONFIGS = {
    "C1": ("II", "INT8", 1024, 1024, 1024, 1, 0.5, dict(reconstruction="OnePass"), INT8_PEAK_TOPS, 1024, 64),
    "C2": ("I", "INT8", 4096, 4096, 4096, 2, 1.0, dict(), INT8_PEAK_TOPS, 4096, 64),
    "C3": ("II", "INT8", 8192, 8192, 8192, 3, 0.5, dict(reconstruction="TwoPass"), INT8_PEAK_TOPS, 8192, 64),
    # the FP8 route's e4m3 digit products on the FP8 matrix cores (dense FP8 peak 5.0 PFLOP/s); the same plan
    # carried by INT8 residues is measured beside it
    "C4": ("II", "FP8", 16384, 16384, 16384, 4, 2.0, dict(), FP8_PEAK_TFLOPS, 1024, 32),
    # BF16 digits (+-32) run on the INT8 matrix cores, so the product roofline is the INT8 peak
    "C5": ("I", "BF16", 8192, 8192, 65536, 5, 4.0, dict(slices=8), INT8_PEAK_TOPS, 512, 32),
}
WORKLOADS = {
    "C1": "C1 Ozaki-II INT8 m=n=k=1024, auto moduli, one-pass reconstruction",
    "C2": "C2 Ozaki-I INT8 m=n=k=4096, automatic slices",
    "C3": "C3 Ozaki-II INT8 m=n=k=8192, auto moduli (<=24), two-pass reconstruction",
    "C4": "C4 Ozaki-II FP8 m=n=k=16384, auto moduli (FP8 route), wide dynamic range phi=2",
    "C5": "C5 Ozaki-I BF16 m=n=8192 k=65536, 8 slices, rows i%100==0 of A and columns j%100==0 of B zero",
}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C3", choices=sorted(CONFIGS), help="BASELINE config (C3: the headline)")
    ap.add_argument("--cpu-rows", type=int, default=-1, help="rows of the CPU baseline slab (0: skip; -1: the "
                                                             "config's default, 10-20 s of Dot2 on 16 host threads)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only copy BYTES device-to-device with the plain copy kernel (calibrates HBM counters)")
    args = ap.parse_args()
    if args.copy_probe:
        return copy_probe(args.copy_probe)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              f"(the path would shard by 2-D output blocks with no exchange between GPUs)", file=sys.stderr)
        return 2
    import oztt_amd as oz

    scheme, fmt, m, n, k, seed, phi, extra, peak, cpu_rows, edge = CONFIGS[args.config]
    if args.cpu_rows >= 0:
        cpu_rows = args.cpu_rows
    log(f"{args.config}: generating inputs {m}x{k} and {k}x{n} (seed {seed}, phi {phi})")
    a, b = oz.eval_inputs(seed, phi, m * k, k * n)
    if args.config == "C5":  # 1% of A's rows and B's columns set to zero (82 of 8192 each)
        a.reshape(m, k)[::100, :] = 0.0
        b.reshape(k, n)[:, ::100] = 0.0
    opts = oz.Options(scheme=oz.Scheme[scheme], format=oz.Format[fmt])
    for key, v in extra.items():
        setattr(opts, key, oz.Reconstruction[v] if key == "reconstruction" else v)
    ctx = oz.Context(0)
    log("planning, first pass, whole-pass replays")
    t0 = time.perf_counter()
    c, info, ev = ctx.evaluate(a, b, m, n, k, opts, warmup=args.warmup, repeats=args.steps)
    log(f"call done in {time.perf_counter() - t0:.1f} s: slices={info.slices} moduli={info.moduli} "
        f"b={info.integer_bits} whole={ev.whole_ms:.3f} ms checked={ev.whole_checked}")
    if not ev.whole_checked:
        raise SystemExit("whole-pass replay output differs from the first pass")
    ms = ev.whole_ms
    value = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    # one plain Context.gemm from host buffers: planning + PCIe transfers + the pass (not the metric)
    c2 = np.empty(m * n)
    t0 = time.perf_counter()
    ctx.gemm(a, b, c2, m, n, k, opts)
    call_ms = (time.perf_counter() - t0) * 1e3
    if not np.array_equal(c2.view(np.uint64), c.view(np.uint64)):
        raise SystemExit("Context.gemm output differs from the evaluated pass")
    del c2

    # resident operands (Context.upload / gemm_resident): the same C from device-resident A and B;
    # the first call plans, later calls on the pair reuse the plan and move only C (or nothing)
    log("resident operands")
    t0 = time.perf_counter()
    rA, rB = ctx.upload(a, m, k), ctx.upload(b, k, n)
    upload_ms = (time.perf_counter() - t0) * 1e3
    c3 = np.empty(m * n)
    t0 = time.perf_counter()
    ctx.gemm_resident(rA, rB, c3, opts)
    first_ms = (time.perf_counter() - t0) * 1e3
    t0 = time.perf_counter()
    ctx.gemm_resident(rA, rB, c3, opts)
    again_ms = (time.perf_counter() - t0) * 1e3
    rC = oz.Matrix()
    ctx.gemm_resident(rA, rB, rC, opts)
    dev_runs = []
    for _ in range(5):  # the median of several calls: a single one can catch a cold start
        t0 = time.perf_counter()
        ctx.gemm_resident(rA, rB, rC, opts)
        dev_runs.append((time.perf_counter() - t0) * 1e3)
    dev_ms = float(np.median(dev_runs))
    if not np.array_equal(c3.view(np.uint64), c.view(np.uint64)):
        raise SystemExit("resident gemm output differs from the evaluated pass")
    resident = {"upload_ms": round(upload_ms, 2), "first_call_ms": round(first_ms, 2),
                "call_ms": round(again_ms, 2), "call_result_on_gpu_ms": round(dev_ms, 2),
                "call_result_on_gpu_tflops": round(2.0 * m * n * k / (dev_ms * 1e-3) / 1e12, 3)}
    for x in (rC, rA, rB):
        x.close()
    del c3

    # accuracy on an edge x edge sample at full K against binary128, next to a native FP64 dot product
    log("accuracy sample (binary128)")
    rng = np.random.default_rng(0)
    rs = np.sort(rng.choice(m, edge, replace=False))
    cs = np.sort(rng.choice(n, edge, replace=False))
    rows = np.repeat(rs, edge).astype(np.int32)
    cols = np.tile(cs, edge).astype(np.int32)
    q = oz.eval_quad_sample(a, b, m, n, k, rows, cols)
    A = a.reshape(m, k)
    B = b.reshape(k, n)
    got = c.reshape(m, n)[rows, cols]
    fp64 = np.einsum("ij,ij->i", A[rows], B[:, cols].T)  # native FP64 dot products
    absab = np.einsum("ij,ij->i", np.abs(A[rows]), np.abs(B[:, cols].T))
    nz = q != 0
    rel = np.abs(got - q)[nz] / np.abs(q[nz])
    rel64 = np.abs(fp64 - q)[nz] / np.abs(q[nz])
    bound = k * 2.0 ** -53 * absab[nz] / np.abs(q[nz])  # FP64 GEMM error bound gamma_k |A||B| relative to |C|
    gemm_ms = ev.gemm_launch_ms
    achieved = ev.product_ops / (gemm_ms * 1e-3) / 1e12
    headline = args.config == "C3"
    traffic, traffic_profile, traffic_products = TRAFFIC[args.config]
    if ev.partial_products != traffic_products:  # another plan than the one measured
        traffic = None
    fp8 = fmt == "FP8"
    kernel = ("gemm_f8_groups_kernel<TERMS> (oz2_gemm_groups_f8)" if fp8 else
              "gemm_i8_kernel" + ("<DIGITS> (oz2_gemm_digits)" if scheme == "II" else "<DIAG> (oz1_gemm_diag_i8)"))
    out = {
        "metric": METRIC if headline else f"effective FP64 TFLOP/s (2mnk/t), {WORKLOADS[args.config]}",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # the products' arithmetic: int8 (C5's BF16-format digits are int8 values), e4m3 for C4
        "dtype": "fp8_e4m3" if fp8 else "int8",
        "data": f"synthetic: reference evaluation generator, seed {seed}, (U(0,1)-0.5)*exp({phi}*N(0,1))",
        "config": {"workload": WORKLOADS[args.config], "m": m, "n": n, "k": k, "scheme": scheme, "format": fmt,
                   "slices": info.slices, "moduli": info.moduli, "integer_bits": info.integer_bits,
                   "reconstruction_passes": info.reconstruction_passes},
        "max_rel_err_vs_binary128": float(rel.max()),
        "fp64_max_rel_err_vs_binary128": float(rel64.max()),
        "max_err_over_fp64_bound": float((rel / bound).max()),
        "phases_ms": {key: round(ev.phase_ms[i], 4) for i, key in enumerate(["scale", "slice", "gemm", "compose", "recon"])},
        "host_call_ms": round(call_ms, 2),
        "host_call_tflops": round(2.0 * m * n * k / (call_ms * 1e-3) / 1e12, 3),
        "resident": resident,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4), "traffic": traffic, "traffic_profile": traffic_profile,
                     "kernel": kernel, "launch_ms": round(gemm_ms, 4), "ops_per_launch": ev.product_ops},
    }
    if scheme == "II":
        # the products computed (INT8 moduli or FP8 digit products) with the CRT window that the operands'
        # bound on |C'| allows, and, as a side measurement, the pass with the set for the reference's
        # window K 2^(2b): the same C bit for bit
        log("the same pass with the set for the window K 2^(2b)")
        cf, inff, evf = ctx.evaluate(a, b, m, n, k, opts, warmup=2, repeats=5, full_window=True)
        if not evf.whole_checked:
            raise SystemExit("full-window whole-pass replay output differs from its first pass")
        out["config"]["products"] = ev.partial_products
        out["full_window"] = {
            "products": evf.partial_products, "ms_per_step": round(evf.whole_ms, 4),
            "value": round(2.0 * m * n * k / (evf.whole_ms * 1e-3) / 1e12, 3),
            "identical_output": bool(np.array_equal(cf.view(np.uint64), c.view(np.uint64)))}
        if not out["full_window"]["identical_output"]:
            raise SystemExit("the full-window pass gives another C")
        del cf
    if fp8:
        out["config"]["transport"] = "the FP8 route's e4m3 digits on the FP8 matrix cores (the library's default)"
        out["config"]["digit_products"] = ev.partial_products
        # the same plan carried by INT8 residues at its width (Transport.Int8Residues): the same exact C'
        log("the FP8 plan on INT8 residues (Transport.Int8Residues)")
        oi = oz.Options(scheme=oz.Scheme[scheme], format=oz.Format[fmt], transport=oz.Transport.Int8Residues)
        ci, ii, ei = ctx.evaluate(a, b, m, n, k, oi, warmup=1, repeats=3)
        if not ei.whole_checked:
            raise SystemExit("INT8-residue whole-pass replay output differs from its first pass")
        i_tops = ei.product_ops / (ei.gemm_launch_ms * 1e-3) / 1e12
        out["int8_residues"] = {
            "ms_per_step": round(ei.whole_ms, 4), "value": round(2.0 * m * n * k / (ei.whole_ms * 1e-3) / 1e12, 3),
            "dtype": "int8", "int8_moduli": ii.moduli, "products": ei.partial_products,
            "phases_ms": {key: round(ei.phase_ms[i], 4)
                          for i, key in enumerate(["scale", "slice", "gemm", "compose", "recon"])},
            "roofline": {"bound": "mfma", "achieved": round(i_tops, 2), "peak": INT8_PEAK_TOPS,
                         "unit": "TFLOP/s", "frac": round(i_tops / INT8_PEAK_TOPS, 4),
                         "kernel": "gemm_i8_kernel<DIGITS> (oz2_gemm_digits)",
                         "launch_ms": round(ei.gemm_launch_ms, 4), "ops_per_launch": ei.product_ops},
            "same_width": (ii.integer_bits, ii.reconstruction_passes) == (info.integer_bits,
                                                                         info.reconstruction_passes),
            "identical_output": bool(np.array_equal(ci.view(np.uint64), c.view(np.uint64)))}
        del ci
    log("native FP64 GEMM on the GPU (rocBLAS dgemm)")
    out["native_fp64_gemm"] = native_fp64_gemm(a, b, m, n, k)
    log("vendor int8 GEMM on one product's shape (hipBLASLt)")
    v = vendor_int8_gemm(m, n, k)
    if "tops" in v:
        # the product kernel's rate per unit of int8 work next to the vendor's on the same shape
        v["product_kernel_tops"] = out["int8_residues"]["roofline"]["achieved"] if fp8 else round(achieved, 2)
    out["vendor_int8_gemm"] = v
    if cpu_rows > 0:
        log(f"CPU baseline: Dot2 on {cpu_rows} rows")
        out["cpu_baseline"], hi, lo = cpu_baseline(a, b, m, n, k, cpu_rows)
        rows = min(cpu_rows, m)
        # effective bits on the Dot2 slab, next to a native FP64 GEMM (BLAS through numpy) of the same rows
        native = a.reshape(m, k)[:rows] @ b.reshape(k, n)
        out["effective_bits"] = {"ozaki": round(effective_bits(c[:rows * n], hi, lo), 3),
                                 "native_fp64": round(effective_bits(native.ravel(), hi, lo), 3),
                                 "rows": rows}
    ctx.close()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
