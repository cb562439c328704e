#!/usr/bin/env python3
"""Headline benchmark: Ozaki-II INT8 FP64 GEMM at m = n = k = 8192 on one MI355X.

Workload: row-major FP64 A, B with entries (U(0,1)-0.5)*exp(0.5*N(0,1)),
the reference's evaluation generator with seed 3; Scheme II, INT8 residues, automatic moduli (<= 24),
forced two-pass reconstruction (the reconstruction here is exact, which serves both pass modes).

A "step" is one whole pass of the device pipeline (scale -> slice -> products -> reconstruction)
with A and B already resident in HBM and C left in HBM: the evaluation hooks replay the recorded
device steps `warmup` times untimed and `steps` times between two HIP events on the library's
stream (the host synchronizes before and after). This is the reference's "Total" (its whole-pass
replay, evaluation_hooks.hpp:175-211); planning and PCIe transfers are outside, as there.

value = 2*m*n*k / (time of one whole pass)  [effective FP64 TFLOP/s]

Also reported: accuracy against binary128 on a 64x64 sample of C at full K (and the same numbers
for a native FP64 dot product), the per-phase device times, the roofline of the product kernel
(algorithmic int8 operations per launch / its average launch time, against 5.0 POP/s dense INT8),
and the reference's host OpenMP Dot2 GEMM (the oracle's restatement) timed on this host on a row
slab of the same problem.
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
# HBM bytes per launch of the product kernel at n = 8192 (17 moduli), from the rocprofv3 FETCH_SIZE and
# WRITE_SIZE passes over this script scaled by the counters' readings for a plain 1 GiB copy
# (factors 2.000 and 1.000): profiles/scheme2_int8_c3_8192_traffic.md.
C3_GEMM_TRAFFIC_BYTES = 15.00e9


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(a, b, n: int, rows: int) -> dict:
    """Reference host path (evaluation/numerics.hpp:58-93 Dot2, OpenMP) on rows [0, rows) of C."""
    from tests.oracle_lib import load_oracle
    orc = load_oracle()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    t0 = time.perf_counter()
    orc.dot2(a, b, n, n, n, 0, rows)
    dt = time.perf_counter() - t0
    return {"value": round(2.0 * rows * n * n / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "sample": f"Dot2 compensated FP64 GEMM (reference_gemm restated in oracle/) on rows "
                                     f"0..{rows - 1} of C (full N={n}, K={n}), {dt:.2f} s; value = 2*rows*N*K/t"}


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--n", type=int, default=8192)
    ap.add_argument("--cpu-rows", type=int, default=1024, help="rows of the CPU baseline slab (0: skip)")
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

    n = args.n
    log(f"generating inputs {n}x{n} (seed 3, phi 0.5)")
    a, b = oz.eval_inputs(3, 0.5, n * n, n * n)
    opts = oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8, reconstruction=oz.Reconstruction.TwoPass)
    ctx = oz.Context(0)
    log("planning, first pass, whole-pass replays")
    t0 = time.perf_counter()
    c, info, ev = ctx.evaluate(a, b, n, n, n, opts, warmup=args.warmup, repeats=args.steps)
    log(f"call done in {time.perf_counter() - t0:.1f} s: moduli={info.moduli} b={info.integer_bits} "
        f"whole={ev.whole_ms:.3f} ms checked={ev.whole_checked}")
    if not ev.whole_checked:
        raise SystemExit("whole-pass replay output differs from the first pass")
    ms = ev.whole_ms
    value = 2.0 * n * n * n / (ms * 1e-3) / 1e12
    # one plain Context.gemm from host buffers: planning + PCIe transfers + the pass (not the metric)
    c2 = np.empty(n * n)
    t0 = time.perf_counter()
    ctx.gemm(a, b, c2, n, n, n, opts)
    call_ms = (time.perf_counter() - t0) * 1e3
    if not np.array_equal(c2.view(np.uint64), c.view(np.uint64)):
        raise SystemExit("Context.gemm output differs from the evaluated pass")
    del c2

    # accuracy on a 64 x 64 sample at full K against binary128, next to a native FP64 dot product
    log("accuracy sample (binary128)")
    rng = np.random.default_rng(0)
    rs = np.sort(rng.choice(n, 64, replace=False))
    cs = np.sort(rng.choice(n, 64, replace=False))
    rows = np.repeat(rs, 64).astype(np.int32)
    cols = np.tile(cs, 64).astype(np.int32)
    q = oz.eval_quad_sample(a, b, n, n, n, rows, cols)
    A = a.reshape(n, n)
    B = b.reshape(n, n)
    got = c.reshape(n, n)[rows, cols]
    fp64 = np.einsum("ij,ij->i", A[rows], B[:, cols].T)  # native FP64 dot products
    absab = np.einsum("ij,ij->i", np.abs(A[rows]), np.abs(B[:, cols].T))
    rel = np.abs(got - q) / np.abs(q)
    rel64 = np.abs(fp64 - q) / np.abs(q)
    bound = n * 2.0 ** -53 * absab / np.abs(q)  # FP64 GEMM error bound gamma_k |A||B| relative to |C|
    gemm_ms = ev.gemm_launch_ms
    achieved = ev.product_ops / (gemm_ms * 1e-3) / 1e12
    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: reference evaluation generator, seed 3, (U(0,1)-0.5)*exp(0.5*N(0,1))",
        "config": {"workload": f"C3 Ozaki-II INT8 m=n=k={n}, auto moduli (<=24), two-pass reconstruction",
                   "m": n, "n": n, "k": n, "moduli": info.moduli, "integer_bits": info.integer_bits,
                   "reconstruction_passes": info.reconstruction_passes},
        "max_rel_err_vs_binary128": float(rel.max()),
        "fp64_max_rel_err_vs_binary128": float(rel64.max()),
        "max_err_over_fp64_bound": float((rel / bound).max()),
        "phases_ms": {k: round(ev.phase_ms[i], 4) for i, k in enumerate(["scale", "slice", "gemm", "compose", "recon"])},
        "host_call_ms": round(call_ms, 2),
        "host_call_tflops": round(2.0 * n * n * n / (call_ms * 1e-3) / 1e12, 3),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / INT8_PEAK_TOPS, 4),
                     "traffic": C3_GEMM_TRAFFIC_BYTES if (n == 8192 and info.moduli == 17) else None,
                     "kernel": "gemm_i8_kernel<true> (oz2_gemm_digits)", "launch_ms": round(gemm_ms, 4),
                     "ops_per_launch": ev.product_ops},
    }
    if args.cpu_rows > 0:
        log(f"CPU baseline: Dot2 on {args.cpu_rows} rows")
        out["cpu_baseline"] = cpu_baseline(a, b, n, args.cpu_rows)
    ctx.close()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
