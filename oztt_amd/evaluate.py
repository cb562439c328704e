"""The paper evaluator on MI355X: the reference's case plan and CSV columns (evaluation/evaluate.cpp:152-480,
evaluation/README.md:146-159), for side-by-side comparison with its results.

    python -m oztt_amd.evaluate --quick --output results.csv
    python -m oztt_amd.evaluate --suite table --sizes 3520,7040 --formats INT8,FP8

Cases (the reference's fixed order): suite "table" runs every size x format x {Scheme I with the
format's slice count, Scheme II one-pass with fixed b = 54 and the format's moduli limit} on the
uniform input; suite "phi" runs BFP8 Scheme I, Scheme II one-pass and two-pass (automatic b, at most
24 moduli) on (U(0,1) - 0.5) exp(phi N(0,1)) at `--phi-size`. Inputs come from the evaluator's
generator (mt19937, seed 7, numerics.hpp:19-38).

Columns as the reference writes them. The phase times are the library's per-phase device times of
the first pass; total_ms is the average uninterrupted whole pass (the paper's Total) replayed on the
device with the inputs resident; effective_tflops = 2 n^3 / total_ms; gemm_tops uses the product
phase; nominal_peak_percent is against the dense MI355X peak of the matrix instructions used
(5.0 POP/s INT8, 5.0 PFLOP/s FP8). partial_products counts the products the device ran: for FP8
the FP8 route's digit products (the reference's count), for the other Scheme II formats but INT8 one
per modulus of the INT8 set that carries the format's width; moduli is the format's own route's (the
reference's). With --int8-residues (Transport.Int8Residues) FP8 is carried by INT8 residues too, and
moduli counts the INT8 moduli that computed. effective_bits / relative_fro compare with the Dot2 reference
(computed by the library's evaluator numerics), cpu_dgemm_bits the host's native FP64 GEMM (BLAS
through numpy) the same way. Columns that describe Tenstorrent telemetry (bw: the Tensix GEMM block
width; gemm_aiclk_mhz; start_temperature_c) are written as 0 / nan.
"""
from __future__ import annotations

import argparse
import csv
import dataclasses
import sys
import time

import numpy as np

from . import Context, Format, Options, Reconstruction, Scheme, Transport, eval_accuracy, eval_hash, eval_inputs, \
    eval_reference_gemm, format_name

COLUMNS = ("suite,n,scheme,format,phi,timing,reference,slices,integer_bits,moduli,passes,partial_products,bw,"
           "scale_ms,slice_ms,gemm_ms,compose_ms,recon_ms,phase_sum_ms,total_ms,effective_tflops,gemm_tops,"
           "nominal_peak_percent,gemm_aiclk_mhz,evaluation_wall_ms,effective_bits,relative_fro,output_hash,"
           "cpu_dgemm_bits,fp64_equivalent,start_temperature_c").split(",")
FORMATS = [Format.BF16, Format.FP16, Format.TF32, Format.BFP8, Format.FP8, Format.INT8, Format.BFP4, Format.BFP2]
# per format (enum order): Scheme I slices and Scheme II moduli limit of the table suite (evaluate.cpp:162)
SLICES = [10, 10, 10, 10, 12, 8, 16, 59]
MODULI = [24, 24, 11, 24, 14, 16, 24, 24]
PEAK_TOPS = 5000.0  # MI355X dense INT8 (POP/s) and FP8 (PFLOP/s) matrix peaks, in TOP/s


def cases(suite, sizes, formats, phis, phi_size):
    out = []
    if suite != "phi":
        for n in sizes:
            for f in formats:
                for scheme in (Scheme.I, Scheme.II):
                    o = Options(scheme=scheme, format=f)
                    if scheme == Scheme.I:
                        o.slices = SLICES[int(f)]
                    else:
                        o.max_moduli = MODULI[int(f)]
                        o.reconstruction = Reconstruction.OnePass
                    out.append(("table", n, -1.0, o, 54 if scheme == Scheme.II else 0))
    if suite != "table":
        for phi in phis:
            out.append(("phi", phi_size, phi, Options(scheme=Scheme.I, format=Format.BFP8), 0))
            for rec in (Reconstruction.OnePass, Reconstruction.TwoPass):
                out.append(("phi", phi_size, phi, Options(scheme=Scheme.II, format=Format.BFP8, max_moduli=24,
                                                           reconstruction=rec), 0))
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--suite", default="all", choices=["table", "phi", "all"])
    ap.add_argument("--sizes", default="3520,7040,14080")
    ap.add_argument("--phi-size", type=int, default=14080)
    ap.add_argument("--phis", default="0.5,1,2,4,8")
    ap.add_argument("--formats", default=",".join(format_name(f) for f in FORMATS))
    ap.add_argument("--repeats", type=int, default=3, help="timed whole-pass replays")
    ap.add_argument("--warmup", type=int, default=5, help="untimed whole-pass replays (0: 'quick' timing)")
    ap.add_argument("--device", type=int, default=0)
    ap.add_argument("--case", type=int, default=None, help="run only this case of the plan (0-based), appending")
    ap.add_argument("--output", default="results.csv")
    ap.add_argument("--list", action="store_true", help="print the plan and exit")
    ap.add_argument("--no-reference", action="store_true", help="no Dot2 reference (and no CPU GEMM)")
    ap.add_argument("--no-cpu", action="store_true", help="no host FP64 GEMM for cpu_dgemm_bits")
    ap.add_argument("--quick", action="store_true", help="sizes 128, phi size 128, phis 0.5,2,8, 1 repeat, no warmup")
    ap.add_argument("--int8-residues", action="store_true",
                    help="Scheme II with Transport.Int8Residues: every format's plan carried by INT8 residues at its "
                         "width (FP8 runs the FP8 route's e4m3 digits on the FP8 matrix cores otherwise; the same "
                         "output either way)")
    args = ap.parse_args(argv)
    sizes = [int(s) for s in args.sizes.split(",")]
    phis = [float(s) for s in args.phis.split(",")]
    phi_size, repeats, warmup = args.phi_size, args.repeats, args.warmup
    if args.quick:
        sizes, phi_size, phis, repeats, warmup = [128], 128, [0.5, 2.0, 8.0], 1, 0
    names = {format_name(f): f for f in FORMATS}
    formats = [names[s] for s in args.formats.split(",")]
    if any(n % 64 or not 64 <= n <= 32768 for n in sizes + [phi_size]):
        raise SystemExit("sizes must be multiples of 64 in [64, 32768]")
    plan = cases(args.suite, sizes, formats, phis, phi_size)
    if args.list:
        print("suite,n,scheme,format,phi,slices,max_moduli,fixed_bits,passes")
        for i, (suite, n, phi, o, bits) in enumerate(plan):
            print(f"{i}: {suite},{n},{o.scheme.name},{format_name(o.format)},{phi},{o.slices},{o.max_moduli},{bits},"
                  f"{o.reconstruction.name}")
        return 0
    run = [plan[args.case]] if args.case is not None else plan
    reference = not args.no_reference
    cpu = reference and not args.no_cpu
    ctx = Context(args.device)
    mode = "a" if args.case is not None else "w"
    cache = {}
    with open(args.output, mode, newline="") as fh:
        w = csv.writer(fh)
        if mode == "w" or fh.tell() == 0:
            w.writerow(COLUMNS)
        for suite, n, phi, o, bits in run:
            print(f"Evaluating {suite} {n} {o.scheme.name}-{format_name(o.format)} phi={phi}", flush=True)
            key = (n, phi)
            if key not in cache:
                a, b = eval_inputs(7, phi, n * n, n * n)
                hi = lo = cpu_bits = None
                if reference:
                    hi, lo = eval_reference_gemm(a, b, n, n, n)
                    if cpu:
                        cpu_bits = eval_accuracy((a.reshape(n, n) @ b.reshape(n, n)).ravel(), hi, lo)[1]
                cache.clear()
                cache[key] = (a, b, hi, lo, cpu_bits)
            a, b, hi, lo, cpu_bits = cache[key]
            t0 = time.perf_counter()
            if args.int8_residues and o.scheme == Scheme.II:
                o = dataclasses.replace(o, transport=Transport.Int8Residues)
            c, info, ev = ctx.evaluate(a, b, n, n, n, o, fixed_bits=bits, warmup=warmup, repeats=max(repeats, 1))
            call_ms = (time.perf_counter() - t0) * 1e3
            if not ev.whole_checked:
                raise SystemExit("whole-pass replay output differs from the first pass")
            rel, ebits = eval_accuracy(c, hi, lo) if reference else (float("nan"), float("nan"))
            phases = [ev.phase_ms[i] for i in range(5)]
            total = ev.whole_ms
            ops = 2.0 * n ** 3
            tops = ops * ev.partial_products / (phases[2] * 1e-3) / 1e12 if phases[2] > 0 else float("nan")
            if not reference:
                equivalent = "unknown"
            elif ebits < 53:
                equivalent = "no"
            elif cpu_bits is None or not np.isfinite(cpu_bits):
                equivalent = "unknown"
            else:
                equivalent = "yes" if ebits >= cpu_bits else "no"
            w.writerow([suite, n, o.scheme.name, format_name(o.format), f"{phi:g}", "steady" if warmup > 0 else "quick",
                        "Dot2" if reference else "none", info.slices, info.integer_bits, info.moduli,
                        info.reconstruction_passes, ev.partial_products, 0, *[f"{x:.12g}" for x in phases],
                        f"{sum(phases):.12g}", f"{total:.12g}", f"{ops / (total * 1e-3) / 1e12:.12g}", f"{tops:.12g}",
                        f"{100 * tops / PEAK_TOPS:.12g}", "nan", f"{call_ms:.12g}", f"{ebits:.12g}", f"{rel:.12g}",
                        f"{eval_hash(c):x}", "nan" if cpu_bits is None else f"{cpu_bits:.12g}", equivalent, "nan"])
            fh.flush()
            print(f"  {ops / (total * 1e-3) / 1e12:.4g} TFlops/s ({total:.4g} ms whole pass, phase sum "
                  f"{sum(phases):.4g} ms), {ebits:.6g} bits, FP64-equivalent={equivalent}", flush=True)
    ctx.close()
    print(f"CSV: {args.output}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
