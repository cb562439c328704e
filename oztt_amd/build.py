"""Builds the native libraries of oztt_amd in-tree (oztt_amd/lib/).

  liboz_hip.so     HIP kernels for gfx950 + the C ABI of include/oz_hip.h (hipcc)
  libozTTgemm.so   C++20 host library: the public ozTTgemm API, planners, backends, C entry
                   points for Python (g++, links liboz_hip.so)

Every HIP source is compiled with -ffp-contract=off (the splitting stages reproduce a specific
sequence of binary32 operations) and with packed FP32 instructions disabled. The Scheme II split
source additionally runs with FP32 denormals flushed (-fgpu-flush-denormals-to-zero), which is the
rule of the reference's operation model.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "lib" / "obj"
INCLUDE = ROOT / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]
HIP_SOURCES = {
    "oz_dev.hip": [],
    "oz_scale.hip": [],
    "oz2_split.hip": ["-fgpu-flush-denormals-to-zero", "-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "oz_gemm.hip": [],
    "oz2_crt.hip": [],
    "oz1_slice.hip": ["-fgpu-flush-denormals-to-zero"],
    "oz1_recon.hip": ["-fgpu-flush-denormals-to-zero"],
    "oz2_digits.hip": ["-fgpu-flush-denormals-to-zero"],
    "oz2_gemm_f8.hip": [],
    "oz2_pass.hip": [],
    "oz2_noalloc.hip": [],
}
HOST_FLAGS = ["-std=c++20", "-O2", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
              "-Wall", "-Wextra", f"-I{INCLUDE}", f"-I{CSRC / 'host'}"]
HOST_SOURCES = ["context.cpp", "dispatch.cpp", "norm.cpp", "pipeline.cpp", "plan1.cpp", "plan2.cpp", "route_digits.cpp", "ozaki1.cpp",
                "ozaki2.cpp", "evaluation.cpp", "capi.cpp"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected
    noise = ("packed-fp32-ops", "unknown target feature")
    err = "\n".join(l for l in r.stderr.splitlines() if not any(n in l for n in noise))
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{err}")


def build(jobs: int | None = None, oracle: bool = True) -> None:
    """Compile everything (always; no up-to-date check, so a changed header is never missed)."""
    OBJ.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    steps = []
    for src, extra in HIP_SOURCES.items():
        steps.append([HIPCC, *HIP_FLAGS, *extra, "-c", str(CSRC / src), "-o", str(OBJ / (src + ".o"))])
    for src in HOST_SOURCES:
        steps.append([CXX, *HOST_FLAGS, "-c", str(CSRC / "host" / src), "-o", str(OBJ / (src + ".o"))])
    with cf.ThreadPoolExecutor(jobs) as ex:
        for f in [ex.submit(_run, s) for s in steps]:
            f.result()
    hip_objs = [str(OBJ / (s + ".o")) for s in HIP_SOURCES]
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(LIB / "liboz_hip.so"), *hip_objs])
    host_objs = [str(OBJ / (s + ".o")) for s in HOST_SOURCES]
    _run([CXX, "-shared", "-fPIC", "-fopenmp", "-o", str(LIB / "libozTTgemm.so"), *host_objs,
          f"-L{LIB}", "-loz_hip", "-Wl,-rpath,$ORIGIN", "-lquadmath"])
    # a C++ caller of the public header (the reference's correctness cases and usage example), linked
    # with the library as a user would link it; run by tests/test_cpp_caller.py
    caller = ROOT / "tests" / "cpp"
    (caller / "build").mkdir(parents=True, exist_ok=True)
    _run([CXX, "-std=c++20", "-O2", "-Wall", "-Wextra", f"-I{INCLUDE}", f"-I{CSRC / 'host'}",
          str(caller / "ozttgemm_caller.cpp"), "-o", str(caller / "build" / "ozttgemm_caller"), f"-L{LIB}",
          "-lozTTgemm", "-Wl,-rpath,$ORIGIN/../../../oztt_amd/lib"])
    if oracle:
        _run(["make", "-s", "-C", str(ROOT / "oracle")])


if __name__ == "__main__":
    build()
    print("built", sorted(p.name for p in LIB.glob("*.so")), file=sys.stderr)
