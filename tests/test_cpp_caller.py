"""The public C++ interface as a C++ user builds it: tests/cpp/ozttgemm_caller.cpp includes only
include/ozTTgemm/ozTTgemm.hpp (and, for its evaluation-hook cases, the library's evaluation header)
and links libozTTgemm.so. It runs the reference's correctness program case for case
(tests/correctness.cpp) and its usage example (examples/gemm.cpp).

CPU: the program compiles from the header here, links, and passes the host-only argument checks
(correctness.cpp:49-85: rejected calls never open the device and leave C untouched).
GPU: the prebuilt program (oztt_amd/build.py writes tests/cpp/build/) passes every device case.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "tests" / "cpp" / "ozttgemm_caller.cpp"
LIB = ROOT / "oztt_amd" / "lib"
PREBUILT = ROOT / "tests" / "cpp" / "build" / "ozttgemm_caller"


def test_header_compiles_links_and_checks_arguments(tmp_path):
    exe = tmp_path / "caller"
    cmd = ["g++", "-std=c++20", "-O1", "-Wall", "-Wextra", "-Werror", f"-I{ROOT / 'include'}",
           f"-I{ROOT / 'oztt_amd' / 'csrc' / 'host'}", str(SRC), "-o", str(exe), f"-L{LIB}", "-lozTTgemm",
           f"-Wl,-rpath,{LIB}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe), "--host-only"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "argument checks passed" in r.stdout
    r = subprocess.run([str(exe), "--bogus"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2


@pytest.mark.gpu
def test_reference_correctness_program_on_device():
    assert PREBUILT.exists(), "build the libraries first (__graft_entry__.build())"
    print(f"running {PREBUILT}", flush=True)
    r = subprocess.run([str(PREBUILT)], capture_output=True, text=True, timeout=600)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr
    assert "all cases passed" in r.stdout
