"""Checks on the gfx950 code generated for the product kernels (oztt_amd/csrc/oz_gemm.hip: int8 x
int8 -> int32; oztt_amd/csrc/oz2_gemm_f8.hip: e4m3 x e4m3 -> fp32).

The kernels load operands with an inline-asm global->LDS copy (ozg::lds_copy_block) that sets M0
itself, so the compiler must not use M0 for anything else in them; and their throughput depends on
the main loop keeping the 256 accumulators in AGPRs and the fragments in VGPRs (when the register
allocator mixes the two classes it adds v_accvgpr moves to every K step, or spills). Both are
properties of the compiled code, so this test compiles the source with the build's flags and reads
the assembly. It needs hipcc (present wherever the library is built) but no GPU.
"""
from __future__ import annotations

import re
import shutil
import subprocess

import pytest

from oztt_amd import build as B


# source -> (kernel name stem, instantiations, MFMA mnemonic, MFMAs per trip of the main loop)
SOURCES = {
    "oz_gemm.hip": ("gemm_i8_kernel", 6, "v_mfma_i32_16x16x64_i8", 128),
    "oz2_gemm_f8.hip": ("gemm_f8_groups_kernel", 4, "v_mfma_f32_32x32x64_f8f6f4", 32),
}


def _kernels(asm: str, stem: str) -> dict[str, list[str]]:
    """Function name -> body lines (label to end marker) for every kernel named `stem` in the listing."""
    out = {}
    for m in re.finditer(r"^(_Z\S*" + stem + r"\S*):.*?$(.*?)^\.Lfunc_end", asm, re.S | re.M):
        out[m.group(1)] = m.group(2).split("\n")
    return out


def _main_loop(lines: list[str]) -> list[str]:
    """Instructions of the innermost loop that contains the MFMAs (header to its last back-branch)."""
    best = []
    for i, l in enumerate(lines):
        h = re.match(r"(\.LBB\d+_\d+):.*Loop Header", l)
        if not h:
            continue
        ends = [k for k in range(i + 1, len(lines)) if re.search(r"s_c?branch\w*\s+" + re.escape(h.group(1)) + r"\b", lines[k])]
        body = [x.strip() for x in lines[i:max(ends) + 1]] if ends else []
        if sum(x.startswith("v_mfma") for x in body) > sum(x.startswith("v_mfma") for x in best):
            best = body
    return [x for x in best if x and not x.startswith(";")]


@pytest.fixture(scope="module", params=sorted(SOURCES))
def gemm_asm(request, tmp_path_factory):
    """(source name, assembly of the source compiled with the build's flags)."""
    if not shutil.which(B.HIPCC) and not shutil.os.path.exists(B.HIPCC):
        pytest.skip("hipcc not available")
    src = request.param
    out = tmp_path_factory.mktemp("asm") / (src + ".s")
    cmd = [B.HIPCC, *B.HIP_FLAGS, *B.HIP_SOURCES[src], "--cuda-device-only", "-S", str(B.CSRC / src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return src, out.read_text()


def test_all_instantiations_present(gemm_asm):
    src, asm = gemm_asm
    stem, count, _, _ = SOURCES[src]
    names = _kernels(asm, stem)
    # oz_gemm.hip: three modes (products, digits, scheme I diagonals) x (even K/64, any K/64);
    # oz2_gemm_f8.hip: two output kinds (int32 sums, uint16 terms) x (even K/64, any K/64)
    assert len(names) == count, sorted(names)


def test_m0_only_feeds_the_lds_copies(gemm_asm):
    src, asm = gemm_asm
    for name, lines in _kernels(asm, SOURCES[src][0]).items():
        body = [l.strip() for l in lines if l.strip() and not l.strip().startswith(";")]
        for i, l in enumerate(body):
            if re.search(r"\bm0\b", l):
                assert re.match(r"s_mov_b32 m0, (s\d+|vcc_lo|vcc_hi)$", l), (name, l)  # an SGPR (VCC is one)
                assert body[i + 1].startswith("global_load_lds_dwordx4"), (name, l, body[i + 1])


def test_no_spills(gemm_asm):
    src, asm = gemm_asm
    stem, count, _, _ = SOURCES[src]
    meta = re.findall(r"\.name:\s+(_Z\S*" + stem + r"\S*)\s.*?\.private_segment_fixed_size:\s+(\d+).*?"
                      r"\.vgpr_spill_count:\s+(\d+)", asm, re.S)
    assert len(meta) == count
    for name, private, spills in meta:
        assert private == "0" and spills == "0", (name, private, spills)


def test_even_main_loops_keep_accumulators_in_agprs(gemm_asm):
    src, asm = gemm_asm
    stem, _, mfma, per_trip = SOURCES[src]
    for name, lines in _kernels(asm, stem).items():
        loop = _main_loop(lines)
        # two K steps per trip: 2 x 64 (int8) or 2 x 16 (fp8) MFMAs, 2 x 16 fragment reads,
        # 2 x 8 global->LDS copies, and no other memory access (a vector load in the loop would
        # also upset the vmcnt waits)
        assert sum(x.startswith(mfma) for x in loop) == per_trip, name
        assert sum(x.startswith("ds_read_b128") for x in loop) == 32, name
        assert sum(x.startswith("global_load_lds_dwordx4") for x in loop) == 16, name
        assert not any(re.match(r"(global|buffer|flat)_load_(?!lds)", x) for x in loop), name
        assert not any(x.startswith("scratch_") for x in loop), name
        if "ELb1E" in name:  # the EVEN instantiations (every production shape with K % 128 == 0)
            assert not any(x.startswith("v_accvgpr") for x in loop), (name, "accumulators moved in the loop")
            assert sum(1 for x in loop if re.match(r"\.LBB", x)) == 1, (name, "branches inside the loop")
