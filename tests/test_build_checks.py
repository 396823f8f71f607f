"""Checks on the gfx950 machine code of the built libkg_gfx950.so (CPU only).

The HBM->LDS copies are inline asm that write M0 themselves (csrc/kg_gfx950/lds_dma.h):
clang treats M0 as reserved and does not know the asm changed it. That is safe only while
the compiler's own code never keeps a value in M0 across one of those statements, i.e.
while nothing else in the code object reads M0. These tests disassemble the code object
built here and check exactly that, so a change that makes the compiler use M0 (dynamic
register indexing, its own LDS DMA, GWS or message instructions) fails the CPU suite
instead of silently corrupting a kernel:

  - every instruction that names M0 is one of our `s_mov_b32 m0, sN`, followed by
    `s_nop 0` and an LDS-DMA load (`global_load_lds_dwordx4`, `buffer_load_dwordx4 ... lds`);
  - every LDS-DMA load is preceded by such a write;
  - no instruction that reads M0 implicitly appears (s_movrel*, v_movrel*, s_set_gpr_idx*,
    s_sendmsg*, ds_gws*, v_interp*, s_ttracedata, GDS forms).

It also checks that the compiler formed no packed-fp32 VALU instruction (the build turns
the feature off) by scanning for the `v_pk_` prefix with an f32 suffix.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from kernelcode_generate_amd import native

LLVM = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _disassemble(tmp_path: Path) -> list[str]:
    lib = native.library_path()
    if not lib.is_file():
        pytest.skip("libkg_gfx950.so is not built")
    tools = [LLVM / "llvm-objcopy", LLVM / "clang-offload-bundler", LLVM / "llvm-objdump"]
    if not all(t.exists() for t in tools):
        pytest.skip("ROCm LLVM tools are not installed")
    fat = tmp_path / "fat.bin"
    co = tmp_path / "gfx950.co"
    subprocess.run([str(tools[0]), f"--dump-section=.hip_fatbin={fat}", str(lib), str(tmp_path / "host.o")],
                   check=True, capture_output=True)
    subprocess.run([str(tools[1]), "--unbundle", "--type=o", f"--targets={TARGET}", f"--input={fat}",
                    f"--output={co}"], check=True, capture_output=True)
    out = subprocess.run([str(tools[2]), "-d", "--mcpu=gfx950", str(co)], check=True, capture_output=True,
                         text=True).stdout
    lines = []
    for line in out.splitlines():
        text = line.split("//", 1)[0].strip()
        if text and not text.endswith(">:") and not text.startswith("Disassembly") and ":" not in text.split()[0]:
            lines.append(text)
    return lines


@pytest.fixture(scope="module")
def instructions(tmp_path_factory):
    return _disassemble(tmp_path_factory.mktemp("isa"))


def _is_lds_dma(ins: str) -> bool:
    return ins.startswith("global_load_lds_") or (ins.startswith("buffer_load_") and re.search(r"\blds\b", ins) is not None)


def test_m0_written_only_for_lds_dma(instructions):
    assert len(instructions) > 1000
    writes = 0
    for i, ins in enumerate(instructions):
        if not re.search(r"\bm0\b", ins):
            continue
        assert re.fullmatch(r"s_mov_b32 m0, s\d+", ins), f"unexpected M0 use: {ins!r}"
        nxt = instructions[i + 1:i + 3]
        assert len(nxt) == 2 and nxt[0] == "s_nop 0" and _is_lds_dma(nxt[1]), f"M0 write not followed by a copy: {nxt}"
        writes += 1
    assert writes > 0


def test_every_lds_dma_sets_m0(instructions):
    copies = 0
    for i, ins in enumerate(instructions):
        if _is_lds_dma(ins):
            copies += 1
            assert i >= 2 and re.fullmatch(r"s_mov_b32 m0, s\d+", instructions[i - 2]), f"copy without its M0 write: {ins!r}"
    assert copies > 0


def test_no_implicit_m0_readers(instructions):
    readers = ("s_movrel", "v_movrel", "s_set_gpr_idx", "s_sendmsg", "ds_gws", "v_interp", "s_ttracedata")
    bad = [ins for ins in instructions if ins.startswith(readers) or re.search(r"\bgds\b", ins)]
    assert not bad, f"instructions that read M0: {bad[:5]}"


def test_no_packed_fp32_valu(instructions):
    bad = [ins for ins in instructions if re.match(r"v_pk_\w+_f32\b", ins)]
    assert not bad, f"packed fp32 instructions: {bad[:5]}"


def test_llvm_tools_present_or_skipped():
    # documents where the tools come from; the checks above skip without them
    assert shutil.which("hipcc") is None or LLVM.exists()
