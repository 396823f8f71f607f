"""Build libkg_gfx950.so in-tree with hipcc for gfx950 (object files under _build/).

    python -m kernelcode_generate_amd.build

Flags: -O3 for gfx950 only, C++17, and the packed-fp32 feature turned off (hipcc -O3
would otherwise form v_pk_{add,mul,fma}_f32 from ordinary float code).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
OUTPUT = PACKAGE_DIR / "libkg_gfx950.so"
PROBE_OUTPUT = PACKAGE_DIR / "libkg_gfx950_probe.so"  # bench.py's measurement library
OFFLOAD_ARCH = "gfx950"

# turns off the packed-fp32 target feature: every hipcc line that builds device code carries it
NO_PACKED_FP32 = ("-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")

HIP_FLAGS = (
    "-O3",
    "-std=c++17",
    f"--offload-arch={OFFLOAD_ARCH}",
    "-fPIC",
    *NO_PACKED_FP32,
)


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the gfx950 backend needs ROCm's hipcc")
    return path


def include_flags() -> list[str]:
    return [f"-I{REPO_ROOT / 'include'}", f"-I{CSRC}"]


SOURCES = ("kg_gfx950_entry.hip", "kg_gfx950_gemm.hip", "kg_gfx950_gemm_quad.hip", "kg_gfx950_fa.hip",
           "kg_gfx950_fa_persist.hip", "kg_gfx950_conv_rowvec.hip", "kg_gfx950_conv_igemm.hip")


def build_library(output: Path = OUTPUT, extra_flags: tuple[str, ...] = (), verbose: bool = False) -> Path:
    """Compile csrc/kg_gfx950_entry.hip and the kernel-family translation units (the
    explicit instantiations of kg_gfx950/instances.h), one hipcc process each, in parallel,
    and link them into `output`."""

    from concurrent.futures import ThreadPoolExecutor

    workdir = output.parent / "_build"
    workdir.mkdir(exist_ok=True)
    env = dict(os.environ)

    def run(cmd: list[str]) -> None:
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, capture_output=True, text=True, env=env)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd[-3:])}\n{proc.stderr[-4000:]}")

    objects = [workdir / (Path(src).stem + ".o") for src in SOURCES]
    cmds = [[hipcc(), *HIP_FLAGS, *extra_flags, "-c", *include_flags(), str(CSRC / src), "-o", str(obj)]
            for src, obj in zip(SOURCES, objects)]
    with ThreadPoolExecutor(max_workers=min(len(cmds), max(1, os.cpu_count() or 1))) as pool:
        for future in [pool.submit(run, cmd) for cmd in cmds]:
            future.result()
    tmp = output.with_suffix(".so.tmp")
    run([hipcc(), *HIP_FLAGS, *extra_flags, "-shared", *(str(o) for o in objects), "-o", str(tmp)])
    os.replace(tmp, output)
    return output


def build_probe_library(output: Path = PROBE_OUTPUT, verbose: bool = False) -> Path:
    """Compile csrc/probe/mfma_rate.hip, the MFMA-rate probe bench.py reports its ceiling
    from, into its own shared object (it is not part of libkg_gfx950.so)."""

    tmp = output.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIP_FLAGS, "-shared", *include_flags(), str(CSRC / "probe" / "mfma_rate.hip"), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True, env=dict(os.environ))
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr[-4000:]}")
    os.replace(tmp, output)
    return output


def main() -> int:
    path = build_library(verbose=True)
    print(f"built {path}")
    print(f"built {build_probe_library(verbose=True)}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
