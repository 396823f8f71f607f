"""Build libkg_gfx950.so in-tree with hipcc for gfx950.

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
OFFLOAD_ARCH = "gfx950"

HIP_FLAGS = (
    "-O3",
    "-std=c++17",
    f"--offload-arch={OFFLOAD_ARCH}",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the gfx950 backend needs ROCm's hipcc")
    return path


def include_flags() -> list[str]:
    return [f"-I{REPO_ROOT / 'include'}", f"-I{CSRC}"]


def build_library(output: Path = OUTPUT, extra_flags: tuple[str, ...] = (), verbose: bool = False) -> Path:
    """Compile csrc/kg_gfx950_entry.hip (+ the kg_gfx950 device headers) into `output`."""

    tmp = output.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIP_FLAGS, *extra_flags, "-shared", *include_flags(), str(CSRC / "kg_gfx950_entry.hip"), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    env = dict(os.environ)
    proc = subprocess.run(cmd, capture_output=True, text=True, env=env)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr[-4000:]}")
    os.replace(tmp, output)
    return output


def main() -> int:
    path = build_library(verbose=True)
    print(f"built {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
