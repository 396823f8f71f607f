"""CompileStrategy for the gfx950 target.

Input: a generated source, either plain HIP/C++ text or a SourceBundle whose files are
introduced by ``// __KG_BUNDLE_FILE__:<relative path>`` lines (the reference's marker,
kernel_gen/dsl/gen_kernel/emit/register.py:69; path checks as in
builtin_strategy/cuda_sm89.py:62-92). The main file is ``kernel.hip``.

Build: ``hipcc -std=c++17 --offload-arch=gfx950 -O2 -shared -fPIC -Xclang -target-feature
-Xclang -packed-fp32-ops -I<repo>/include -I<bundle dir> kernel.hip -o libkernel.so`` (the
packed-fp32 feature is always off, whatever flags the request carries) linked against libkg_gfx950.so (the prebuilt
gfx950 kernels and their C ABI), in a private work directory that
``CompiledKernel.close()`` removes (compiler.py:232-246 of the reference). Failures map to
``source_empty_or_invalid`` / ``compile_failed``.
"""

from __future__ import annotations

import shutil
import subprocess
import tempfile
from functools import partial
from pathlib import Path

from .. import native
from ..build import NO_PACKED_FP32, OFFLOAD_ARCH, REPO_ROOT, hipcc
from .compiler import COMPILE_FAILED, SOURCE_EMPTY_OR_INVALID, CompiledKernel, CompileRequest, execute_engine_error
from .runtime_args import parse_allow_absent
from .strategy import register_compile_strategy

BUNDLE_MARKER_PREFIX = "// __KG_BUNDLE_FILE__:"
MAIN_FILE = "kernel.hip"


def unbundle(source: str) -> dict[str, str]:
    lines = source.splitlines()
    if not lines or not lines[0].startswith(BUNDLE_MARKER_PREFIX):
        return {MAIN_FILE: source}
    files: dict[str, list[str]] = {}
    current: str | None = None
    for line in lines:
        if line.startswith(BUNDLE_MARKER_PREFIX):
            path = line[len(BUNDLE_MARKER_PREFIX):].strip()
            bad = (
                not path
                or path.startswith("/")
                or "\\" in path
                or "\x00" in path
                or path in files
                or any(part in {"", ".", ".."} for part in path.split("/"))
            )
            if bad:
                raise execute_engine_error(SOURCE_EMPTY_OR_INVALID, "source_bundle_malformed")
            files[path] = []
            current = path
            continue
        files[current].append(line)
    if MAIN_FILE not in files:
        raise execute_engine_error(SOURCE_EMPTY_OR_INVALID, "source_bundle_missing_hip_source")
    return {path: "\n".join(body) + "\n" for path, body in files.items()}


def _remove(path: Path) -> None:
    shutil.rmtree(path, ignore_errors=True)


class Gfx950CompileStrategy:
    """hipcc for gfx950 -> libkernel.so exporting the request's entry point."""

    def compile(self, request: CompileRequest) -> CompiledKernel:
        if request.target != "gfx950":
            raise execute_engine_error("target_header_mismatch", f"gfx950 strategy cannot build {request.target}")
        library = native.library_path()
        if not library.is_file():
            raise execute_engine_error(COMPILE_FAILED, f"{library} is missing; build the gfx950 library first")
        files = unbundle(request.source)
        work = Path(tempfile.mkdtemp(prefix="kg_execute_engine_gfx950_"))
        try:
            for rel, text in files.items():
                out = (work / "source" / rel).resolve()
                if not str(out).startswith(str((work / "source").resolve())):
                    raise execute_engine_error(SOURCE_EMPTY_OR_INVALID, "source_bundle_path_escape")
                out.parent.mkdir(parents=True, exist_ok=True)
                out.write_text(text)
            soname = work / "libkernel.so"
            flags = list(request.compiler_flags)
            if not any(f.startswith("--offload-arch") for f in flags):
                flags.append(f"--offload-arch={OFFLOAD_ARCH}")
            for extra in ("-O2", "-shared", "-fPIC"):
                if extra not in flags:
                    flags.append(extra)
            flags.extend(NO_PACKED_FP32)
            cmd = [
                request.compiler or hipcc(),
                *flags,
                f"-I{REPO_ROOT / 'include'}",
                f"-I{work / 'source'}",
                str(work / "source" / MAIN_FILE),
                "-o",
                str(soname),
                f"-L{library.parent}",
                f"-l:{library.name}",
                f"-Wl,-rpath,{library.parent}",
                *request.link_flags,
            ]
            proc = subprocess.run(cmd, capture_output=True, text=True)
            if proc.returncode != 0 or not soname.is_file():
                raise execute_engine_error(COMPILE_FAILED, f"hipcc returned {proc.returncode}: {proc.stderr[-2000:]}")
        except Exception:
            _remove(work)
            raise
        return CompiledKernel(
            target=request.target,
            soname_path=str(soname),
            function=request.function,
            entry_point=request.entry_point,
            compile_stdout=proc.stdout,
            compile_stderr=proc.stderr,
            allow_absent_memory_args=parse_allow_absent(request.source),
            _cleanup=partial(_remove, work),
        )


def register_gfx950_strategy(override: bool = False) -> None:
    register_compile_strategy("gfx950", Gfx950CompileStrategy(), override=override)
