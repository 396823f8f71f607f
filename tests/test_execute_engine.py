"""CPU tests of the gfx950 drop-in boundary: target registry, strategy registry, the
SourceBundle emitter, the gfx950 compile strategy (real hipcc cross-compile and a fake
compiler that records its command line, as test/execute_engine/test_cuda_sm89_strategy.py
does with a fake nvcc) and the stable failure phrases of the execute engine."""

from __future__ import annotations

import ctypes
import os
import stat
from pathlib import Path

import pytest

from kernelcode_generate_amd import native
from kernelcode_generate_amd.core.config import restore_config, set_target, snapshot_config
from kernelcode_generate_amd.core.error import KernelCodeError
from kernelcode_generate_amd.execute_engine import (
    CompileRequest,
    ExecuteRequest,
    ExecutionEngine,
    get_compile_strategy,
    register_compile_strategy,
)
from kernelcode_generate_amd.execute_engine.compiler import CompiledKernel
from kernelcode_generate_amd.execute_engine.gfx950_strategy import Gfx950CompileStrategy, unbundle
from kernelcode_generate_amd.execute_engine.runtime_args import parse_allow_absent, validate_args
from kernelcode_generate_amd.dsl import mlir_gen
from kernelcode_generate_amd.gen_kernel import gen_kernel
from kernelcode_generate_amd.kernel.conv2d.inputs_dynamic_tile_dynamic import conv2d_inputs_dynamic_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.conv2d.inputs_static_tile_dynamic import conv2d_inputs_static_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.conv2d.inputs_static_tile_static import conv2d_inputs_static_tile_static_kernel
from kernelcode_generate_amd.kernel.flash_attention.inputs_dynamic_tile_dynamic import (
    flash_attention_inputs_dynamic_tile_dynamic_kernel,
)
from kernelcode_generate_amd.kernel.flash_attention.inputs_static_tile_static import (
    flash_attention_inputs_static_tile_static_kernel,
)
from kernelcode_generate_amd.kernel.flash_attention.scaled import flash_attention_scaled_causal_kernel
from kernelcode_generate_amd.kernel.matmul.inputs_static_tile_dynamic import matmul_inputs_static_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.matmul.inputs_static_tile_static import matmul_inputs_static_tile_static_kernel
from kernelcode_generate_amd.kernel.runner import run_lowering_demo
from kernelcode_generate_amd.pipeline import build_gfx950_lowering_pipeline, get_pipeline
from kernelcode_generate_amd.target import get_target_hardware, is_arch_op_supported
from kernelcode_generate_amd.tools import dsl_run

T = native.TensorSpec
_M2, _B1, _X4 = T((4, 5), "float32"), T((5,), "float32"), T((1, 2, 4, 5), "float32")
ALL_DEMOS = [
    (matmul_inputs_static_tile_static_kernel, (_M2, _M2, _M2, None), "matmul"),
    (matmul_inputs_static_tile_dynamic_kernel, (_M2, _M2, _M2, _B1, 2, 2, 2), "matmul"),
    (conv2d_inputs_static_tile_static_kernel, (_X4, _X4, _X4, None), "conv2d"),
    (conv2d_inputs_static_tile_dynamic_kernel, (_X4, _X4, _X4, _B1, 7, 18, 3, 9, 8), "conv2d"),
    (conv2d_inputs_dynamic_tile_dynamic_kernel, (_X4, _X4, _X4, None) + (1,) * 8 + (7, 18, 3, 9, 8), "conv2d"),
    (flash_attention_inputs_static_tile_static_kernel, (_X4,) * 4, "flash_attention"),
    (flash_attention_inputs_dynamic_tile_dynamic_kernel, (_X4,) * 4 + (2, 2), "flash_attention"),
    (flash_attention_scaled_causal_kernel, (_X4,) * 4 + (2, 2, 0.5), "flash_attention"),
]


def lower(fn, *args, **options):
    return get_pipeline("gfx950-lowering", options or None).run(mlir_gen(fn, args))


def test_gfx950_target_spec():
    assert get_target_hardware("gfx950", "block_num") == 256
    assert get_target_hardware("gfx950", "subthread_num") == 64
    assert get_target_hardware("gfx950", "sm_memory_size") == 160 * 1024
    assert is_arch_op_supported("gfx950", "arch.barrier")
    assert not is_arch_op_supported("gfx950", "arch.launch_kernel")
    assert get_target_hardware("npu_demo", "block_num") == 2


def test_strategy_registry_phrases():
    assert isinstance(get_compile_strategy("gfx950"), Gfx950CompileStrategy)
    with pytest.raises(KernelCodeError) as err:
        get_compile_strategy("npu_demo")  # registered target, no strategy here
    assert err.value.failure_phrase == "target_header_mismatch"
    with pytest.raises(KernelCodeError) as err:
        get_compile_strategy("not_a_target")
    assert err.value.failure_phrase == "target_header_mismatch"
    with pytest.raises(KernelCodeError) as err:
        register_compile_strategy("gfx950", Gfx950CompileStrategy())
    assert err.value.failure_phrase == "compile_failed"  # duplicate without override


@pytest.mark.parametrize("fn,args,family", ALL_DEMOS, ids=lambda v: getattr(v, "__name__", ""))
def test_generated_sources(fn, args, family):
    lowered, source = run_lowering_demo("case", fn, *args)
    assert lowered.fused is not None and lowered.fused.family == family
    assert source.startswith("// __KG_BUNDLE_FILE__:kernel.hip")
    assert 'extern "C" int kg_execute_entry(const KgArgSlot* s, unsigned long long n)' in source
    assert f"kg_gfx950_{family}_entry(slots," in source
    assert f"n != {len(args)}ULL" in source
    assert lowered.hardware["subthread_num"] == 64
    assert "kernel-pattern-fuse" in lowered.applied
    files = unbundle(source)
    assert set(files) == {"kernel.hip"}
    # the per-operation path renders the same kernel as one HIP kernel of kg_tile calls
    per_op = gen_kernel(lower(fn, *args, fuse="false"))
    assert "kg_gfx950_generated_kernel" in per_op and "kg_tile::" in per_op and "kg_gfx950_" + family not in per_op


def test_static_demo_constants_are_baked():
    # stride 8 and the seeded pads of kernel/conv2d/inputs_static_tile_static.py: (3, 3, 4, 0)
    lowered = lower(conv2d_inputs_static_tile_static_kernel, _X4, _X4, _X4, None)
    src = gen_kernel(lowered)
    assert "slots[4].int_value = 8LL;" in src and "slots[5].int_value = 8LL;" in src
    assert "slots[8].int_value = 3LL;" in src and "slots[10].int_value = 4LL;" in src
    mm = lower(matmul_inputs_static_tile_static_kernel, _M2, _M2, _M2, None).fused
    assert tuple(t.value for t in mm.ints) == (48, 80, 56)
    fa = gen_kernel(lower(flash_attention_scaled_causal_kernel, *((T((1, 2, 8, 64), "bfloat16"),) * 4), 64, 64, 0.1))
    assert "slots[7].int_value = 1LL;" in fa  # causal flag appended after the scale slot


def test_allow_absent_metadata_roundtrip():
    src = gen_kernel(lower(matmul_inputs_static_tile_static_kernel, _M2, _M2, _M2, None))
    specs = parse_allow_absent(src)
    assert len(specs) == 1 and specs[0].index == 3 and specs[0].dtype == "float32" and specs[0].rank == 1
    with pytest.raises(KernelCodeError) as err:
        validate_args((1, 2, None), ())
    assert err.value.failure_phrase == "runtime_throw_or_abort"


def test_pipeline_registry_and_options():
    assert get_pipeline("gfx950-lowering").name == "gfx950-lowering"
    with pytest.raises(KernelCodeError):
        build_gfx950_lowering_pipeline({"target": "cuda_sm89"})
    with pytest.raises(KernelCodeError):
        build_gfx950_lowering_pipeline({"fold": "true"})
    with pytest.raises(KernelCodeError):
        build_gfx950_lowering_pipeline({"fuse": "maybe"})


@pytest.mark.parametrize(
    "bad",
    [
        "// __KG_BUNDLE_FILE__:../escape.hip\nint x;",
        "// __KG_BUNDLE_FILE__:/abs.hip\nint x;",
        "// __KG_BUNDLE_FILE__:kernel.hip\nint x;\n// __KG_BUNDLE_FILE__:kernel.hip\nint y;",
        "// __KG_BUNDLE_FILE__:other.hip\nint x;",
    ],
)
def test_malformed_bundles(bad):
    with pytest.raises(KernelCodeError) as err:
        unbundle(bad)
    assert err.value.failure_phrase == "source_empty_or_invalid"


def test_engine_rejects_empty_source():
    with pytest.raises(KernelCodeError) as err:
        ExecutionEngine("gfx950").compile(source="   ", function="f")
    assert err.value.failure_phrase == "source_empty_or_invalid"


def _fake_hipcc(tmp_path: Path, rc: int = 0) -> Path:
    log = tmp_path / "argv.log"
    script = tmp_path / "fake-hipcc"
    script.write_text(
        "#!/bin/bash\n"
        f'echo "$@" >> {log}\n'
        'out=""; prev=""; for a in "$@"; do if [ "$prev" = "-o" ]; then out="$a"; fi; prev="$a"; done\n'
        f'if [ {rc} -ne 0 ]; then echo "fake failure" >&2; exit {rc}; fi\n'
        'touch "$out"\n'
    )
    script.chmod(script.stat().st_mode | stat.S_IEXEC)
    return script


def test_fake_compiler_command_line(tmp_path):
    fake = _fake_hipcc(tmp_path)
    src = gen_kernel(lower(matmul_inputs_static_tile_dynamic_kernel, _M2, _M2, _M2, None, 2, 2, 2))
    kernel = ExecutionEngine("gfx950", compiler=str(fake)).compile(source=src, function="matmul")
    argv = (tmp_path / "argv.log").read_text()
    assert "--offload-arch=gfx950" in argv and "-shared" in argv and "-fPIC" in argv and "-std=c++17" in argv
    assert "kernel.hip" in argv and "libkg_gfx950.so" in argv and "-Wl,-rpath," in argv
    assert "-Xclang -target-feature -Xclang -packed-fp32-ops" in argv
    assert kernel.target == "gfx950" and kernel.entry_point == "kg_execute_entry"
    work = Path(kernel.soname_path).parent
    assert work.is_dir()
    kernel.close()
    assert not work.exists()
    kernel.close()  # idempotent


def test_packed_fp32_stays_off_with_caller_flags(tmp_path):
    """A caller's own flag list replaces the default one, but every device build still
    turns the packed-fp32 target feature off."""

    fake = _fake_hipcc(tmp_path)
    kernel = ExecutionEngine("gfx950", compiler=str(fake), compiler_flags=("-std=c++17", "-O1")).compile(
        source="int x;", function="f")
    argv = (tmp_path / "argv.log").read_text()
    assert "-O1" in argv and "-Xclang -target-feature -Xclang -packed-fp32-ops" in argv
    kernel.close()


def test_fake_compiler_failure_phrase(tmp_path):
    fake = _fake_hipcc(tmp_path, rc=3)
    with pytest.raises(KernelCodeError) as err:
        ExecutionEngine("gfx950", compiler=str(fake)).compile(source="int x;", function="f")
    assert err.value.failure_phrase == "compile_failed"


@pytest.mark.parametrize("fuse", ["true", "false"])
def test_real_hipcc_builds_generated_source(fuse):
    """hipcc cross-compiles the generated source for gfx950 here (no GPU needed), fused
    glue and per-operation kernel alike, and the shared object exports kg_execute_entry;
    it is loaded but not executed."""

    src = gen_kernel(lower(flash_attention_inputs_static_tile_static_kernel, *((_X4,) * 4), fuse=fuse))
    kernel = ExecutionEngine("gfx950").compile(source=src, function="fa")
    try:
        lib = ctypes.CDLL(kernel.soname_path)
        assert hasattr(lib, "kg_execute_entry")
        fn = lib.kg_execute_entry
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(native.KgArgSlot), ctypes.c_ulonglong]
        slots = (native.KgArgSlot * 3)()
        assert fn(slots, 3) == -1  # arity check in the generated entry, before any GPU work
        assert "expects 4 slots" in native.last_error()
        if fuse == "false":  # include/gfx950/kg_generated.h: the allocation-free entry too
            assert hasattr(lib, "kg_execute_entry_noalloc")
            lib.kg_execute_entry_noalloc.restype = ctypes.c_int
            lib.kg_execute_entry_noalloc.argtypes = fn.argtypes
            assert lib.kg_execute_entry_noalloc(slots, 3) == -1
    finally:
        kernel.close()


def test_execute_phrases_without_gpu(tmp_path):
    fake = _fake_hipcc(tmp_path)
    kernel = ExecutionEngine("gfx950", compiler=str(fake)).compile(source="int x;", function="f")
    with pytest.raises(KernelCodeError) as err:
        kernel.execute(args=None)
    assert err.value.failure_phrase == "runtime_throw_or_abort"
    with pytest.raises(KernelCodeError) as err:
        kernel.execute(args=[1])
    assert err.value.failure_phrase == "runtime_throw_or_abort"
    with pytest.raises(KernelCodeError) as err:
        kernel.execute(args=(), entry_point="other")
    assert err.value.failure_phrase == "symbol_resolve_failed"
    with pytest.raises(KernelCodeError) as err:
        kernel.execute(request=ExecuteRequest(args=(), capture_function_output=True))
    assert err.value.failure_phrase == "function_output_capture_not_supported"
    other = CompiledKernel(target="npu_demo", soname_path=kernel.soname_path, function="f", entry_point="kg_execute_entry")
    with pytest.raises(KernelCodeError) as err:
        other.execute(args=())
    assert err.value.failure_phrase == "execution_unsupported"
    kernel.close()


def test_dsl_run_contract_checks():
    snap = snapshot_config()
    try:
        set_target("npu_demo")
        with pytest.raises(KernelCodeError):
            dsl_run(matmul_inputs_static_tile_static_kernel, (1, 2, 3, None), "gfx950-lowering")
        set_target("gfx950")
        with pytest.raises(KernelCodeError):
            dsl_run(matmul_inputs_static_tile_static_kernel, (1, 2, 3), "gfx950-lowering")  # arity
        with pytest.raises(KernelCodeError):
            dsl_run(matmul_inputs_static_tile_static_kernel, (1, 2, 3, None), "no-such-pipeline")
    finally:
        restore_config(snap)


def test_memory_stage_option_drives_every_fused_ring_depth():
    """memory_stage (MultiBufferAnalysisPass's option, kernel_gen/passes/memory/multi_buffer.py)
    reaches each fused entry as its trailing INT slot: matmul slot 7, attention slot 8 (after
    the causal flag), conv2d slot 17 (after the nest's five tile steps); a per-operation
    kernel, which stages nothing through LDS, is left alone."""

    pm = get_pipeline("gfx950-lowering", {"memory_stage": "3"})
    b16 = T((256, 256), "bfloat16")
    for fn, extra in ((matmul_inputs_static_tile_static_kernel, ()), (matmul_inputs_static_tile_dynamic_kernel, (64, 64, 64))):
        lowered = pm.run(mlir_gen(fn, (b16, b16, b16, None) + extra))
        assert "multi-buffer{memory-stage=3}" in lowered.applied and lowered.memory_stage == 3
        src = gen_kernel(lowered)
        assert "slots[7].int_value = 3LL;" in src and "kg_gfx950_matmul_entry(slots, 8ULL)" in src
    x = T((1, 2, 64, 64), "bfloat16")
    fa = pm.run(mlir_gen(flash_attention_scaled_causal_kernel, (x, x, x, x, 64, 64, 0.1)))
    assert fa.memory_stage == 3
    src = gen_kernel(fa)
    assert "slots[8].int_value = 3LL;" in src and "kg_gfx950_flash_attention_entry(slots, 9ULL)" in src
    conv = pm.run(mlir_gen(conv2d_inputs_static_tile_static_kernel, (_X4, _X4, _X4, None)))
    assert conv.memory_stage == 3
    src = gen_kernel(conv)
    assert "slots[17].int_value = 3LL;" in src and "kg_gfx950_conv2d_entry(slots, 18ULL)" in src
    assert "slots[12].int_value = 7LL;" in src  # the static demo's filter tile step
    per_op = get_pipeline("gfx950-lowering", {"memory_stage": "3", "fuse": "false"})
    assert per_op.run(mlir_gen(flash_attention_scaled_causal_kernel, (x, x, x, x, 64, 64, 0.1))).memory_stage is None
    for bad in ("1", "5", "two"):
        with pytest.raises(KernelCodeError):
            build_gfx950_lowering_pipeline({"memory_stage": bad})


def test_memory_stage_slot_validated_without_gpu():
    lib = native.load_library()
    from kernelcode_generate_amd.native import TensorSpec as T

    base = [T((256, 256), "bfloat16"), T((256, 64), "bfloat16"), T((64, 256), "bfloat16"), None, 64, 64, 64]
    assert native.cost("matmul", base + [2])["MAC"] == 256 * 256 * 64
    x = T((1, 2, 128, 64), "bfloat16")
    fa = [x, x, x, x, 64, 64, 0.125, 0]
    c = T((1, 8, 16, 16), "float16")
    conv = [c, c, T((8, 8, 3, 3), "float16"), None, 1, 1, 1, 1, 1, 1, 1, 1, 8, 8, 1, 8, 8]
    for family, args in (("matmul", base), ("flash_attention", fa), ("conv2d", conv)):
        assert native.cost(family, args + [4])["MAC"] > 0
        for bad in (1, 5):
            with pytest.raises(native.NativeLibraryError, match="memory_stage"):
                native.cost(family, args + [bad])
    assert lib is not None


def test_real_hipcc_builds_every_demo_per_operation():
    """The per-operation kernels of the matmul and conv demo programs (loads, stores, frees,
    reshaped accumulators, img2col) cross-compile too."""

    import numpy as np

    a = np.zeros((4, 4), np.float32)
    x = np.zeros((1, 2, 6, 6), np.float32)
    w = np.zeros((2, 2, 3, 3), np.float32)
    for fn, args in ((matmul_inputs_static_tile_dynamic_kernel, (a, a, a, a[0], 4, 4, 4)),
                     (conv2d_inputs_dynamic_tile_dynamic_kernel, (x, x, w, None, 1, 1, 1, 1, 1, 1, 1, 1, 2, 2, 1, 3, 3))):
        kernel = ExecutionEngine("gfx950").compile(source=gen_kernel(lower(fn, *args, fuse="false")), function="demo")
        try:
            assert hasattr(ctypes.CDLL(kernel.soname_path), "kg_execute_entry")
        finally:
            kernel.close()
