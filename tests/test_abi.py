"""CPU checks of the gfx950 C ABI: the library loads, exports every symbol include/kg_gfx950.h
declares, and its slot layout is byte-for-byte the reference's _CArgSlot
(kernel_gen/execute_engine/runtime_args.py:217-237). Only argument-validation paths that
return before touching the GPU are called here."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from kernelcode_generate_amd import native

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "kg_gfx950.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:int|const char\*|void\*)\s+(kg_gfx950_\w+)\s*\(", text, flags=re.M)


def test_header_declares_entries():
    names = declared_functions()
    assert set(native.ENTRY_POINTS) <= set(names)
    assert set(native.CONTROL_SYMBOLS) <= set(names)


def test_library_exports_every_declared_symbol():
    lib = native.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.kg_gfx950_abi_version() == 3


def test_slot_layout_matches_reference():
    # _CArgSlot on LP64: int kind (+4 pad); void* data; long long* shape; long long* stride;
    # unsigned long long rank; int dtype_code (+4 pad); long long int_value; double float_value
    expect = [("kind", 0), ("data", 8), ("shape", 16), ("stride", 24), ("rank", 32), ("dtype_code", 40),
              ("int_value", 48), ("float_value", 56)]
    got = [(name, getattr(native.KgArgSlot, name).offset) for name, _ in native.KgArgSlot._fields_]
    assert got == expect
    assert ctypes.sizeof(native.KgArgSlot) == 64


def test_marshal_scalars_and_absent():
    arr, keep = native.marshal_slots((None, 3, 2.5))
    assert arr[0].kind == native.KG_ARG_MEMORY and not arr[0].data and arr[0].rank == 1 and arr[0].shape[0] == 0
    assert arr[1].kind == native.KG_ARG_INT and arr[1].int_value == 3
    assert arr[2].kind == native.KG_ARG_FLOAT and arr[2].float_value == 2.5
    with pytest.raises(native.NativeLibraryError):
        native.marshal_slots((True,))


@pytest.mark.parametrize("entry,count", [("kg_gfx950_matmul_entry", 5), ("kg_gfx950_conv2d_entry", 4),
                                         ("kg_gfx950_flash_attention_entry", 5)])
def test_wrong_arity_is_rejected_without_gpu(entry, count):
    lib = native.load_library()
    fn = getattr(lib, entry)
    slots = (native.KgArgSlot * count)()
    assert fn(slots, count) == -1
    assert "expects" in native.last_error()
    assert fn(None, 0) == -1


def test_wrong_slot_kind_is_rejected_without_gpu():
    lib = native.load_library()
    arr, keep = native.marshal_slots((1, 2, 3, None))
    assert lib.kg_gfx950_matmul_entry(arr, 4) == -1
    assert "expected memory slot" in native.last_error()


def test_mfma_rate_probe_rejects_bad_arguments():
    """bench.py's probe library (libkg_gfx950_probe.so, not the product library) validates
    before touching the GPU: no device is needed here."""
    import ctypes

    import bench

    lib = bench.probe_library()
    tf, ghz = ctypes.c_double(0.0), ctypes.c_double(0.0)
    rate = lib.kg_gfx950_probe_mfma_rate
    assert rate(1, 16, 0, 10, 4, ctypes.byref(tf), ctypes.byref(ghz)) == -1  # fp32: not 16-bit
    assert b"bf16" in lib.kg_gfx950_probe_last_error()
    assert rate(6, 8, 0, 10, 4, ctypes.byref(tf), ctypes.byref(ghz)) == -1
    assert b"mfma_m" in lib.kg_gfx950_probe_last_error()
    assert rate(6, 32, 0, 0, 4, ctypes.byref(tf), ctypes.byref(ghz)) == -1
    assert rate(6, 16, 0, 10, 1 << 17, ctypes.byref(tf), ctypes.byref(ghz)) == -1
    assert not hasattr(native.load_library(), "kg_gfx950_mfma_rate")