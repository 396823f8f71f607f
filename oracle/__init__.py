"""TEST INFRASTRUCTURE ONLY: numpy front end of the C oracle (kg_oracle.c).

The oracle restates, on the CPU, what kernelcode_generate executes on the host for its
matmul / conv2d / flash-attention demos (the npu_demo target): see the header of
kg_oracle.c for the reference files and lines each function follows. It is the checker
for the gfx950 kernels and the timed CPU baseline of bench.py; only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline may import it.

``reference_primitives()`` loads ``_ref/libkg_npu_demo_ref.so``: the reference's own
npu_demo primitives compiled from its headers (see Makefile), used to pin the restated
primitives. It is None where that library has not been built.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
_LIB: dict[str, ctypes.CDLL] = {}

_F = ctypes.POINTER(ctypes.c_float)
_L = ctypes.c_long
_LL = ctypes.c_longlong


def build(reference: bool = False) -> None:
    """Compile the oracle (and, if asked and available, the reference primitives)."""

    targets = ["all"]
    if reference and Path("/root/reference/include/npu_demo/npu_demo.h").is_file():
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), *targets], check=True)


def _lib(optimized: bool = True) -> ctypes.CDLL:
    name = "liboracle.so" if optimized else "liboracle_O0.so"
    if name in _LIB:
        return _LIB[name]
    path = ORACLE_DIR / name
    if not path.is_file():
        build()
    lib = ctypes.CDLL(str(path))
    lib.kgo_matmul.argtypes = [_F, _L, _F, _L, _F, _L, _L, _L, _L, ctypes.c_int]
    lib.kgo_matmul.restype = None
    lib.kgo_img2col2d.argtypes = [_F, _F] + [_L] * 14
    lib.kgo_img2col2d.restype = ctypes.c_int
    lib.kgo_exp.argtypes = [ctypes.c_float]
    lib.kgo_exp.restype = ctypes.c_float
    lib.kgo_reduce_max_rows.argtypes = [_F, _F, _L, _L, _L]
    lib.kgo_reduce_sum_rows.argtypes = [_F, _F, _L, _L, _L]
    lib.kgo_matmul_demo.argtypes = [_F, _F, _F, _F, _L, _L, _L, _L, _L, _L, ctypes.c_int, ctypes.c_int, _L, _L]
    lib.kgo_matmul_demo.restype = None
    lib.kgo_conv2d_demo.argtypes = [_F, _F, _F, _F] + [_L] * 20 + [ctypes.c_int, _L, _L]
    lib.kgo_conv2d_demo.restype = ctypes.c_int
    lib.kgo_flash_attention_demo.argtypes = [_F, _F, _F, _F] + [_L] * 6 + [
        ctypes.c_int,
        ctypes.c_float,
        ctypes.c_int,
        ctypes.c_int,
        _L,
        _L,
    ]
    lib.kgo_flash_attention_demo.restype = None
    _LIB[name] = lib
    return lib


def _f32(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_F)


# ------------------------------------------------------------------------------------
# primitives
# ------------------------------------------------------------------------------------


def matmul(lhs: np.ndarray, rhs: np.ndarray, out: np.ndarray | None = None, acc: bool = False) -> np.ndarray:
    """npu_demo::matmul: sequential-k fp32 (include/npu_demo/Kernel.h:900-948)."""

    lhs, rhs = _f32(lhs), _f32(rhs)
    m, k = lhs.shape
    n = rhs.shape[1]
    res = np.zeros((m, n), np.float32) if out is None else _f32(out).copy()
    _lib().kgo_matmul(_ptr(res), n, _ptr(lhs), k, _ptr(rhs), n, m, n, k, int(acc))
    return res


def img2col2d(x: np.ndarray, kh, kw, sh, sw, dh, dw, ph, pw, pl, pr) -> np.ndarray:
    """npu_demo::img2col2d (Kernel.h:1041-1123); ph/pw = top/bottom, pl/pr = left/right."""

    x = _f32(x)
    n, c, h, w = x.shape
    ho = (h + ph + pw - dh * (kh - 1) - 1) // sh + 1
    wo = (w + pl + pr - dw * (kw - 1) - 1) // sw + 1
    out = np.zeros((n, c, kh, kw, ho, wo), np.float32)
    rc = _lib().kgo_img2col2d(_ptr(out), _ptr(x), n, c, h, w, kh, kw, sh, sw, dh, dw, ph, pw, pl, pr)
    if rc != 0:
        raise ValueError("img2col2d rejected its arguments")
    return out


def exp(x: np.ndarray) -> np.ndarray:
    """npu_demo::exp: (float)exp((double)x) (Kernel.h:621-641)."""

    f = _lib().kgo_exp
    flat = _f32(x).ravel()
    return np.array([f(float(v)) for v in flat], np.float32).reshape(np.shape(x))


def reduce_rows(x: np.ndarray, kind: str) -> np.ndarray:
    """npu_demo::reduce_max / reduce_sum with axis=1, keepdim (Kernel.h:701-750, :831-881)."""

    x = _f32(x)
    rows, cols = x.shape
    out = np.zeros((rows, 1), np.float32)
    fn = _lib().kgo_reduce_max_rows if kind == "max" else _lib().kgo_reduce_sum_rows
    fn(_ptr(out), _ptr(x), rows, cols, cols)
    return out


# ------------------------------------------------------------------------------------
# demo loop nests
# ------------------------------------------------------------------------------------


def matmul_demo(lhs, rhs, bias=None, tiles=(72, 56, 48), *, fused=True, threads=2, m_range=None, optimized=True):
    """kernel/matmul/inputs_static_tile_static.py:56-110 on the npu_demo path."""

    lhs, rhs = _f32(lhs), _f32(rhs)
    b = None if bias is None else _f32(bias)
    m, k = lhs.shape
    n = rhs.shape[1]
    out = np.zeros((m, n), np.float32)
    m_begin, m_end = (0, 0) if m_range is None else m_range
    _lib(optimized).kgo_matmul_demo(
        _ptr(out), _ptr(lhs), _ptr(rhs), _ptr(b), m, n, k, tiles[0], tiles[1], tiles[2], int(fused), threads, m_begin, m_end
    )
    return out


def conv2d_out_hw(h, w, kh, kw, stride, dilation, padding):
    pt, pb, pl, pr = padding
    ho = (h + pt + pb - dilation[0] * (kh - 1) - 1) // stride[0] + 1
    wo = (w + pl + pr - dilation[1] * (kw - 1) - 1) // stride[1] + 1
    return ho, wo


def conv2d_demo(x, w, bias=None, stride=(1, 1), dilation=(1, 1), padding=(0, 0, 0, 0), tiles=(8, 16, 4, 8, 9), *, threads=2,
                f_range=None, optimized=True):
    """kernel/conv2d/inputs_static_tile_static.py:115-215; padding = (top, bottom, left, right)."""

    x, w = _f32(x), _f32(w)
    b = None if bias is None else _f32(bias)
    n, c, h, ww = x.shape
    f, _, kh, kw = w.shape
    ho, wo = conv2d_out_hw(h, ww, kh, kw, stride, dilation, padding)
    out = np.zeros((n, f, ho, wo), np.float32)
    f_begin, f_end = (0, 0) if f_range is None else f_range
    rc = _lib(optimized).kgo_conv2d_demo(
        _ptr(out), _ptr(x), _ptr(w), _ptr(b), n, c, h, ww, f, kh, kw, stride[0], stride[1], dilation[0], dilation[1],
        padding[0], padding[1], padding[2], padding[3], *tiles, threads, f_begin, f_end,
    )
    if rc != 0:
        raise ValueError("conv2d_demo rejected its arguments")
    return out


def flash_attention_demo(q, k, v, br=64, bc=80, *, scale=None, causal=False, threads=2, m_range=None, optimized=True):
    """kernel/flash_attention/inputs_static_tile_static.py:90-190 (+ scale / causal extensions)."""

    q, k, v = _f32(q), _f32(k), _f32(v)
    bsz, h, s, d = q.shape
    out = np.zeros_like(q)
    m_begin, m_end = (0, 0) if m_range is None else m_range
    _lib(optimized).kgo_flash_attention_demo(
        _ptr(out), _ptr(q), _ptr(k), _ptr(v), bsz, h, s, d, br, bc, int(scale is not None),
        float(scale if scale is not None else 1.0), int(causal), threads, m_begin, m_end,
    )
    return out


# ------------------------------------------------------------------------------------
# the reference's own primitives (oracle/_ref)
# ------------------------------------------------------------------------------------


class ReferencePrimitives:
    """npu_demo primitives from the reference headers, via _ref/libkg_npu_demo_ref.so."""

    def __init__(self, lib: ctypes.CDLL) -> None:
        self._lib = lib
        lib.kgr_matmul.argtypes = [_F, _F, _F, _LL, _LL, _LL, ctypes.c_int]
        lib.kgr_img2col2d.argtypes = [_F, _F] + [_LL] * 14
        lib.kgr_exp.argtypes = [_F, _F, _LL, _LL]
        lib.kgr_reduce_rows.argtypes = [_F, _F, _LL, _LL, ctypes.c_int]
        lib.kgr_binary.argtypes = [_F, _F, _F, _LL, _LL, ctypes.c_int]
        for fn in (lib.kgr_matmul, lib.kgr_img2col2d, lib.kgr_exp, lib.kgr_reduce_rows, lib.kgr_binary):
            fn.restype = ctypes.c_int

    def matmul(self, lhs, rhs, out=None, acc=False):
        lhs, rhs = _f32(lhs), _f32(rhs)
        m, k = lhs.shape
        n = rhs.shape[1]
        res = np.zeros((m, n), np.float32) if out is None else _f32(out).copy()
        assert self._lib.kgr_matmul(_ptr(res), _ptr(lhs), _ptr(rhs), m, n, k, int(acc)) == 0
        return res

    def img2col2d(self, x, kh, kw, sh, sw, dh, dw, ph, pw, pl, pr):
        x = _f32(x)
        n, c, h, w = x.shape
        ho = (h + ph + pw - dh * (kh - 1) - 1) // sh + 1
        wo = (w + pl + pr - dw * (kw - 1) - 1) // sw + 1
        out = np.zeros((n, c, kh, kw, ho, wo), np.float32)
        rc = self._lib.kgr_img2col2d(_ptr(out), _ptr(x), n, c, h, w, kh, kw, sh, sw, dh, dw, ph, pw, pl, pr)
        if rc != 0:
            raise ValueError("reference img2col2d returned kError")
        return out

    def exp(self, x):
        x = _f32(np.atleast_2d(x))
        out = np.zeros_like(x)
        assert self._lib.kgr_exp(_ptr(out), _ptr(x), x.shape[0], x.shape[1]) == 0
        return out

    def reduce_rows(self, x, kind):
        x = _f32(x)
        out = np.zeros((x.shape[0], 1), np.float32)
        assert self._lib.kgr_reduce_rows(_ptr(out), _ptr(x), x.shape[0], x.shape[1], int(kind == "max")) == 0
        return out

    def binary(self, lhs, rhs, op):
        codes = {"max": 0, "truediv": 1, "sub": 2, "mul": 3, "add": 4}
        lhs, rhs = _f32(np.atleast_2d(lhs)), _f32(np.atleast_2d(rhs))
        out = np.zeros_like(lhs)
        assert self._lib.kgr_binary(_ptr(out), _ptr(lhs), _ptr(rhs), lhs.shape[0], lhs.shape[1], codes[op]) == 0
        return out


def reference_primitives() -> ReferencePrimitives | None:
    path = ORACLE_DIR / "_ref" / "libkg_npu_demo_ref.so"
    if not path.is_file():
        return None
    return ReferencePrimitives(ctypes.CDLL(str(path)))
