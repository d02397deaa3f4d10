"""ctypes binding of oracle/_build/liboracle.so (the C restatement; test infrastructure only)."""

from __future__ import annotations

import ctypes
import os

import numpy as np

from .build import LIB, build

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build(verbose=False)
        h = ctypes.CDLL(LIB)
        vp, i64, i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        h.oracle_dequantize_nbits.argtypes = [vp, vp, vp, vp, i64, i64, i, i, i, vp]
        h.oracle_gemm_f32.argtypes = [vp, vp, i64, i64, i64, vp, i]
        h.oracle_gemm_f16w.argtypes = [vp, vp, i64, i64, i64, vp, i]
        h.oracle_matmul_nbits_in_graph.argtypes = [vp, vp, vp, vp, i64, i64, i64, i, i, i, vp, vp, i]
        h.oracle_matmul_integer.argtypes = [vp, i, vp, i, vp, i64, vp, i64, i64, i64, i64, i64, i, vp]
        h.oracle_f32_to_f16_array.argtypes = [vp, vp, i64]
        h.oracle_f16_to_f32_array.argtypes = [vp, vp, i64]
        _lib = h
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def dequantize_nbits(b, scales, zp, k, n, bits, block_size, out_f16=False):
    b = np.ascontiguousarray(b, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    zp_packed = zp_float = None
    if zp is not None:
        zp = np.ascontiguousarray(zp)
        if zp.dtype.kind == "f":
            zp_float = zp.astype(np.float32)
        else:
            zp_packed = zp.astype(np.uint8)
    out = np.empty((n, k), np.uint16 if out_f16 else np.float32)
    st = lib().oracle_dequantize_nbits(_p(b), _p(scales), _p(zp_packed), _p(zp_float), k, n, bits, block_size,
                                       1 if out_f16 else 0, _p(out))
    if st:
        raise ValueError("bad arguments")
    return out.view(np.float16) if out_f16 else out


def gemm(a, w, threads=1):
    """Y = A . W^T with f32 accumulation; w is f32 or f16."""
    a = np.ascontiguousarray(a, np.float32)
    w = np.ascontiguousarray(w)
    m, k = a.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    if w.dtype == np.float16:
        lib().oracle_gemm_f16w(_p(a), _p(w.view(np.uint16)), m, n, k, _p(y), threads)
    else:
        lib().oracle_gemm_f32(_p(a), _p(np.ascontiguousarray(w, np.float32)), m, n, k, _p(y), threads)
    return y


def matmul_nbits_in_graph(a, b, scales, zp, k, n, bits, block_size, f16_weights, threads=1, scratch=None):
    """MatMulNBits without move/2: dequantize W (f16 or f32) on every call, then Y = A . W^T."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    zp = None if zp is None else np.ascontiguousarray(zp, np.uint8)
    if scratch is None:
        scratch = np.empty((n, k), np.uint16 if f16_weights else np.float32)
    y = np.empty((a.shape[0], n), np.float32)
    if lib().oracle_matmul_nbits_in_graph(_p(a), _p(b), _p(scales), _p(zp), a.shape[0], k, n, bits, block_size,
                                          1 if f16_weights else 0, _p(scratch), _p(y), threads):
        raise ValueError("bad arguments")
    return y


def matmul_integer(a, b, az=None, bz=None):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    m, k = a.shape[-2], a.shape[-1]
    n = b.shape[-1]
    batch = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    y = np.empty(a.shape[:-2] + (m, n), np.int32)
    azr = None if az is None else np.ascontiguousarray(az).reshape(-1).view(np.uint8)
    bzr = None if bz is None else np.ascontiguousarray(bz).reshape(-1).view(np.uint8)
    lib().oracle_matmul_integer(_p(a.view(np.uint8)), int(a.dtype == np.int8), _p(b.view(np.uint8)),
                                int(b.dtype == np.int8), _p(azr), 0 if azr is None else azr.size, _p(bzr),
                                0 if bzr is None else bzr.size, batch, m, k, n, int(b.ndim > 2), _p(y))
    return y


def f32_to_f16(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_f16_array(_p(x), _p(out), x.size)
    return out.view(np.float16)
