"""Device-resident MatMulNBits weights (tmh_weight handles).

A `PackedWeight` is what `Transmuter.move/2` stores under "<B>:packed" on this backend
(lib/transmuter.ex:1155-1164): the packed bytes, scales and zero points of one weight, kept
packed on the device. Like the MLX quantized tensor of `Transmuter.EMLX.weight/6`
(lib/transmuter/emlx.ex:104-148) it presents as an {N, K} weight, so the MatMulNBits handler
takes its fast branch (`Nx.shape(b) == {n, k}`, lib/transmuter/ops/quantized.ex:39-42).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import lib
from .device import FLOAT_TYPES, NX_TO_TMH, Context, DeviceTensor, nx_type


def _host(x, name: str):
    """A host array of a weight part: numpy as is; a DeviceTensor is copied back."""
    if x is None:
        return None, None
    if isinstance(x, DeviceTensor):
        return np.ascontiguousarray(x.numpy()), x.dtype
    return np.ascontiguousarray(x), nx_type(x)


class PackedWeight:
    """One MatMulNBits weight on the device, in the library's tiled layout."""

    MAX_CONCAT = 8  # parts tmh_weight_concat_nbits takes at once

    def __init__(self, ctx: Context, handle: ctypes.c_void_p, k: int, n: int, bits: int, block_size: int,
                 dtype: str, zp_kind: int = _lib.ZP_NONE):
        self.ctx = ctx
        self.handle = handle
        self.k, self.n, self.bits, self.block_size = k, n, bits, block_size
        self.dtype = dtype  # the type the weights dequantize in
        self.zp_kind = zp_kind  # ZP_NONE, ZP_PACKED or ZP_FLOAT

    @property
    def shape(self) -> tuple[int, int]:
        return (self.n, self.k)

    @classmethod
    def upload(cls, ctx: Context, b, scales, zero_points, *, k: int, n: int, bits: int, block_size: int,
               weight_dtype: str, scales_dtype: str | None = None, zero_points_dtype: str | None = None
               ) -> "PackedWeight":
        """Packs B [N, blocks, block_size*bits/8] (u8), scales [N*blocks] and zero points (none,
        packed u8 rows, or floats) into a device weight whose values dequantize in weight_dtype.
        bf16 host values come as BF16Host arrays; plain uint16 bit patterns need scales_dtype /
        zero_points_dtype."""
        if weight_dtype not in FLOAT_TYPES:
            raise ValueError(f"weight type must be one of {FLOAT_TYPES}, got {weight_dtype}")
        hb, bdt = _host(b, "B")
        if bdt != "u8":
            raise _lib.TmhArgumentError(_lib.ERR_INVALID, f"MatMulNBits B must be u8 bytes, got {bdt}")
        hs, sdt = _host(scales, "scales")
        sdt = scales_dtype or sdt
        hz, zdt = _host(zero_points, "zero_points")
        if hz is None:
            zp_kind, zdt = _lib.ZP_NONE, "u8"
        else:
            zdt = zero_points_dtype or zdt
            zp_kind = _lib.ZP_FLOAT if zdt in FLOAT_TYPES else _lib.ZP_PACKED
        handle = ctypes.c_void_p()
        status = lib().tmh_weight_upload_nbits(
            ctx.handle, hb.ctypes.data_as(ctypes.c_void_p), hb.nbytes,
            hs.ctypes.data_as(ctypes.c_void_p), NX_TO_TMH[sdt], hs.size,
            hz.ctypes.data_as(ctypes.c_void_p) if hz is not None else None, zp_kind, NX_TO_TMH[zdt],
            hz.size if hz is not None else 0, k, n, bits, block_size, NX_TO_TMH[weight_dtype],
            ctypes.byref(handle))
        ctx.check(status)
        return cls(ctx, handle, k, n, bits, block_size, weight_dtype, zp_kind)

    @classmethod
    def pack_device(cls, ctx: Context, b: DeviceTensor, scales: DeviceTensor, zero_points: DeviceTensor | None, *,
                    k: int, n: int, bits: int, block_size: int, weight_dtype: str, stream=None) -> "PackedWeight":
        """The weight of `upload` from buffers already on the device (tmh_weight_pack_nbits): B,
        scales and zero points in their ONNX layouts, repacked by a device kernel on `stream`."""
        if weight_dtype not in FLOAT_TYPES:
            raise ValueError(f"weight type must be one of {FLOAT_TYPES}, got {weight_dtype}")
        if b.dtype != "u8":
            raise _lib.TmhArgumentError(_lib.ERR_INVALID, f"MatMulNBits B must be u8 bytes, got {b.dtype}")
        if zero_points is None:
            zp_kind, zp_code, zp_ptr, zp_count = _lib.ZP_NONE, _lib.U8, None, 0
        else:
            zp_kind = _lib.ZP_FLOAT if zero_points.dtype in FLOAT_TYPES else _lib.ZP_PACKED
            zp_code, zp_ptr, zp_count = zero_points.tmh_dtype, zero_points.ptr, zero_points.size
        handle = ctypes.c_void_p()
        ctx.check(lib().tmh_weight_pack_nbits(ctx.handle, b.ptr, b.nbytes, scales.ptr, scales.tmh_dtype, scales.size,
                                              zp_ptr, zp_kind, zp_code, zp_count, k, n, bits, block_size,
                                              NX_TO_TMH[weight_dtype], stream, ctypes.byref(handle)))
        return cls(ctx, handle, k, n, bits, block_size, weight_dtype, zp_kind)

    @classmethod
    def concat(cls, parts: list["PackedWeight"]) -> "PackedWeight":
        """One weight with the rows of every part in order (tmh_weight_concat_nbits): the
        concatenation of Fusion.matmuls/2 (lib/transmuter/fusion.ex:430-539), kept packed."""
        if not parts:
            raise ValueError("nothing to concatenate")
        ctx = parts[0].ctx
        handles = (ctypes.c_void_p * len(parts))(*[p.handle.value for p in parts])
        handle = ctypes.c_void_p()
        ctx.check(lib().tmh_weight_concat_nbits(ctx.handle, handles, len(parts), ctypes.byref(handle)))
        p0 = parts[0]
        return cls(ctx, handle, p0.k, sum(p.n for p in parts), p0.bits, p0.block_size, p0.dtype, p0.zp_kind)

    def device_bytes(self) -> int:
        size = ctypes.c_size_t()
        _lib.check(lib().tmh_weight_info(self.handle, None, None, None, None, None, ctypes.byref(size)))
        return size.value

    def dequantize(self, dtype: str | None = None, stream=None) -> DeviceTensor:
        """The {N, K} float weights (tmh_dequantize_nbits), in `dtype` (default: its own type)."""
        dtype = dtype or self.dtype
        out = self.ctx.empty((self.n, self.k), dtype)
        self.ctx.check(lib().tmh_dequantize_nbits(self.ctx.handle, self.handle, out.ptr, NX_TO_TMH[dtype], stream))
        return out

    def free(self) -> None:
        if self.handle:
            lib().tmh_weight_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __repr__(self) -> str:
        return f"PackedWeight(N={self.n}, K={self.k}, bits={self.bits}, block_size={self.block_size}, {self.dtype})"


class Int8Weight:
    """A MatMulInteger B prepared once on the device (tmh_int8_weight): B^T as s8 rows of k, its
    column sums and its zero-point terms. What the load-time move stores under "<B>:int8" for a
    MatMulInteger whose B (and b_zero_point) are initializers; the handler then computes what
    MatMulInteger computes over B and b_zero_point (lib/transmuter/ops/quantized.ex:105-110)."""

    def __init__(self, ctx: Context, handle: ctypes.c_void_p, k: int, n: int, dtype: str):
        self.ctx, self.handle, self.k, self.n, self.dtype = ctx, handle, k, n, dtype

    @property
    def shape(self) -> tuple[int, int]:
        return (self.k, self.n)

    PAD = 256  # a prepared B's rows of k are zero-padded to a multiple of this (the C library's kQPad)

    @staticmethod
    def supported(k: int, n: int) -> bool:
        """Shapes tmh_int8_weight_prepare takes: K a multiple of 16, and (N + 128) * K padded to
        256 below 2^31 (the prepared B's 32-bit offsets; the same test as the C library's)."""
        kp = -(-k // Int8Weight.PAD) * Int8Weight.PAD
        return k > 0 and n > 0 and k % 16 == 0 and (n + 128) * kp < 2 ** 31

    @classmethod
    def prepare(cls, ctx: Context, b, b_zero=None) -> "Int8Weight":
        """Prepares B [K, N] (u8 or s8, host or device) with b_zero_point (None, one value or
        [N] of B's type)."""
        b_t = b if isinstance(b, DeviceTensor) else ctx.put(np.ascontiguousarray(b))
        z_t = b_zero if (b_zero is None or isinstance(b_zero, DeviceTensor)) else ctx.put(np.ascontiguousarray(b_zero))
        try:
            if len(b_t.shape) != 2:
                raise _lib.TmhArgumentError(_lib.ERR_INVALID, f"a prepared MatMulInteger B is 2-D, got {b_t.shape}")
            k, n = b_t.shape
            handle = ctypes.c_void_p()
            ctx.check(lib().tmh_int8_weight_prepare(ctx.handle, b_t.ptr, b_t.tmh_dtype,
                                                    z_t.ptr if z_t is not None else None,
                                                    z_t.size if z_t is not None else 0, k, n, None,
                                                    ctypes.byref(handle)))
            ctx.synchronize()
        finally:
            if b_t is not b:
                b_t.free()
            if z_t is not None and z_t is not b_zero:
                z_t.free()
        return cls(ctx, handle, k, n, b_t.dtype)

    def device_bytes(self) -> int:
        size = ctypes.c_size_t()
        _lib.check(lib().tmh_int8_weight_info(self.handle, None, None, ctypes.byref(size)))
        return size.value

    def free(self) -> None:
        if self.handle:
            lib().tmh_int8_weight_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __repr__(self) -> str:
        return f"Int8Weight(K={self.k}, N={self.n}, {self.dtype})"
