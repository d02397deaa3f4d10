"""Device context and device-resident tensors over the C ABI of libtmhip.

Types are named as Nx names them ("f32", "f16", "bf16", "u8", "s8", "s32", "s64", ...). bf16
host arrays are uint16 bit patterns in a `BF16Host` array, which `nx_type` names "bf16".
"""

from __future__ import annotations

import ctypes
import os
import math

import numpy as np

from . import _lib
from ._lib import check, lib

NX_TO_TMH = {
    "f32": _lib.F32, "f16": _lib.F16, "bf16": _lib.BF16,
    "u8": _lib.U8, "s8": _lib.S8, "u16": _lib.U16, "s16": _lib.S16,
    "s32": _lib.S32, "s64": _lib.S64,
}
NX_TO_NUMPY = {
    "f32": np.float32, "f16": np.float16, "bf16": np.uint16,
    "u8": np.uint8, "s8": np.int8, "u16": np.uint16, "s16": np.int16,
    "s32": np.int32, "s64": np.int64,
}
NUMPY_TO_NX = {
    np.dtype(np.float32): "f32", np.dtype(np.float16): "f16",
    np.dtype(np.uint8): "u8", np.dtype(np.int8): "s8", np.dtype(np.uint16): "u16",
    np.dtype(np.int16): "s16", np.dtype(np.int32): "s32", np.dtype(np.int64): "s64",
}
FLOAT_TYPES = ("f32", "f16", "bf16")


class BF16Host(np.ndarray):
    """A host array of bfloat16 values held as their uint16 bit patterns (numpy has no bfloat16
    type). Its views and slices keep the type; `nx_type` names it "bf16" where a plain uint16
    array is "u16"."""


def bf16_host(bits) -> BF16Host:
    """uint16 bit patterns as a BF16Host array (a view when `bits` already is uint16)."""
    return np.asarray(bits, dtype=np.uint16).view(BF16Host)


def f32_to_bf16_bits(x) -> np.ndarray:
    """f32 values rounded to bfloat16 (to nearest, ties to even; NaN stays a quiet NaN)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    out = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def bf16_bits_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def float_values(array) -> np.ndarray:
    """The f32 values of a float host array (f16, f32, or bf16 bit patterns)."""
    if isinstance(array, BF16Host):
        return bf16_bits_to_f32(array)
    return np.asarray(array, dtype=np.float32)


def cast_float(array, dtype: str) -> np.ndarray:
    """A float host array in another float type ("f32", "f16" or "bf16"), each value rounded
    once from its exact f32 value, as Nx.as_type/2 does."""
    values = float_values(array)
    if dtype == "f32":
        return values
    if dtype == "f16":
        return values.astype(np.float16)
    if dtype == "bf16":
        return bf16_host(f32_to_bf16_bits(values))
    raise ValueError(f"{dtype} is not a float type")


def nx_type(array: np.ndarray) -> str:
    if isinstance(array, BF16Host):
        return "bf16"
    try:
        return NUMPY_TO_NX[np.asarray(array).dtype]
    except KeyError:
        raise TypeError(f"no device type for {np.asarray(array).dtype}") from None


def merge_types(a: str, b: str) -> str:
    """Nx.Type.merge/2 for the float types the operators produce."""
    return a if a == b else "f32"


def _device_nbytes(obj) -> int:
    """Device bytes a temporary holds (a tensor's buffer, a packed weight's tiles)."""
    if hasattr(obj, "device_bytes"):
        try:
            return obj.device_bytes()
        except Exception:
            return 0
    return getattr(obj, "nbytes", 0)


class Context:
    """One device and its stream (tmh_ctx).

    Temporaries of an asynchronous call (inputs a handler uploaded, a weight it repacked) are
    handed to `defer_free` instead of being freed after a synchronize: an event recorded behind
    the call's work fences them, and they are freed once that work is done, at the next point
    where the host waits anyway (`synchronize`, a download) or when more than DEFER_LIMIT bytes
    are waiting. hipFree itself waits for the device, so a free right after a launch would cost
    the round trip the deferral saves."""

    DEFER_LIMIT = 1 << 30

    def __init__(self, device: int = 0):
        handle = ctypes.c_void_p()
        check(lib().tmh_ctx_create(device, ctypes.byref(handle)))
        self.handle = handle
        self.device = device
        self._pending = []  # (event, [objects]) in record order
        self._pending_bytes = 0
        self._events = []  # recycled events

    def defer_free(self, *objs, stream=None) -> None:
        """Frees `objs` (DeviceTensor, PackedWeight or anything with free()) once the work queued
        on `stream` (None: the context's) so far has finished."""
        objs = [o for o in objs if o is not None]
        if not objs:
            return
        ev = self._events.pop() if self._events else None
        if ev is None:
            ev = ctypes.c_void_p()
            self.check(lib().tmh_event_create(self.handle, ctypes.byref(ev)))
        self.check(lib().tmh_event_record(self.handle, ev, stream))
        self._pending.append((ev, objs))
        self._pending_bytes += sum(_device_nbytes(o) for o in objs)
        if self._pending_bytes > self.DEFER_LIMIT:
            self.synchronize()

    def pending_frees(self) -> int:
        """Temporaries waiting for their work to finish."""
        return sum(len(objs) for _ev, objs in self._pending)

    def reap(self) -> None:
        """Frees the deferred temporaries whose work has finished (it never waits)."""
        if not self._pending:
            return
        keep = []
        done = ctypes.c_int()
        for ev, objs in self._pending:
            self.check(lib().tmh_event_query(self.handle, ev, ctypes.byref(done)))
            if not done.value:
                keep.append((ev, objs))
                continue
            for o in objs:
                o.free()
            self._events.append(ev)
        self._pending = keep
        self._pending_bytes = sum(_device_nbytes(o) for _ev, objs in keep for o in objs)

    @property
    def stream(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(lib().tmh_ctx_stream(self.handle))

    def check(self, status: int) -> None:
        check(status, self.handle)

    def alloc(self, nbytes: int) -> ctypes.c_void_p:
        ptr = ctypes.c_void_p()
        self.check(lib().tmh_alloc(self.handle, nbytes, ctypes.byref(ptr)))
        return ptr

    def free(self, ptr) -> None:
        self.check(lib().tmh_free(self.handle, ptr))

    def empty(self, shape, dtype: str) -> "DeviceTensor":
        shape = tuple(int(s) for s in shape)
        nbytes = math.prod(shape) * np.dtype(NX_TO_NUMPY[dtype]).itemsize
        return DeviceTensor(self, self.alloc(nbytes), shape, dtype, nbytes)

    def put(self, array: np.ndarray, dtype: str | None = None) -> "DeviceTensor":
        """Copies a host array to the device. `dtype` names bf16 for uint16 bit patterns. The
        tensor keeps the array's shape, rank 0 included (np.ascontiguousarray alone makes a 0-d
        array 1-d)."""
        shape = np.shape(array)
        dtype = dtype or nx_type(array)
        host = np.ascontiguousarray(array)
        t = self.empty(shape, dtype)
        if t.nbytes:
            self.check(lib().tmh_upload(self.handle, t.ptr, host.ctypes.data_as(ctypes.c_void_p), t.nbytes))
        return t

    def put_file(self, path: str, offset: int, shape, dtype: str) -> "DeviceTensor":
        """A tensor whose bytes lie in a file at `offset` (an ONNX external data file), copied
        to the device without a host copy of the whole tensor (tmh_upload_file)."""
        t = self.empty(shape, dtype)
        if t.nbytes:
            self.check(lib().tmh_upload_file(self.handle, t.ptr, os.fsencode(path), offset, t.nbytes))
        return t

    def synchronize(self) -> None:
        self.check(lib().tmh_synchronize(self.handle, None))
        self.reap()

    def close(self) -> None:
        if self.handle:
            if self._pending:
                lib().tmh_synchronize(self.handle, None)
                for _ev, objs in self._pending:
                    for o in objs:
                        try:
                            o.free()
                        except Exception:
                            pass
                self._events.extend(ev for ev, _objs in self._pending)
                self._pending = []
            for ev in self._events:
                lib().tmh_event_destroy(self.handle, ev)
            self._events = []
            lib().tmh_ctx_destroy(self.handle)
            self.handle = None


class DeviceTensor:
    """A device buffer with a shape and an Nx type, owned by this object."""

    def __init__(self, ctx: Context, ptr, shape, dtype: str, nbytes: int):
        self.ctx = ctx
        self.ptr = ptr
        self.shape = tuple(shape)
        self.dtype = dtype
        self.nbytes = nbytes

    @property
    def size(self) -> int:
        return math.prod(self.shape)

    @property
    def tmh_dtype(self) -> int:
        return NX_TO_TMH[self.dtype]

    def numpy(self) -> np.ndarray:
        """A host copy (bf16 as a BF16Host array of bit patterns)."""
        host = np.empty(self.shape, dtype=NX_TO_NUMPY[self.dtype])
        if self.nbytes:
            self.ctx.check(lib().tmh_download(self.ctx.handle, host.ctypes.data_as(ctypes.c_void_p),
                                              self.ptr, self.nbytes))
            self.ctx.reap()  # the download drained the context's stream
        return bf16_host(host) if self.dtype == "bf16" else host

    def reshape(self, shape) -> "DeviceTensor":
        """A view with another shape over the same buffer (the view does not own it)."""
        shape = tuple(int(s) for s in shape)
        if math.prod(shape) != self.size:
            raise ValueError(f"cannot reshape {self.shape} to {shape}")
        view = DeviceTensor(self.ctx, self.ptr, shape, self.dtype, self.nbytes)
        view._base = self
        view._owner = False
        return view

    def free(self) -> None:
        if getattr(self, "_owner", True) and self.ptr:
            self.ctx.free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            if getattr(self, "_owner", True) and self.ptr and self.ctx.handle:
                lib().tmh_free(self.ctx.handle, self.ptr)
                self.ptr = None
        except Exception:
            pass

    def __repr__(self) -> str:
        return f"DeviceTensor({self.shape}, {self.dtype})"
