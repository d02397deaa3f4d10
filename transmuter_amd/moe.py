"""QMoE on the HIP library: the QMoE handler of `Transmuter.Ops.MoE` (lib/transmuter/ops/moe.ex).

`apply(node, inputs)` takes QMoE's positional inputs (moe.ex:42-45): input, router_probs, then
fc1_w, fc1_scales, fc1_bias, fc2_w, fc2_scales, fc2_bias, fc3_w, fc3_scales, fc3_bias, fc1_zp,
fc2_zp, fc3_zp (None when absent) and its attributes: k, expert_weight_bits (4), block_size (0),
activation_type ("relu"), swiglu_fusion (0), activation_alpha (1.0), activation_beta (0.0),
swiglu_limit (0.0). normalize_routing_weights changes nothing for QMoE: the weights of a token
already add up to 1 after the softmax over its k values (moe.ex:40-41).

Expert weights are packed on the device once per (fc, dtype) as `ExpertWeight`s
(tmh_weight_upload_qmoe); host arrays given to `apply` are packed for that call.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _lib
from ._lib import lib
from .device import FLOAT_TYPES, NX_TO_TMH, Context, DeviceTensor, nx_type
from .quantized import ArgumentError, attr, optional

OP_TYPES = ["QMoE"]


def op_types() -> list[str]:
    return list(OP_TYPES)


def _host(x):
    if x is None:
        return None, None
    if isinstance(x, DeviceTensor):
        return np.ascontiguousarray(x.numpy()), x.dtype
    arr = np.ascontiguousarray(x)
    return arr, nx_type(arr)


class ExpertWeight:
    """The E experts of one QMoE weight input, packed on the device (E*N rows of K values)."""

    def __init__(self, ctx: Context, handle: ctypes.c_void_p, experts: int, n: int, k: int, bits: int, dtype: str):
        self.ctx, self.handle = ctx, handle
        self.experts, self.n, self.k, self.bits, self.dtype = experts, n, k, bits, dtype

    @classmethod
    def upload(cls, ctx: Context, packed, scales, zero_points, *, bits: int, block_size: int, dtype: str,
               scales_dtype: str | None = None) -> "ExpertWeight":
        """packed [E, N, K*bits/8] u8; scales [E, N, blocks] (block_size > 0) or [E, N] / [E, N, 1]
        or None; zero points packed along the blocks or along N (moe.ex:216-253)."""
        w, wdt = _host(packed)
        if wdt != "u8" or w.ndim != 3:
            raise ArgumentError(f"QMoE expert weights must be u8 [E, N, K*bits/8], got {wdt} {w.shape}")
        experts, n, row_bytes = w.shape
        k = row_bytes * 8 // bits
        s, sdt = _host(scales)
        sdt = scales_dtype or sdt
        if s is not None and sdt not in FLOAT_TYPES:
            raise ArgumentError(f"QMoE scales must be float, got {sdt}")
        z, zdt = _host(zero_points)
        if z is not None and zdt not in ("u8",):
            raise ArgumentError(f"QMoE zero points must be packed u8, got {zdt}")
        handle = ctypes.c_void_p()
        ctx.check(lib().tmh_weight_upload_qmoe(
            ctx.handle, w.ctypes.data_as(ctypes.c_void_p), w.nbytes,
            s.ctypes.data_as(ctypes.c_void_p) if s is not None else None, NX_TO_TMH[sdt] if s is not None else 0,
            s.size if s is not None else 0, z.ctypes.data_as(ctypes.c_void_p) if z is not None else None,
            z.nbytes if z is not None else 0, experts, n, k, bits, block_size if s is not None else 0,
            NX_TO_TMH[dtype], ctypes.byref(handle)))
        return cls(ctx, handle, experts, n, k, bits, dtype)

    def free(self) -> None:
        if self.handle:
            lib().tmh_weight_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _expert_weight(ctx, w, s, z, bits, block_size, dtype):
    if w is None or isinstance(w, ExpertWeight):
        return w, False
    return ExpertWeight.upload(ctx, w, s, z, bits=bits, block_size=block_size, dtype=dtype), True


def qmoe(node, inputs: list) -> DeviceTensor:
    """`MoE.op/2` for QMoE (moe.ex:42-61) and experts/4 (:64-102)."""
    x, router, *rest = inputs
    fc1_w, fc1_s, fc1_b, fc2_w, fc2_s, fc2_b, fc3_w, fc3_s, fc3_b, z1, z2, z3 = optional(rest, 12)
    if not isinstance(x, DeviceTensor):
        raise ArgumentError("QMoE input must live on the device")
    ctx = x.ctx
    dtype = x.dtype
    if dtype not in FLOAT_TYPES:
        raise ArgumentError(f"QMoE input must be float, got {dtype}")
    bits = attr(node, "expert_weight_bits", 4)
    block_size = attr(node, "block_size", 0)
    k = attr(node, "k")
    activation = attr(node, "activation_type", "relu")
    if activation not in _lib.ACTIVATIONS:
        raise ArgumentError(f"QMoE activation_type {activation} is not supported")
    fusion = attr(node, "swiglu_fusion", 0)
    alpha = attr(node, "activation_alpha", 1.0)
    beta = attr(node, "activation_beta", 0.0)
    limit = attr(node, "swiglu_limit", 0.0)
    h = x.shape[-1]
    t = math.prod(x.shape[:-1])
    router_t = router if isinstance(router, DeviceTensor) else ctx.put(np.asarray(router))
    experts = router_t.shape[-1]
    owned = []
    weights = []
    for w, s, z in ((fc1_w, fc1_s, z1), (fc2_w, fc2_s, z2), (fc3_w, fc3_s, z3)):
        ew, own = _expert_weight(ctx, w, s, z, bits, block_size, dtype)
        weights.append(ew)
        if own:
            owned.append(ew)
    fc1, fc2, fc3 = weights
    biases = []
    for b in (fc1_b, fc2_b, fc3_b):
        if b is None or isinstance(b, DeviceTensor):
            biases.append(b)
        else:
            bt = ctx.put(np.asarray(b).astype({"f32": np.float32, "f16": np.float16}.get(dtype, np.float32)))
            biases.append(bt)
            owned.append(bt)
    bias_dt = next((b.dtype for b in biases if b is not None), dtype)
    y = ctx.empty(x.shape, dtype)
    try:
        ctx.check(lib().tmh_qmoe(
            ctx.handle, x.ptr, x.tmh_dtype, t, h, router_t.ptr, router_t.tmh_dtype, experts, k, fc1.handle,
            biases[0].ptr if biases[0] is not None else None, fc2.handle,
            biases[1].ptr if biases[1] is not None else None, fc3.handle if fc3 is not None else None,
            biases[2].ptr if biases[2] is not None else None, NX_TO_TMH[bias_dt], _lib.ACTIVATIONS[activation],
            fusion, alpha, beta, limit, y.ptr, None))
    finally:
        ctx.defer_free(*owned, router_t if router_t is not router else None)
    return y


_HANDLERS = {"QMoE": qmoe}


def apply(node, inputs: list) -> list:
    """`MoE.apply/2` (moe.ex:18): the outputs of one node as a list."""
    handler = _HANDLERS.get(node.op_type)
    if handler is None:
        raise NotImplementedError(f"{node.op_type} stays on the Nx backend; the HIP path runs {OP_TYPES}")
    return [handler(node, list(inputs))]
