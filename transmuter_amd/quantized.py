"""The quantized operators on the HIP library: the handlers of `Transmuter.Ops.Quantized`.

Mirrors lib/transmuter/ops/quantized.ex: `op_types/0`, `apply/2` (one node, its positional
inputs, a list of outputs), `nbits_sizes/1`, and the same attributes, defaults and errors.
Inputs are `DeviceTensor`s on one context; quantization parameters may also be host arrays
(the reference keeps small initializers as static host values, lib/transmuter.ex:29-32).
A missing optional input is None (lib/transmuter.ex:796).

The operators of the quantized-weight path run on the GPU: MatMulNBits (:30-46),
GatherBlockQuantized (:49-66), DequantizeLinear (:70-84), MatMulInteger (:105-110) and the
DynamicQuantizeLinear (:94-103) that feeds it u8 activations. The other handlers of the
reference's op list (:19-21) stay on the Nx backend and raise here.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _lib
from ._lib import TmhArgumentError, lib
from .device import FLOAT_TYPES, NX_TO_TMH, Context, DeviceTensor, merge_types, nx_type
from .onnx_wire import ATTR_FLOAT, ATTR_FLOATS, ATTR_INT, ATTR_INTS, ATTR_STRING, ATTR_TENSOR
from .packed import Int8Weight, PackedWeight

OP_TYPES = ["MatMulNBits", "GatherBlockQuantized", "DequantizeLinear", "MatMulInteger", "DynamicQuantizeLinear"]
# The reference's other quantized handlers (quantized.ex:19-21), not on this path.
NX_OP_TYPES = ["QuantizeLinear", "ConvInteger", "QLinearMatMul",
               "QLinearConv", "QLinearAdd", "QLinearMul"]


class ArgumentError(TmhArgumentError):
    """The reference's ArgumentError (unsupported attribute or input)."""

    def __init__(self, message: str):
        super().__init__(_lib.ERR_UNSUPPORTED, message)


def op_types() -> list[str]:
    return list(OP_TYPES)


def attr(node, name: str, default=None):
    """`Ops.attr/3` (lib/transmuter/ops.ex:582-594)."""
    for a in node.attribute:
        if a.name != name:
            continue
        if a.type == ATTR_INT:
            return a.i
        if a.type == ATTR_INTS:
            return list(a.ints)
        if a.type == ATTR_FLOAT:
            return a.f
        if a.type == ATTR_FLOATS:
            return list(a.floats)
        if a.type == ATTR_STRING:  # an Elixir binary: text
            return a.s.decode() if isinstance(a.s, bytes) else a.s
        if a.type == ATTR_TENSOR:
            return a.t
    return default


def optional(inputs: list, count: int) -> list:
    """`Ops.optional/2` (lib/transmuter/ops.ex:446): pads with None to `count` values."""
    return (list(inputs) + [None] * count)[:count]


def normalize_axis(axis: int, rank: int) -> int:
    """`Ops.normalize_axis/2` (lib/transmuter/ops.ex:435-436)."""
    return axis + rank if axis < 0 else axis


def nbits_sizes(node) -> tuple[int, int, int, int]:
    """`Quantized.nbits_sizes/1` (quantized.ex:226-228): {K, N, bits (4 by default), block_size}."""
    return attr(node, "K"), attr(node, "N"), attr(node, "bits", 4), attr(node, "block_size")


def apply(node, inputs: list) -> list:
    """`Quantized.apply/2` (quantized.ex:27): the outputs of one node as a list."""
    handler = _HANDLERS.get(node.op_type)
    if handler is None:
        if node.op_type in NX_OP_TYPES:
            raise NotImplementedError(f"{node.op_type} stays on the Nx backend; the HIP path runs {OP_TYPES}")
        raise ValueError(f"{node.op_type} is not a quantized operator")
    out = handler(node, list(inputs))
    return out if isinstance(out, list) else [out]


# ---------------------------------------------------------------- helpers


def _ctx_of(*values) -> Context:
    for v in values:
        if isinstance(v, (DeviceTensor, PackedWeight)):
            return v.ctx
    raise ValueError("no input lives on a device")


def _device(ctx: Context, x, dtype: str | None = None) -> tuple[DeviceTensor | None, bool]:
    """x on the device; True when this call uploaded it (and must free it)."""
    if x is None:
        return None, False
    if isinstance(x, DeviceTensor):
        return x, False
    return ctx.put(x if isinstance(x, np.ndarray) else np.asarray(x), dtype), True


def _ptr_offset(t: DeviceTensor, elements: int) -> ctypes.c_void_p:
    item = np.dtype({"f32": np.float32, "f16": np.float16, "bf16": np.uint16, "u8": np.uint8, "s8": np.int8,
                     "s32": np.int32, "s64": np.int64, "u16": np.uint16, "s16": np.int16}[t.dtype]).itemsize
    if t.ptr.value is None:  # a tensor of no bytes has no buffer; the ABI takes NULL with zero sizes
        return ctypes.c_void_p(None)
    return ctypes.c_void_p(t.ptr.value + elements * item)


def _type_of(x) -> str:
    return x.dtype if isinstance(x, (DeviceTensor, PackedWeight)) else nx_type(np.asarray(x))


def _shape_of(x) -> tuple:
    return tuple(x.shape) if isinstance(x, (DeviceTensor, PackedWeight)) else np.asarray(x).shape


# ---------------------------------------------------------------- MatMulNBits


def matmul_nbits(a: DeviceTensor, w: PackedWeight, bias=None, stream=None) -> DeviceTensor:
    """Y = A . W^T (+ bias) over a packed weight: Nx.dot(a, [-1], w, [1]) and Nx.add (:44-45).
    A is [..., K]; Y is [..., N] in the merged type of A and W (then of the bias)."""
    ctx = a.ctx
    if a.dtype not in FLOAT_TYPES:
        raise ArgumentError(f"MatMulNBits A must be a float tensor, got {a.dtype}")
    if a.shape[-1] != w.k:
        raise ArgumentError(f"MatMulNBits A has {a.shape[-1]} columns, K is {w.k}")
    m = math.prod(a.shape[:-1])
    dot_type = merge_types(a.dtype, w.dtype)
    bias_t, own_bias = _device(ctx, bias)
    y_type = merge_types(dot_type, bias_t.dtype) if bias_t is not None else dot_type
    y = ctx.empty(a.shape[:-1] + (w.n,), y_type)
    try:
        ctx.check(lib().tmh_matmul_nbits(
            ctx.handle, w.handle, a.ptr, a.tmh_dtype, m, w.k, bias_t.ptr if bias_t is not None else None,
            bias_t.tmh_dtype if bias_t is not None else 0, y.ptr, NX_TO_TMH[y_type], w.n, stream))
    finally:
        if own_bias:
            ctx.defer_free(bias_t, stream=stream)
    return y


def _op_matmul_nbits(node, inputs):
    a, b, scales, *rest = inputs
    zero_points, g_idx, bias = optional(rest, 3)
    if g_idx is not None:
        raise ArgumentError("MatMulNBits with the g_idx input is not supported")
    k, n, bits, block_size = nbits_sizes(node)
    # B given as an {N, K} weight (a moved model) needs no unpacking (quantized.ex:38-42).
    if isinstance(b, PackedWeight) and b.shape == (n, k):
        return matmul_nbits(a, b, bias)
    # In the graph, the weights dequantize in A's type (quantized.ex:42), at every call and on the
    # device: a B that lives there is repacked by a device kernel (small host-side scales and zero
    # points, static values in the reference, are copied up first); a host B is packed on the host.
    ctx = a.ctx
    temps = []
    if isinstance(b, DeviceTensor):
        parts = []
        for x in (scales, zero_points):
            t, own = _device(ctx, x)
            parts.append(t)
            if own:
                temps.append(t)
        w = PackedWeight.pack_device(ctx, b, parts[0], parts[1], k=k, n=n, bits=bits, block_size=block_size,
                                     weight_dtype=a.dtype)
    else:
        w = PackedWeight.upload(ctx, b, scales, zero_points, k=k, n=n, bits=bits, block_size=block_size,
                                weight_dtype=a.dtype)
    try:
        return matmul_nbits(a, w, bias)
    finally:
        # Freed once the call's work is done, without a wait here.
        ctx.defer_free(w, *temps)


# ---------------------------------------------------------------- GatherBlockQuantized


def _op_gather_block_quantized(node, inputs):
    data, indices, scales, *rest = inputs
    zero_points = rest[0] if rest else None
    ctx = _ctx_of(data, indices, scales, zero_points)
    dshape = _shape_of(data)
    last = len(dshape) - 1
    if not (attr(node, "gather_axis", 0) == 0 and normalize_axis(attr(node, "quantize_axis", 1), len(dshape)) == last):
        raise ArgumentError("GatherBlockQuantized supports gather_axis 0 and quantize_axis on the last axis")
    bits = attr(node, "bits", 4)
    if bits not in (2, 4, 8):
        raise ArgumentError(f"GatherBlockQuantized bits must be 2, 4 or 8, got {bits}")
    dtype = _type_of(scales)
    if dtype not in FLOAT_TYPES:
        raise ArgumentError(f"GatherBlockQuantized scales must be float, got {dtype}")
    if _type_of(data) not in ("u8", "s8"):
        raise ArgumentError(f"GatherBlockQuantized data must be u8 or s8 bytes, got {_type_of(data)}")
    sshape = _shape_of(scales)
    if sshape[0] != dshape[0] or math.prod(sshape[1:-1]) != math.prod(dshape[1:-1]):
        raise ArgumentError(f"GatherBlockQuantized scales {sshape} do not match data {dshape}")
    blocks_per_row = math.prod(sshape[1:])
    if zero_points is not None:
        zshape = _shape_of(zero_points)
        if _type_of(zero_points) in FLOAT_TYPES:
            expect = dshape[0] * blocks_per_row
        else:
            expect = dshape[0] * -(-blocks_per_row * bits // 8)
        if math.prod(zshape) != expect:
            raise ArgumentError(f"GatherBlockQuantized zero points {zshape} hold {math.prod(zshape)} values, "
                                f"{expect} expected")
    data_t, own_d = _device(ctx, data)
    ids_t, own_i = _device(ctx, indices)
    sc_t, own_s = _device(ctx, scales, dtype)
    zp_t, own_z = _device(ctx, zero_points)
    try:
        rows = dshape[0]
        row_bytes = math.prod(dshape[1:])
        sshape = _shape_of(scales)
        blocks = math.prod(sshape[1:])
        per = 8 // bits
        out_shape = tuple(_shape_of(indices)) + tuple(dshape[1:-1]) + (dshape[-1] * per,)
        out = ctx.empty(out_shape, dtype)
        ctx.check(lib().tmh_gather_block_quantized(
            ctx.handle, data_t.ptr, data_t.tmh_dtype, rows, row_bytes, ids_t.ptr, ids_t.tmh_dtype, ids_t.size,
            sc_t.ptr, sc_t.tmh_dtype, blocks, zp_t.ptr if zp_t is not None else None,
            zp_t.tmh_dtype if zp_t is not None else 0, bits, out.ptr, None))
    finally:
        ctx.defer_free(*[t for t, own in ((data_t, own_d), (ids_t, own_i), (sc_t, own_s), (zp_t, own_z)) if own])
    return out


# ---------------------------------------------------------------- DequantizeLinear


def _op_dequantize_linear(node, inputs):
    x, scale, *rest = inputs
    zero = rest[0] if rest else None
    ctx = _ctx_of(x, scale, zero)
    shape = _shape_of(x)
    rank = len(shape)
    out_type = _type_of(scale)
    if out_type not in FLOAT_TYPES:
        raise ArgumentError(f"DequantizeLinear scale must be float, got {out_type}")
    sshape = _shape_of(scale)
    ssize = math.prod(sshape)
    block_size = attr(node, "block_size", 0)
    if rank == 0:
        outer, dim, inner, axis = 1, 1, 1, 0
    else:
        axis = normalize_axis(attr(node, "axis", 1), rank)
        if not 0 <= axis < rank:
            raise ArgumentError(f"DequantizeLinear axis {attr(node, 'axis', 1)} is out of range for rank {rank}")
        outer, dim, inner = math.prod(shape[:axis]), shape[axis], math.prod(shape[axis + 1:])
    # expand_quant_param/3 (quantized.ex:328-353): one value, blocks along the axis, or the axis.
    if ssize == 1:
        mode = _lib.QPARAM_TENSOR
    elif block_size > 0:
        mode = _lib.QPARAM_BLOCKED
        expect = tuple(shape[:axis]) + (-(-dim // block_size),) + tuple(shape[axis + 1:])
        if tuple(sshape) != expect:
            raise ArgumentError(f"blocked DequantizeLinear scale has shape {sshape}, expected {expect}")
    else:
        mode = _lib.QPARAM_AXIS
        if ssize != dim:
            raise ArgumentError(f"DequantizeLinear scale has {ssize} values for an axis of {dim}")
    if zero is not None and math.prod(_shape_of(zero)) != ssize:
        raise ArgumentError("DequantizeLinear zero point and scale differ in size")
    x_t, own_x = _device(ctx, x)
    s_t, own_s = _device(ctx, scale, out_type)
    z_t, own_z = _device(ctx, zero)
    try:
        y = ctx.empty(shape, out_type)
        ctx.check(lib().tmh_dequantize_linear(
            ctx.handle, x_t.ptr, x_t.tmh_dtype, outer, dim, inner, s_t.ptr, s_t.tmh_dtype,
            z_t.ptr if z_t is not None else None, z_t.tmh_dtype if z_t is not None else 0, mode,
            block_size, y.ptr, None))
    finally:
        ctx.defer_free(*[t for t, own in ((x_t, own_x), (s_t, own_s), (z_t, own_z)) if own])
    return y


# ---------------------------------------------------------------- MatMulInteger


def _op_matmul_integer(node, inputs):
    a, b, *rest = inputs
    a_zero, b_zero = optional(rest, 2)
    if isinstance(b, Int8Weight):
        return _matmul_integer_prepared(a, b, a_zero, b_zero)
    ctx = _ctx_of(a, b, a_zero, b_zero)
    ashape, bshape = _shape_of(a), _shape_of(b)
    if len(ashape) < 1 or len(bshape) < 2:
        raise ArgumentError(f"MatMulInteger of shapes {ashape} and {bshape} is not supported")
    squeeze = len(ashape) == 1
    if squeeze:
        ashape = (1,) + tuple(ashape)
    m, k = ashape[-2], ashape[-1]
    kb, n = bshape[-2], bshape[-1]
    if k != kb:
        raise ArgumentError(f"MatMulInteger contracts {k} with {kb}")
    a_batch, b_batch = tuple(ashape[:-2]), tuple(bshape[:-2])
    if b_batch and a_batch and a_batch != b_batch:
        raise ArgumentError(f"MatMulInteger batch shapes {a_batch} and {b_batch} differ")
    batch_shape = a_batch or b_batch
    batch = math.prod(batch_shape) if batch_shape else 1
    for zero, size, what in ((a_zero, m, "a_zero_point"), (b_zero, n, "b_zero_point")):
        if zero is not None and math.prod(_shape_of(zero)) not in (1, size):
            raise ArgumentError(f"MatMulInteger {what} has {math.prod(_shape_of(zero))} values")
    a_t, own_a = _device(ctx, a)
    b_t, own_b = _device(ctx, b)
    az_t, own_az = _device(ctx, a_zero)
    bz_t, own_bz = _device(ctx, b_zero)
    try:
        out_shape = tuple(batch_shape) + (m, n)
        y = ctx.empty(out_shape, "s32")
        args = (az_t.ptr if az_t is not None else None, az_t.size if az_t is not None else 0,
                bz_t.ptr if bz_t is not None else None, bz_t.size if bz_t is not None else 0)
        if a_batch or not b_batch:
            ctx.check(lib().tmh_matmul_integer(ctx.handle, a_t.ptr, a_t.tmh_dtype, b_t.ptr, b_t.tmh_dtype, *args,
                                               batch, m, k, n, 1 if b_batch else 0, y.ptr, None))
        else:
            # A plain matrix applies to every batch of b (Ops.matmul/2, ops.ex:477-483).
            for i in range(batch):
                ctx.check(lib().tmh_matmul_integer(ctx.handle, a_t.ptr, a_t.tmh_dtype, _ptr_offset(b_t, i * k * n),
                                                   b_t.tmh_dtype, *args, 1, m, k, n, 0,
                                                   _ptr_offset(y, i * m * n), None))
    finally:
        ctx.defer_free(*[t for t, own in ((a_t, own_a), (b_t, own_b), (az_t, own_az), (bz_t, own_bz)) if own])
    if squeeze:
        return y.reshape(out_shape[:-2] + (n,))
    return y


def _matmul_integer_prepared(a, w: "Int8Weight", a_zero, b_zero):
    """MatMulInteger over a B prepared at load (its b_zero_point is part of it): the same s32
    sums as the plain path, through tmh_matmul_integer_prepared."""
    if b_zero is not None:
        raise ArgumentError("a prepared MatMulInteger B carries its own b_zero_point")
    ctx = w.ctx
    ashape = _shape_of(a)
    if len(ashape) < 1:
        raise ArgumentError(f"MatMulInteger of shape {ashape} is not supported")
    squeeze = len(ashape) == 1
    if squeeze:
        ashape = (1,) + tuple(ashape)
    m, k = ashape[-2], ashape[-1]
    if k != w.k:
        raise ArgumentError(f"MatMulInteger contracts {k} with {w.k}")
    batch_shape = tuple(ashape[:-2])
    batch = math.prod(batch_shape) if batch_shape else 1
    if a_zero is not None and math.prod(_shape_of(a_zero)) not in (1, m):
        raise ArgumentError(f"MatMulInteger a_zero_point has {math.prod(_shape_of(a_zero))} values")
    a_t, own_a = _device(ctx, a)
    az_t, own_az = _device(ctx, a_zero)
    temps = [t for t, own in ((a_t, own_a), (az_t, own_az)) if own]
    try:
        out_shape = batch_shape + (m, w.n)
        y = ctx.empty(out_shape, "s32")
        if a_t.ptr.value and a_t.ptr.value % 16:
            # The prepared GEMM streams A 16 bytes at a time: an A that does not start on a 16-byte
            # boundary (an offset view) is copied to a fresh buffer first.
            a_al = ctx.empty(a_t.shape, a_t.dtype)
            temps.append(a_al)
            ctx.check(lib().tmh_copy_2d(ctx.handle, a_al.ptr, a_t.nbytes, a_t.ptr, a_t.nbytes, a_t.nbytes, 1, None))
            a_t = a_al
        rows = _prepared_rows(k)
        per_row_zero = az_t is not None and az_t.size == m and m > 1
        if m <= rows:
            ctx.check(lib().tmh_matmul_integer_prepared(ctx.handle, a_t.ptr, a_t.tmh_dtype,
                                                        az_t.ptr if az_t is not None else None,
                                                        az_t.size if az_t is not None else 0, batch, m, w.handle,
                                                        y.ptr, None))
        else:
            # One launch addresses (rows + 128) * K bytes of A with 32-bit offsets: longer A goes in
            # blocks of rows, batch by batch (row offsets keep A 16-byte aligned, K being a
            # multiple of 16).
            for bi in range(batch):
                for r0 in range(0, m, rows):
                    mb = min(rows, m - r0)
                    zero = _ptr_offset(az_t, r0) if per_row_zero else (az_t.ptr if az_t is not None else None)
                    zcount = mb if per_row_zero else (az_t.size if az_t is not None else 0)
                    ctx.check(lib().tmh_matmul_integer_prepared(
                        ctx.handle, _ptr_offset(a_t, (bi * m + r0) * k), a_t.tmh_dtype, zero, zcount, 1, mb,
                        w.handle, _ptr_offset(y, (bi * m + r0) * w.n), None))
    finally:
        ctx.defer_free(*temps)
    if squeeze:
        return y.reshape(out_shape[:-2] + (w.n,))
    return y


# Rows of A one prepared MatMulInteger launch takes: its 32-bit offsets cover (rows + 128) * K
# bytes of A. None: the largest count that fits; tests set a small value to reach the row blocks.
PREPARED_ROW_LIMIT = None


def _prepared_rows(k: int) -> int:
    fit = (2 ** 31 - 1) // k - 128
    return max(1, min(fit, PREPARED_ROW_LIMIT) if PREPARED_ROW_LIMIT else fit)


# ---------------------------------------------------------------- DynamicQuantizeLinear


def _op_dynamic_quantize_linear(node, inputs):
    """[y, scale, zero] of quantized.ex:94-103: u8 y of x's shape, f32 scale and u8 zero point
    as scalars, all on the device."""
    (x,) = inputs[:1]
    ctx = _ctx_of(x)
    if _type_of(x) != "f32":
        raise ArgumentError(f"DynamicQuantizeLinear takes f32 values, got {_type_of(x)}")
    x_t, own = _device(ctx, x)
    try:
        y = ctx.empty(tuple(_shape_of(x)), "u8")
        scale = ctx.empty((), "f32")
        zero = ctx.empty((), "u8")
        ctx.check(lib().tmh_dynamic_quantize_linear(ctx.handle, x_t.ptr, x_t.tmh_dtype, x_t.size, y.ptr, scale.ptr,
                                                    zero.ptr, None))
    finally:
        if own:
            ctx.defer_free(x_t)
    return [y, scale, zero]


_HANDLERS = {
    "MatMulNBits": _op_matmul_nbits,
    "GatherBlockQuantized": _op_gather_block_quantized,
    "DequantizeLinear": _op_dequantize_linear,
    "MatMulInteger": _op_matmul_integer,
    "DynamicQuantizeLinear": _op_dynamic_quantize_linear,
}
