"""Load-time weight preparation on the HIP backend: the hooks `Transmuter.move/2` calls.

`Transmuter.move/2` (lib/transmuter.ex:1104-1182) picks a triple {compatible?, weight,
evaluate} by backend; `Transmuter.EMLX` (lib/transmuter/emlx.ex:86-161) is the one device-
packed precedent. This module is the third branch, with the same signatures:

    compatible(node) -> bool
    weight(node, b, scales, zero_points, model, backend) -> PackedWeight
    evaluate(t) -> t

and `move(model, ctx)` restates the node rewrite of move/2 over this package's model record:
each packable, compatible MatMulNBits node reads [A, "<B>:packed", "", "", ...] afterwards, the
weight is packed once per distinct B, and the B, scales and zero points no other node or graph
output reads leave the params and static values. A second move leaves the model as it is.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace

import numpy as np

from .device import FLOAT_TYPES, Context, DeviceTensor, cast_float, nx_type
from .packed import Int8Weight, PackedWeight
from .quantized import nbits_sizes


@dataclass
class Model:
    """The parts of a loaded model that move/2 reads and writes (lib/transmuter.ex:186-242):
    the nodes in order, the params (device values), the static (host) values, the graph
    outputs, and :compute_type."""

    nodes: list
    params: dict = field(default_factory=dict)
    static: dict = field(default_factory=dict)
    outputs: list = field(default_factory=list)
    compute_type: str | None = None
    backend: object = None
    inputs: list = field(default_factory=list)


def _deferred(value) -> bool:
    """A DeferredTensor of the loader: an initializer still in its external data file."""
    return hasattr(value, "proto") and hasattr(value, "to_device")


def _host_value(value):
    """A host array of a value: a deferred tensor is read (memory-mapped), a device tensor
    copied back."""
    if _deferred(value):
        return value.value()
    if isinstance(value, DeviceTensor):
        return value.numpy()
    return value


def upcast(value, compute_type: str | None):
    """`Transmuter.upcast/2` (lib/transmuter.ex:1323-1324): f16 and bf16 values take the
    compute type (Nx.as_type/2, one rounding from the exact value); other values stay as they
    are. Returns (value, its float type or None)."""
    if value is None:
        return None, None
    try:
        dtype = nx_type(value)
    except TypeError:
        dtype = None
    if compute_type and dtype in ("f16", "bf16") and compute_type != dtype:
        return cast_float(value, compute_type), compute_type
    return value, dtype if dtype in FLOAT_TYPES else None


def compatible(node) -> bool:
    """A MatMulNBits weight the library packs: 2, 4 or 8 bits and a power-of-two block of at
    least 16 weights (any K; the last block may be partial). Compare
    Transmuter.EMLX.compatible?/1 (emlx.ex:94-99), which also requires K % block_size == 0."""
    k, n, bits, block = nbits_sizes(node)
    return bits in (2, 4, 8) and block is not None and block >= 16 and block & (block - 1) == 0 \
        and k > 0 and n > 0


def packable(node, model: Model) -> bool:
    """`packable?/2` (lib/transmuter.ex:1209-1216): scales named, no g_idx, bits in {2,4,8}, and a
    B param of exactly N*K*bits/8 u8 bytes."""
    if node.op_type != "MatMulNBits" or len(node.input) < 3:
        return False
    _a, b, scales, *rest = node.input
    k, n, bits, _block = nbits_sizes(node)
    g_idx = rest[1] if len(rest) > 1 else ""
    value = model.params.get(b)
    if scales == "" or g_idx != "" or bits not in (2, 4, 8) or value is None:
        return False
    if isinstance(value, PackedWeight):
        return False
    if isinstance(value, DeviceTensor):
        dtype, size = value.dtype, value.size
    else:
        dtype = "u8" if np.dtype(value.dtype) == np.uint8 else None
        size = int(np.prod(value.shape, dtype=np.int64))
    return dtype == "u8" and size * 8 == n * k * bits


def weight(node, b, scales, zero_points, model: Model, backend: Context) -> PackedWeight:
    """The packed weight of a MatMulNBits node: its dequantization type is the scales' type
    after :compute_type (dequantized_weight/6, lib/transmuter.ex:1230-1240)."""
    k, n, bits, block = nbits_sizes(node)
    scales, stype = upcast(_host_value(scales), model.compute_type)
    return PackedWeight.upload(backend, _host_value(b), scales, _host_value(zero_points), k=k, n=n, bits=bits,
                               block_size=block, weight_dtype=stype)


def evaluate(t):
    """Finishes a value made on the device: waits until its copies are done."""
    if isinstance(t, (PackedWeight, DeviceTensor)):
        t.ctx.synchronize()
    return t


def _packed_name(b: str) -> str:
    return b + ":packed"


def _packed_inputs(inputs: list, model: Model) -> list:
    """The inputs of a packed node: the weight in place of B, no scales and zero points
    (packed_inputs/2, lib/transmuter.ex:1185-1193)."""
    a, b, *rest = inputs
    name = _packed_name(b)
    if name in model.params or name in model.static:
        raise ValueError(f"the model already has a value named {name}")
    out = [a, name, *rest]
    while len(out) < 4:
        out.append("")
    out[2] = ""
    out[3] = ""
    return out


def move(model: Model, ctx: Context) -> Model:
    """`Transmuter.move/2` (lib/transmuter.ex:1104-1182) with the HIP hooks."""
    packed = [node for node in model.nodes if packable(node, model) and compatible(node)]
    packed_outputs = {node.output[0] for node in packed}
    nodes = [replace(node, input=_packed_inputs(node.input, model)) if node.output and node.output[0] in packed_outputs
             else node for node in model.nodes]
    used = set(model.outputs)
    for node in nodes:
        used.update(node.input)
    freed = {name for node in packed for name in node.input[1:4] if name and name not in used}
    values = {**model.static, **model.params}
    weights = {}
    for node in packed:
        b_name = node.input[1]
        if _packed_name(b_name) in weights:
            continue
        scales = values[node.input[2]]
        zp_name = node.input[3] if len(node.input) > 3 else ""
        zero_points = values.get(zp_name) if zp_name else None
        weights[_packed_name(b_name)] = evaluate(weight(node, values[b_name], scales, zero_points, model, ctx))
    params = {name: _to_device(value, ctx, model.compute_type) for name, value in model.params.items()
              if name not in freed}
    params.update(weights)
    static = {name: value for name, value in model.static.items() if name not in freed}
    # Device copies this move made itself (not the caller's own device tensors) may be released.
    made = {name for name, value in params.items() if value is not model.params.get(name)}
    moved = prepare_matmul_integer(replace(model, nodes=nodes, params=params, static=static, backend=ctx), ctx,
                                   release=made)
    # move/2 ends with Fusion.matmuls/2 (lib/transmuter.ex:1181).
    return merge_matmuls(moved)


# ---------------------------------------------------------------- MatMulInteger B at load


def _int8_name(b: str) -> str:
    return b + ":int8"


def _int8_preparable(node, values: dict) -> bool:
    """A MatMulInteger whose B is a 2-D u8/s8 initializer (and b_zero_point absent or an
    initializer) of a shape the prepared GEMM takes."""
    if node.op_type != "MatMulInteger" or len(node.input) < 2 or not node.input[1]:
        return False
    b = values.get(node.input[1])
    if b is None or isinstance(b, (PackedWeight, Int8Weight)):
        return False
    shape = tuple(b.shape)
    dtype = b.dtype if isinstance(b, DeviceTensor) else getattr(b, "nx_dtype", None) or nx_type(np.asarray(b))
    bz = node.input[3] if len(node.input) > 3 else ""
    if bz and bz not in values:
        return False
    return len(shape) == 2 and dtype in ("u8", "s8") and Int8Weight.supported(*shape)


def prepare_matmul_integer(model: Model, ctx: Context, release=frozenset()) -> Model:
    """MatMulInteger nodes whose B is an initializer read "<B>:int8" afterwards: B transposed once
    into the int8 GEMM's layout with its b_zero_point folded in (no counterpart in move/2, which
    leaves MatMulInteger to the backend's dot; the outputs are the same s32 sums). The node keeps
    A and a_zero_point; B and b_zero_point leave the params when nothing else reads them; those
    named in `release` (the device copies move/2 made itself) are freed at once."""
    values = {**model.static, **model.params}
    prepared = [node for node in model.nodes if _int8_preparable(node, values)]
    if not prepared:
        return model
    prepared_ids = {id(node) for node in prepared}
    weights = {}
    nodes = []
    for node in model.nodes:
        if id(node) not in prepared_ids:
            nodes.append(node)
            continue
        b_name = node.input[1]
        bz_name = node.input[3] if len(node.input) > 3 else ""
        name = _int8_name(b_name) + (f":{bz_name}" if bz_name else "")
        if name not in weights:
            if name in values:
                raise ValueError(f"the model already has a value named {name}")
            # A B already on the device (move/2 put the params there) is prepared from there, with
            # no host round trip; a static (host) B is uploaded by prepare.
            b_val, bz_val = values[b_name], values[bz_name] if bz_name else None
            weights[name] = Int8Weight.prepare(
                ctx, b_val if isinstance(b_val, DeviceTensor) else _host_value(b_val),
                bz_val if bz_val is None or isinstance(bz_val, DeviceTensor) else _host_value(bz_val))
        a_zero = node.input[2] if len(node.input) > 2 else ""
        nodes.append(replace(node, input=[node.input[0], name, a_zero, ""]))
    used = set(model.outputs)
    for node in nodes:
        used.update(node.input)
    freed = {name for node in prepared for name in (node.input[1], node.input[3] if len(node.input) > 3 else "")
             if name and name not in used}
    # The device copies of B and b_zero_point that nothing reads any more are released now rather
    # than when the old params are dropped, so a load does not hold each int8 weight twice.
    for name in freed & set(release):
        value = model.params.get(name)
        if isinstance(value, DeviceTensor):
            value.free()
    params = {name: value for name, value in model.params.items() if name not in freed}
    params.update(weights)
    static = {name: value for name, value in model.static.items() if name not in freed}
    return replace(model, nodes=nodes, params=params, static=static)


def _to_device(value, ctx: Context, compute_type: str | None):
    """A param on the device (move/2 transfers every param to the backend, lib/transmuter.ex:
    1104-1182): packed weights and device tensors stay; a deferred tensor is copied from its
    file; a host array is uploaded, f16/bf16 taking the compute type first."""
    if isinstance(value, (PackedWeight, DeviceTensor)):
        return value
    if _deferred(value) and not (compute_type and value.nx_dtype in ("f16", "bf16")):
        return value.to_device(ctx)
    arr, _dtype = upcast(_host_value(value), compute_type)
    return ctx.put(arr)


# ---------------------------------------------------------------- merged matmuls


def _mergeable(node, model: Model, uses) -> bool:
    """`Fusion.mergeable?/3` (lib/transmuter/fusion.ex:467-476) for packed MatMulNBits: a
    non-empty input A, no other inputs (no bias), and an {N, K} packed weight read once."""
    if node.op_type != "MatMulNBits" or len(node.input) < 2:
        return False
    a, w, *rest = node.input
    weight = model.params.get(w)
    k, n, _bits, _block = nbits_sizes(node)
    return a != "" and all(x == "" for x in rest) and uses.get(w, 0) == 1 \
        and isinstance(weight, PackedWeight) and weight.shape == (n, k)


def merge_matmuls(model: Model) -> Model:
    """`Fusion.matmuls/2` (lib/transmuter/fusion.ex:430-539) on this backend: the MatMulNBits
    nodes that read one input merge into one MatMulNBits over the concatenated packed weights
    (rows of the first, then the next, ...) and a Split of its output along the last axis.
    The merged node keeps the first node's name and reads "<first B>:merged"."""
    from collections import Counter

    from .onnx_wire import ATTR_INT, ATTR_INTS, AttributeProto, NodeProto

    uses = Counter(name for node in model.nodes for name in node.input)
    uses.update(model.outputs)
    groups: dict = {}
    for node in model.nodes:
        if _mergeable(node, model, uses):
            weight = model.params[node.input[1]]
            # The reference's merge key is (op_type, A, type, K) (fusion.ex:467-488); packed
            # weights concatenate only when they also share bits, block size and zero point
            # kind, so a mixed-precision group (an 8-bit v_proj beside 4-bit q/k) splits by
            # layout. Each merged part still computes exactly what its own node did.
            key = (node.op_type, node.input[0], weight.dtype, weight.k, weight.bits, weight.block_size,
                   weight.zp_kind)
            groups.setdefault(key, []).append(node)
    # tmh_weight_concat_nbits takes at most MAX_CONCAT parts: larger groups merge in runs.
    runs = [group[i:i + PackedWeight.MAX_CONCAT] for group in groups.values()
            for i in range(0, len(group), PackedWeight.MAX_CONCAT)]
    params = dict(model.params)
    replacements = {}
    for group in runs:
        if len(group) < 2:
            continue
        first = group[0]
        weights = [params[node.input[1]] for node in group]
        sizes = [w.n for w in weights]
        name = first.input[1] + ":merged"
        output = first.output[0] + ":merged"
        if name in params:
            raise ValueError(f"the model already has a param {name}")
        attrs = [replace(a, i=sum(sizes)) if a.name == "N" else a for a in first.attribute]
        merged = replace(first, input=[first.input[0], name, *first.input[2:]], output=[output], attribute=attrs)
        split = NodeProto(op_type="Split", name=f"{first.name}:split", input=[output],
                          output=[node.output[0] for node in group],
                          attribute=[AttributeProto(name="axis", type=ATTR_INT, i=-1),
                                     AttributeProto(name="split", type=ATTR_INTS, ints=list(sizes))])
        for node in group:
            params.pop(node.input[1])
        params[name] = evaluate(PackedWeight.concat(weights))
        replacements[id(first)] = [merged, split]
        for node in group[1:]:
            replacements[id(node)] = []
    nodes = []
    for node in model.nodes:
        nodes.extend(replacements.get(id(node), [node]))
    return replace(model, nodes=nodes, params=params)


def split_last_axis(x: DeviceTensor, sizes: list[int]) -> list[DeviceTensor]:
    """`Split` along the last axis on the device (tmh_copy_2d per part)."""
    from ._lib import lib
    from .device import NX_TO_NUMPY

    total = x.shape[-1]
    if sum(sizes) != total:
        raise ValueError(f"split sizes {sizes} do not add up to {total}")
    rows = x.size // total if total else 0
    item = np.dtype(NX_TO_NUMPY[x.dtype]).itemsize
    outs, offset = [], 0
    for size in sizes:
        out = x.ctx.empty(x.shape[:-1] + (size,), x.dtype)
        if size and rows:
            src = ctypes_offset(x.ptr, offset * item)
            x.ctx.check(lib().tmh_copy_2d(x.ctx.handle, out.ptr, size * item, src, total * item, size * item, rows, None))
        outs.append(out)
        offset += size
    return outs


def ctypes_offset(ptr, nbytes: int):
    import ctypes

    return ctypes.c_void_p(ptr.value + nbytes)


def run_nodes(model: Model, inputs: dict) -> dict:
    """Walks the nodes in order, as `Transmuter.run_nodes/3` does (lib/transmuter.ex:647-684),
    for graphs of this path: the quantized operators and the Splits of merged matmuls. Returns
    every value the graph outputs name."""
    from . import quantized

    values = {**model.static, **model.params, **inputs}
    for node in model.nodes:
        args = [values[name] if name else None for name in node.input]
        if node.op_type in quantized.op_types():
            outs = quantized.apply(node, args)
        elif node.op_type == "Split":
            split = next(a for a in node.attribute if a.name == "split")
            axis = next(a for a in node.attribute if a.name == "axis").i
            if axis not in (-1, len(args[0].shape) - 1):
                raise NotImplementedError("only Splits along the last axis run here")
            outs = split_last_axis(args[0], list(split.ints))
        else:
            raise NotImplementedError(f"{node.op_type} stays on the Nx backend")
        for name, value in zip(node.output, outs):
            values[name] = value
    return {name: values[name] for name in model.outputs}
