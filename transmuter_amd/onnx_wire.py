"""A minimal reader of the ONNX protobuf wire format, for single-node operator graphs.

Transmuter decodes `.onnx` files with a generated protobuf module (lib/transmuter/onnx.pb.ex:
NodeProto :4638, AttributeProto :574, TensorProto :1913, GraphProto :2724, ModelProto :6417).
This module decodes the same messages, by field number, into plain Python objects whose
attribute names follow those structs (`op_type`, `domain`, `input`, `output`, `attribute`),
so the operator handlers read a node as the reference's handlers do.

Only the fields the quantized operators need are decoded; every other field is skipped.
Initializers decode as `Ops.tensor/2` does (lib/transmuter/ops.ex:597-670): raw little-endian
data, or the typed repeated fields, and 4-bit tensors (ONNX types 21/22) stay packed two
values per byte, as u8 (uint4) or s8 (int4), with the last axis halved (ops.ex:632-639).
"""

from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field

import numpy as np

from .device import bf16_host

# ONNX TensorProto.DataType -> numpy dtype (lib/transmuter/ops.ex:700-713).
ONNX_DTYPES = {
    1: np.float32,
    2: np.uint8,
    3: np.int8,
    4: np.uint16,
    5: np.int16,
    6: np.int32,
    7: np.int64,
    9: np.uint8,  # bool
    10: np.float16,
    11: np.float64,
    12: np.uint32,
    13: np.uint64,
}
BFLOAT16 = 16
UINT4 = 21
INT4 = 22

# AttributeProto.AttributeType
ATTR_FLOAT, ATTR_INT, ATTR_STRING, ATTR_TENSOR, ATTR_GRAPH = 1, 2, 3, 4, 5
ATTR_FLOATS, ATTR_INTS, ATTR_STRINGS = 6, 7, 8


def _varint(buf: bytes, pos: int) -> tuple[int, int]:
    result = 0
    shift = 0
    while True:
        if pos >= len(buf):
            raise ValueError("truncated varint")
        b = buf[pos]
        pos += 1
        result |= (b & 0x7F) << shift
        if not b & 0x80:
            return result, pos
        shift += 7
        if shift > 70:
            raise ValueError("varint too long")


def _text(v) -> str:
    return (v.tobytes() if isinstance(v, memoryview) else v).decode()


def _signed64(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


def fields(buf: bytes):
    """Yields (field_number, wire_type, value) for each field of one message.

    value is an int for varints, bytes for length-delimited fields, and the raw 4 or 8 bytes
    for fixed-width fields.
    """
    pos = 0
    n = len(buf)
    while pos < n:
        key, pos = _varint(buf, pos)
        number, wire = key >> 3, key & 7
        if wire == 0:
            value, pos = _varint(buf, pos)
        elif wire == 1:
            value, pos = buf[pos:pos + 8], pos + 8
        elif wire == 2:
            length, pos = _varint(buf, pos)
            value, pos = buf[pos:pos + length], pos + length
        elif wire == 5:
            value, pos = buf[pos:pos + 4], pos + 4
        else:
            raise ValueError(f"unsupported wire type {wire}")
        if pos > n:
            raise ValueError("truncated message")
        yield number, wire, value


def _packed_varints(value, wire) -> list[int]:
    if wire == 0:
        return [value]
    out, pos = [], 0
    while pos < len(value):
        v, pos = _varint(value, pos)
        out.append(v)
    return out


def _packed_fixed(value, wire, fmt: str, size: int) -> list:
    if wire in (1, 5):
        return [struct.unpack("<" + fmt, value)[0]]
    return list(struct.unpack("<%d%s" % (len(value) // size, fmt), value))


@dataclass
class TensorProto:
    name: str = ""
    dims: list = field(default_factory=list)
    data_type: int = 0
    raw_data: bytes = b""
    float_data: list = field(default_factory=list)
    int32_data: list = field(default_factory=list)
    int64_data: list = field(default_factory=list)
    double_data: list = field(default_factory=list)
    uint64_data: list = field(default_factory=list)
    external_data: dict = field(default_factory=dict)
    data_location: int = 0


@dataclass
class AttributeProto:
    name: str = ""
    type: int = 0
    f: float = 0.0
    i: int = 0
    s: bytes = b""
    t: TensorProto | None = None
    floats: list = field(default_factory=list)
    ints: list = field(default_factory=list)
    strings: list = field(default_factory=list)


@dataclass
class NodeProto:
    input: list = field(default_factory=list)
    output: list = field(default_factory=list)
    name: str = ""
    op_type: str = ""
    domain: str = ""
    attribute: list = field(default_factory=list)


@dataclass
class GraphProto:
    name: str = ""
    node: list = field(default_factory=list)
    initializer: list = field(default_factory=list)
    input: list = field(default_factory=list)
    output: list = field(default_factory=list)


@dataclass
class ModelProto:
    ir_version: int = 0
    opset_import: dict = field(default_factory=dict)
    graph: GraphProto | None = None


def decode_tensor(buf: bytes) -> TensorProto:
    t = TensorProto()
    for number, wire, value in fields(buf):
        if number == 1:
            t.dims.extend(_signed64(v) for v in _packed_varints(value, wire))
        elif number == 2:
            t.data_type = value
        elif number == 4:
            t.float_data.extend(_packed_fixed(value, wire, "f", 4))
        elif number == 5:
            t.int32_data.extend(_signed64(v) for v in _packed_varints(value, wire))
        elif number == 7:
            t.int64_data.extend(_signed64(v) for v in _packed_varints(value, wire))
        elif number == 8:
            t.name = _text(value)
        elif number == 9:
            # A view into the model's buffer when it is a memoryview (a mapped file): no copy.
            t.raw_data = value if isinstance(value, memoryview) else bytes(value)
        elif number == 10:
            t.double_data.extend(_packed_fixed(value, wire, "d", 8))
        elif number == 11:
            t.uint64_data.extend(_packed_varints(value, wire))
        elif number == 13:
            key = val = ""
            for n2, _w2, v2 in fields(value):
                if n2 == 1:
                    key = _text(v2)
                elif n2 == 2:
                    val = _text(v2)
            t.external_data[key] = val
        elif number == 14:
            t.data_location = value
    return t


def decode_attribute(buf: bytes) -> AttributeProto:
    a = AttributeProto()
    for number, wire, value in fields(buf):
        if number == 1:
            a.name = _text(value)
        elif number == 20:
            a.type = value
        elif number == 2:
            a.f = struct.unpack("<f", value)[0]
        elif number == 3:
            a.i = _signed64(value)
        elif number == 4:
            a.s = bytes(value)
        elif number == 5:
            a.t = decode_tensor(value)
        elif number == 7:
            a.floats.extend(_packed_fixed(value, wire, "f", 4))
        elif number == 8:
            a.ints.extend(_signed64(v) for v in _packed_varints(value, wire))
        elif number == 9:
            a.strings.append(bytes(value))
    return a


def decode_node(buf: bytes) -> NodeProto:
    node = NodeProto()
    for number, _wire, value in fields(buf):
        if number == 1:
            node.input.append(_text(value))
        elif number == 2:
            node.output.append(_text(value))
        elif number == 3:
            node.name = _text(value)
        elif number == 4:
            node.op_type = _text(value)
        elif number == 5:
            node.attribute.append(decode_attribute(value))
        elif number == 7:
            node.domain = _text(value)
    return node


def _value_info_name(buf: bytes) -> str:
    for number, _wire, value in fields(buf):
        if number == 1:
            return _text(value)
    return ""


def decode_graph(buf: bytes) -> GraphProto:
    g = GraphProto()
    for number, _wire, value in fields(buf):
        if number == 1:
            g.node.append(decode_node(value))
        elif number == 2:
            g.name = _text(value)
        elif number == 5:
            g.initializer.append(decode_tensor(value))
        elif number == 11:
            g.input.append(_value_info_name(value))
        elif number == 12:
            g.output.append(_value_info_name(value))
    return g


def decode_model(buf: bytes) -> ModelProto:
    m = ModelProto()
    for number, _wire, value in fields(buf):
        if number == 1:
            m.ir_version = value
        elif number == 7:
            m.graph = decode_graph(value)
        elif number == 8:
            domain, version = "", 0
            for n2, _w2, v2 in fields(value):
                if n2 == 1:
                    domain = _text(v2)
                elif n2 == 2:
                    version = _signed64(v2)
            m.opset_import[domain] = version
    if m.graph is None:
        raise ValueError("the model has no graph")
    return m


def load_model(path: str, mapped: bool = False) -> ModelProto:
    """Decodes an .onnx file. With mapped=True the file is memory-mapped and the raw data of the
    initializers are views into the mapping (no copy of the weights)."""
    if mapped:
        import mmap

        with open(path, "rb") as f:
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        return decode_model(memoryview(mm))
    with open(path, "rb") as f:
        return decode_model(f.read())


def _bf16_to_f32(raw: np.ndarray) -> np.ndarray:
    return (raw.astype(np.uint32) << 16).view(np.float32)


def tensor(t: TensorProto, directory: str | None = None) -> np.ndarray:
    """The value of an initializer, as `Ops.tensor/2` gives it (lib/transmuter/ops.ex:597-670).

    uint4/int4 tensors stay packed: the last axis holds ceil(last/2) bytes, u8 for uint4 and s8
    for int4 (ops.ex:632-639). bfloat16 data returns as a BF16Host array of the raw bits
    (uint16 elements that nx_type names "bf16"); callers that compute read it with `bf16_to_f32`.
    """
    if t.data_location == 1:
        t = _read_external(t, directory)
    dims = list(t.dims)
    if t.data_type in (UINT4, INT4):
        last = dims[-1] if dims else 1
        shape = dims[:-1] + [(last + 1) // 2]
        dtype = np.int8 if t.data_type == INT4 else np.uint8
        raw = t.raw_data if t.raw_data else bytes(v & 0xFF for v in t.int32_data)
        return np.frombuffer(raw, dtype=dtype).reshape(shape).copy()
    if t.data_type == BFLOAT16:
        if t.raw_data:
            flat = np.frombuffer(t.raw_data, dtype=np.uint16)
        else:
            flat = np.asarray(t.int32_data, dtype=np.uint16)
        return bf16_host(flat.reshape(dims).copy())
    if t.data_type not in ONNX_DTYPES:
        raise ValueError(f"ONNX type {t.data_type} has no array type here")
    dtype = ONNX_DTYPES[t.data_type]
    if t.raw_data:
        flat = np.frombuffer(t.raw_data, dtype=dtype)
    elif t.float_data:
        flat = np.asarray(t.float_data, dtype=dtype)
    elif t.int64_data:
        flat = np.asarray(t.int64_data, dtype=dtype)
    elif t.int32_data:
        if dtype == np.float16:
            flat = np.asarray(t.int32_data, dtype=np.uint16).view(np.float16)
        else:
            flat = np.asarray(t.int32_data).astype(dtype)
    elif t.double_data:
        flat = np.asarray(t.double_data, dtype=dtype)
    elif t.uint64_data:
        flat = np.asarray(t.uint64_data, dtype=dtype)
    else:
        flat = np.zeros(0, dtype=dtype)
    return flat.reshape(dims).copy()


def external_location(t: TensorProto, directory: str | None) -> tuple[str, int, int]:
    """(path, offset, length) of a tensor kept in an external data file (ops.ex:674-697):
    without a length, the data runs to the end of the file."""
    if directory is None:
        raise ValueError(f"tensor {t.name} keeps its data in a file, and no directory is known")
    path = os.path.join(directory, t.external_data["location"])
    offset = int(t.external_data.get("offset", "0"))
    length = t.external_data.get("length")
    length = int(length) if length is not None else os.path.getsize(path) - offset
    return path, offset, length


def shape_type(t: TensorProto) -> tuple[tuple, np.dtype] | None:
    """The shape and array type `tensor` gives for t, without its data
    (`Ops.tensor_shape_type/1`, ops.ex:610-625); None for types not held here."""
    dims = list(t.dims)
    if t.data_type in (UINT4, INT4):
        last = dims[-1] if dims else 1
        return tuple(dims[:-1] + [(last + 1) // 2]), np.dtype(np.int8 if t.data_type == INT4 else np.uint8)
    if t.data_type == BFLOAT16:
        return tuple(dims), np.dtype(np.uint16)
    if t.data_type in ONNX_DTYPES:
        return tuple(dims), np.dtype(ONNX_DTYPES[t.data_type])
    return None


def tensor_view(t: TensorProto, directory: str | None = None) -> np.ndarray:
    """`tensor` without copies where the data allows: raw data becomes a read-only view of the
    model's buffer, and external data a read-only memory map of its file."""
    st = shape_type(t)
    if st is not None and t.data_location == 1:
        path, offset, length = external_location(t, directory)
        shape, dtype = st
        if length != int(np.prod(shape, dtype=np.int64)) * dtype.itemsize:
            raise ValueError(f"tensor {t.name}: {length} bytes in {path} do not hold {shape} {dtype}")
        view = np.memmap(path, dtype=dtype, mode="r", offset=offset, shape=shape)
        return bf16_host(view) if t.data_type == BFLOAT16 else view
    if st is not None and len(t.raw_data):
        shape, dtype = st
        view = np.frombuffer(t.raw_data, dtype=dtype).reshape(shape)
        return bf16_host(view) if t.data_type == BFLOAT16 else view
    return tensor(t, directory)


def _read_external(t: TensorProto, directory: str | None) -> TensorProto:
    """Reads external data as `Ops.read_external/2` does (lib/transmuter/ops.ex:674-697)."""
    path, offset, length = external_location(t, directory)
    with open(path, "rb") as f:
        f.seek(offset)
        raw = f.read(length)
    return TensorProto(name=t.name, dims=t.dims, data_type=t.data_type, raw_data=raw)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return _bf16_to_f32(np.asarray(bits, dtype=np.uint16))
