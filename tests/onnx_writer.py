"""A minimal writer of the ONNX protobuf messages the loader tests need (ModelProto, GraphProto,
NodeProto, AttributeProto, TensorProto with raw or external data), by field number."""

from __future__ import annotations

import struct

import numpy as np

DTYPES = {np.dtype(np.float32): 1, np.dtype(np.uint8): 2, np.dtype(np.int8): 3, np.dtype(np.int32): 6,
          np.dtype(np.int64): 7, np.dtype(np.float16): 10}


def _varint(v: int) -> bytes:
    v &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        out.append(b | (0x80 if v else 0))
        if not v:
            return bytes(out)


def _key(number: int, wire: int) -> bytes:
    return _varint(number << 3 | wire)


def _len(number: int, payload: bytes) -> bytes:
    return _key(number, 2) + _varint(len(payload)) + payload


def _int(number: int, v: int) -> bytes:
    return _key(number, 0) + _varint(v)


def tensor(name: str, array: np.ndarray, external: tuple[str, int] | None = None) -> bytes:
    """A TensorProto: raw data inline, or (location, offset) in an external file (the caller
    writes the bytes there)."""
    arr = np.ascontiguousarray(array)
    out = b"".join(_int(1, d) for d in arr.shape) + _int(2, DTYPES[arr.dtype]) + _len(8, name.encode())
    if external is None:
        return out + _len(9, arr.tobytes())
    location, offset = external
    entries = [("location", location), ("offset", str(offset)), ("length", str(arr.nbytes))]
    for k, v in entries:
        out += _len(13, _len(1, k.encode()) + _len(2, v.encode()))
    return out + _int(14, 1)


def tensor_raw(name: str, dims: list[int], data_type: int, raw: bytes) -> bytes:
    """A TensorProto of any ONNX data type from its raw bytes (e.g. UINT4 = 21, INT4 = 22, two
    values per byte, the lower element in the low nibble)."""
    out = b"".join(_int(1, d) for d in dims) + _int(2, data_type) + _len(8, name.encode())
    return out + _len(9, raw)


def attribute_int(name: str, value: int) -> bytes:
    return _len(1, name.encode()) + _int(20, 2) + _int(3, value)


def node(op_type: str, inputs: list[str], outputs: list[str], attributes: list[bytes], domain: str = "") -> bytes:
    out = b"".join(_len(1, i.encode()) for i in inputs) + b"".join(_len(2, o.encode()) for o in outputs)
    out += _len(4, op_type.encode()) + b"".join(_len(5, a) for a in attributes)
    return out + (_len(7, domain.encode()) if domain else b"")


def model(nodes: list[bytes], initializers: list[bytes], inputs: list[str], outputs: list[str]) -> bytes:
    graph = b"".join(_len(1, n) for n in nodes) + _len(2, b"g") + b"".join(_len(5, t) for t in initializers)
    graph += b"".join(_len(11, _len(1, i.encode())) for i in inputs)
    graph += b"".join(_len(12, _len(1, o.encode())) for o in outputs)
    opsets = _len(8, _len(1, b"") + _int(2, 21)) + _len(8, _len(1, b"com.microsoft") + _int(2, 1))
    return _int(1, 8) + opsets + _len(7, graph)


def float32(v: float) -> bytes:
    return struct.pack("<f", v)
