"""Reads the reference's operator fixtures (tests/golden/ops/<case>): one ONNX graph, raw
little-endian inputs and ONNX Runtime outputs, and meta.json, as the reference's
test/transmuter/ops_test.exs:478-619 reads them."""

from __future__ import annotations

import json
import os

import numpy as np

from transmuter_amd import onnx_wire

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ops")

NX_DTYPES = {
    "f32": np.float32, "f16": np.float16, "f64": np.float64,
    "s64": np.int64, "s32": np.int32, "s16": np.int16, "s8": np.int8,
    "u64": np.uint64, "u32": np.uint32, "u16": np.uint16, "u8": np.uint8,
}


class Fixture:
    def __init__(self, name: str):
        self.name = name
        self.dir = os.path.join(GOLDEN, name)
        with open(os.path.join(self.dir, "meta.json")) as f:
            self.meta = json.load(f)
        self.model = onnx_wire.load_model(os.path.join(self.dir, self.meta["onnx_path"]))
        self.nodes = self.model.graph.node
        self.initializers = {t.name: onnx_wire.tensor(t, self.dir) for t in self.model.graph.initializer}
        self.inputs = {spec["name"]: self._read(spec) for spec in self.meta["inputs"]}
        self.outputs = {spec["name"]: self._read(spec) for spec in self.meta["outputs"]}
        self.atol = self.meta.get("atol")

    def _read(self, spec):
        data = np.fromfile(os.path.join(self.dir, spec["file"]), dtype=NX_DTYPES[spec["dtype"]])
        return data.reshape(spec["shape"])

    @property
    def node(self):
        assert len(self.nodes) == 1, self.name
        return self.nodes[0]

    def values(self) -> dict:
        """Every named value of the graph: graph inputs and initializers."""
        return {**self.initializers, **self.inputs}

    def node_inputs(self, node=None) -> list:
        """The positional inputs of a node, None for an empty name (lib/transmuter.ex:796)."""
        node = node or self.node
        values = self.values()
        return [values[name] if name else None for name in node.input]


def attrs(node) -> dict:
    out = {}
    for a in node.attribute:
        t = a.type
        if t == onnx_wire.ATTR_INT:
            out[a.name] = a.i
        elif t == onnx_wire.ATTR_FLOAT:
            out[a.name] = a.f
        elif t == onnx_wire.ATTR_STRING:
            out[a.name] = a.s.decode()
        elif t == onnx_wire.ATTR_INTS:
            out[a.name] = list(a.ints)
        elif t == onnx_wire.ATTR_FLOATS:
            out[a.name] = list(a.floats)
    return out


def names(prefix: str) -> list[str]:
    return sorted(d for d in os.listdir(GOLDEN) if d.startswith(prefix))


def tolerance(expected: np.ndarray) -> float:
    """1e-4 + 1e-3 * max|expected| over the finite expected values (ops_test.exs:579-598)."""
    e = np.asarray(expected, dtype=np.float64)
    finite = np.isfinite(e)
    scale = np.abs(e[finite]).max() if finite.any() else 0.0
    return 1e-4 + 1e-3 * scale


def max_diff(actual, expected) -> float:
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    same = (np.isnan(a) & np.isnan(e)) | (a == e)
    d = np.where(same, 0.0, np.abs(a - e))
    return float(d.max()) if d.size else 0.0
