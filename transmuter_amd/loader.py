"""Loading an ONNX model onto this path: the initializer handling of `Transmuter.load!/2`
(lib/transmuter.ex:144-242) with the HIP backend.

Initializers split into static values (host arrays: empty tensors, integer tensors of at most
4096 values, float tensors of at most 16 values when not trainable; lib/transmuter.ex:
1310-1320) and params. With a backend, a param kept in an external data file is a
`DeferredTensor` (lib/transmuter/deferred_tensor.ex) that the move reads: a MatMulNBits B is
packed from a read-only memory map of its file, and any other param is copied from the file
to the device through pinned staging buffers (tmh_upload_file), so no host copy of the whole
file data exists at once and no weight is ever expanded to floats on the host. Inline raw data
is read through a memory map of the .onnx file as well.
"""

from __future__ import annotations

import os

import numpy as np

from . import onnx_wire
from .device import Context, DeviceTensor, nx_type
from .hip import Model, move, upcast

STATIC_MAX_SIZE = 16  # @static_max_size (lib/transmuter.ex:31)
STATIC_INT_MAX_SIZE = 4096  # @static_int_max_size (lib/transmuter.ex:32)


class DeferredTensor:
    """An initializer in the external data file, read when the move takes it
    (`Transmuter.DeferredTensor`, lib/transmuter/deferred_tensor.ex)."""

    def __init__(self, shape: tuple, dtype: np.dtype, proto, directory: str):
        self.shape, self.dtype, self.proto, self.directory = shape, dtype, proto, directory

    @classmethod
    def new(cls, proto, directory: str) -> "DeferredTensor | None":
        """The deferred tensor of an external initializer, or None (DeferredTensor.new/2)."""
        if proto.data_location != 1:
            return None
        st = onnx_wire.shape_type(proto)
        if st is None or 0 in st[0]:
            return None
        return cls(st[0], st[1], proto, directory)

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    def value(self) -> np.ndarray:
        """The tensor, as a read-only memory map of the file (DeferredTensor.value/1)."""
        return onnx_wire.tensor_view(self.proto, self.directory)

    @property
    def nx_dtype(self) -> str:
        """The tensor's Nx type ("bf16" for bfloat16 initializers, held as uint16 bits)."""
        return "bf16" if self.proto.data_type == onnx_wire.BFLOAT16 else nx_type(np.zeros(0, self.dtype))

    def to_device(self, ctx: Context) -> DeviceTensor:
        """The tensor on the device, copied from the file without a host copy."""
        path, offset, _length = onnx_wire.external_location(self.proto, self.directory)
        return ctx.put_file(path, offset, self.shape, self.nx_dtype)


def static_initializer(shape: tuple, dtype: np.dtype, trainable: bool = False) -> bool:
    """`static_initializer?/2` (lib/transmuter.ex:1310-1320)."""
    size = int(np.prod(shape, dtype=np.int64))
    if size == 0:
        return True
    if np.dtype(dtype).kind in "iub":
        return size <= STATIC_INT_MAX_SIZE
    return not trainable and size <= STATIC_MAX_SIZE


def load(path: str, ctx: Context | None = None, compute_type: str | None = None, trainable: bool = False) -> Model:
    """The model of an .onnx file with its initializers split as load!/2 splits them; with a
    context, the params move to the device (`move/2`: packed MatMulNBits weights, other params
    as device tensors)."""
    proto = onnx_wire.load_model(path, mapped=True)
    directory = os.path.dirname(os.path.abspath(path))
    graph = proto.graph
    static, params = {}, {}
    for t in graph.initializer:
        value = DeferredTensor.new(t, directory) if ctx is not None else None
        if value is None:
            value = onnx_wire.tensor_view(t, directory)
        if static_initializer(value.shape, value.dtype, trainable):
            static[t.name] = upcast(_host_copy(value), compute_type)[0]
        else:
            params[t.name] = value
    initializers = {t.name for t in graph.initializer}
    model = Model(nodes=list(graph.node), params=params, static=static, outputs=list(graph.output),
                  compute_type=compute_type, inputs=[i for i in graph.input if i not in initializers])
    if ctx is not None:
        return move(model, ctx)
    model.params = {name: upcast(v, compute_type)[0] for name, v in params.items()}
    return model


def _host_copy(value) -> np.ndarray:
    """An in-memory copy of an initializer (of its file mapping), keeping a bf16 tag."""
    if isinstance(value, DeferredTensor):
        value = value.value()
    return np.array(value, subok=True)
