"""The loader on the CPU: initializers split into static values and params as load!/2 splits
them (lib/transmuter.ex:1310-1320), external data read through memory maps, deferred tensors
(lib/transmuter/deferred_tensor.ex) only with a backend."""

import numpy as np

import synth_model
from transmuter_amd import onnx_wire
from transmuter_amd.loader import DeferredTensor, load, static_initializer


def test_load_without_backend_reads_every_initializer(tmp_path):
    path, values = synth_model.write(str(tmp_path))
    model = load(path)
    # B (12288 u8) and scales (768 f16) and extra (64 f32) are params; zp (384 u8) is static.
    assert set(model.params) == {"B", "scales", "extra"}
    assert set(model.static) == {"zp"}
    for name in ("B", "scales", "extra"):
        assert np.array_equal(np.asarray(model.params[name]), values[name]), name
    assert np.array_equal(model.static["zp"], values["zp"])
    assert model.inputs == ["A"] and model.outputs == ["Y"]
    assert model.nodes[0].op_type == "MatMulNBits"


def test_external_data_is_a_memory_map(tmp_path):
    path, values = synth_model.write(str(tmp_path))
    proto = onnx_wire.load_model(path, mapped=True)
    b = next(t for t in proto.graph.initializer if t.name == "B")
    loc = onnx_wire.external_location(b, str(tmp_path))
    assert loc == (str(tmp_path / "weights.bin"), 100, values["B"].nbytes)
    view = onnx_wire.tensor_view(b, str(tmp_path))
    assert isinstance(view, np.memmap) and np.array_equal(view, values["B"])
    scales = next(t for t in proto.graph.initializer if t.name == "scales")
    sv = onnx_wire.tensor_view(scales)
    assert not sv.flags.owndata and np.array_equal(sv, values["scales"])  # a view of the mapped file


def test_deferred_tensor_only_for_external_data(tmp_path):
    path, values = synth_model.write(str(tmp_path))
    proto = onnx_wire.load_model(path)
    by_name = {t.name: t for t in proto.graph.initializer}
    d = DeferredTensor.new(by_name["B"], str(tmp_path))
    assert d.shape == values["B"].shape and d.dtype == np.uint8 and d.size == values["B"].size
    assert np.array_equal(d.value(), values["B"])
    assert DeferredTensor.new(by_name["scales"], str(tmp_path)) is None


def test_static_initializer_rule():
    assert static_initializer((4096,), np.dtype(np.int64))
    assert not static_initializer((4097,), np.dtype(np.uint8))
    assert static_initializer((16,), np.dtype(np.float32))
    assert not static_initializer((17,), np.dtype(np.float16))
    assert not static_initializer((4,), np.dtype(np.float32), trainable=True)
    assert static_initializer((0, 5), np.dtype(np.float32))
