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


def _nibbles(values) -> bytes:
    """Two 4-bit values per byte, the lower element in the low nibble."""
    v = [x & 15 for x in values]
    v += [0] * (len(v) % 2)
    return bytes(v[i] | (v[i + 1] << 4) for i in range(0, len(v), 2))


def test_int4_and_uint4_initializers_stay_packed(tmp_path):
    """ONNX UINT4 (21) and INT4 (22) initializers load packed two values per byte, the last axis
    halved (rounded up), as u8 and s8 (Ops.tensor_data/2 and tensor_shape_type/1,
    lib/transmuter/ops.ex:610-639). The unpacked nibbles give back the values, sign extended
    for int4."""
    import onnx_writer as w
    from oracle import oracle as o

    rng = np.random.default_rng(21)
    u4 = rng.integers(0, 16, (3, 8))
    s4 = rng.integers(-8, 8, (2, 6))
    odd = rng.integers(0, 16, (1, 5))  # one row of an odd length: ceil(5/2) = 3 bytes
    inits = [w.tensor_raw("u4", [3, 8], 21, _nibbles(u4.ravel())),
             w.tensor_raw("s4", [2, 6], 22, _nibbles(s4.ravel())),
             w.tensor_raw("odd", [1, 5], 21, _nibbles(odd.ravel()))]
    path = tmp_path / "int4.onnx"
    path.write_bytes(w.model([], inits, [], ["u4"]))
    proto = onnx_wire.load_model(str(path))
    by_name = {t.name: t for t in proto.graph.initializer}
    got = {name: onnx_wire.tensor(t) for name, t in by_name.items()}
    assert got["u4"].dtype == np.uint8 and got["u4"].shape == (3, 4)
    assert got["s4"].dtype == np.int8 and got["s4"].shape == (2, 3)
    assert got["odd"].dtype == np.uint8 and got["odd"].shape == (1, 3)
    for name, t in by_name.items():
        assert onnx_wire.shape_type(t) == (got[name].shape, got[name].dtype), name
    assert np.array_equal(o.unpack(got["u4"], 4), u4)
    assert np.array_equal(o.unpack_signed(got["s4"], 4), s4)
    assert np.array_equal(o.unpack(got["odd"], 4)[:, :5], odd)
    model = load(str(path))  # small integer tensors are static values
    assert np.array_equal(model.static["u4"], got["u4"]) and model.static["s4"].dtype == np.int8


def test_bf16_initializers_keep_their_type_through_upcast(tmp_path):
    """bf16 initializers load as BF16Host bit patterns (typed "bf16"), and Transmuter.upcast/2
    (lib/transmuter.ex:1323-1324) casts f16/bf16 values to the compute type with one rounding."""
    import onnx_writer as w
    from transmuter_amd.device import BF16Host, nx_type
    from transmuter_amd.hip import upcast

    bits = np.array([0x3F80, 0x4049, 0xC2F7, 0x3EAB, 0x0001], np.uint16)  # 1, 3.140625, -123.5, 0.333984375, denormal
    path = tmp_path / "bf16.onnx"
    path.write_bytes(w.model([], [w.tensor_raw("s", [5], 16, bits.tobytes())], [], ["s"]))
    t = onnx_wire.load_model(str(path)).graph.initializer[0]
    value = onnx_wire.tensor(t)
    assert isinstance(value, BF16Host) and nx_type(value) == "bf16" and nx_type(onnx_wire.tensor_view(t)) == "bf16"
    f32 = np.array([1.0, 3.140625, -123.5, 0.333984375, 2.0 ** -133], np.float32)
    up, dtype = upcast(value, "f32")
    assert dtype == "f32" and np.array_equal(up, f32)
    up16, dtype16 = upcast(value, "f16")
    assert dtype16 == "f16" and np.array_equal(up16, f32.astype(np.float16))
    same, dtype_same = upcast(value, "bf16")
    assert dtype_same == "bf16" and np.array_equal(np.asarray(same), bits)
    back, dtype_back = upcast(np.array([1.0, 1.0 / 3.0, 65504.0], np.float16), "bf16")
    assert dtype_back == "bf16" and isinstance(back, BF16Host)
    assert np.asarray(back).tolist() == [0x3F80, 0x3EAB, 0x4780]  # RNE of 0.33325195 and 65504
    model = load(str(path), compute_type="f32")
    assert model.static["s"].dtype == np.float32 and np.array_equal(model.static["s"], f32)
