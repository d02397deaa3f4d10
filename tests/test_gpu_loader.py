"""The loader with the HIP backend: the external MatMulNBits weight is packed from its memory
map, other params go to the device (the external ones straight from the file), and the moved
model runs MatMulNBits as the oracle does; file uploads through the staging buffers are
byte-exact across chunk boundaries."""

import numpy as np
import pytest

import synth_model
from oracle import oracle as o
from transmuter_amd import DeviceTensor, PackedWeight
from transmuter_amd.hip import run_nodes
from transmuter_amd.loader import load

pytestmark = pytest.mark.gpu


def test_loaded_model_runs_on_the_device(ctx, tmp_path):
    path, values = synth_model.write(str(tmp_path))
    print(f"load {path}", flush=True)
    model = load(path, ctx)
    assert model.nodes[0].input == ["A", "B:packed", "", ""]
    assert isinstance(model.params["B:packed"], PackedWeight)
    assert isinstance(model.params["extra"], DeviceTensor)
    assert np.array_equal(model.params["extra"].numpy(), values["extra"])
    a = np.random.default_rng(1).standard_normal((3, synth_model.K)).astype(np.float16)
    y = run_nodes(model, {"A": ctx.put(a)})["Y"].numpy()
    ref = o.matmul_nbits(a, values["B"], values["scales"].astype(np.float32), values["zp"], k=synth_model.K,
                         n=synth_model.N, bits=synth_model.BITS, block_size=synth_model.BS, weight_dtype="f16")
    assert np.abs(y.astype(np.float64) - ref).max() <= 1e-2 * np.abs(ref).max()


def test_put_file_is_byte_exact_across_chunks(ctx, tmp_path):
    rng = np.random.default_rng(2)
    data = rng.integers(0, 256, 40 << 20, dtype=np.uint8)  # 40 MiB: three 16 MiB chunks
    f = tmp_path / "blob.bin"
    data.tofile(f)
    offset, n = 12345, (40 << 20) - 12345 - 7
    t = ctx.put_file(str(f), offset, (n,), "u8")
    assert np.array_equal(t.numpy(), data[offset:offset + n])


def test_put_file_rejects_ranges_past_the_end(ctx, tmp_path):
    from transmuter_amd._lib import TmhError

    f = tmp_path / "small.bin"
    f.write_bytes(b"x" * 100)
    with pytest.raises(TmhError, match="holds no"):
        ctx.put_file(str(f), 50, (60,), "u8")


def _nibbles(values) -> bytes:
    """Two 4-bit values per byte, the lower element in the low nibble (ONNX INT4 / UINT4)."""
    v = [int(x) & 15 for x in np.asarray(values).ravel()]
    v += [0] * (len(v) % 2)
    return bytes(v[i] | (v[i + 1] << 4) for i in range(0, len(v), 2))


@pytest.mark.parametrize("signed", [False, True], ids=["uint4", "int4"])
def test_int4_initializers_gather_on_the_device(ctx, tmp_path, signed):
    """A GatherBlockQuantized whose table (and zero points) are ONNX UINT4 / INT4 initializers
    (types 21 / 22): the loader keeps them packed as u8 / s8, the table goes to the device, and
    the HIP gather sign-extends int4 values as the reference's unpack does (Ops.tensor/2 int4
    branch, lib/transmuter/ops.ex:632-639; Quantized.unpack/2, quantized.ex:294-300), bit-exactly
    against the oracle."""
    import onnx_writer as wr
    from transmuter_amd.hip import Model, run_nodes

    rng = np.random.default_rng(4 + signed)
    rows, cols, bs = 512, 256, 32
    blocks = cols // bs
    q = rng.integers(-8, 8, (rows, cols)) if signed else rng.integers(0, 16, (rows, cols))
    scales = (np.abs(rng.standard_normal((rows, blocks))) * 0.01 + 1e-4).astype(np.float16)
    inits = [wr.tensor_raw("table", [rows, cols], 22 if signed else 21, _nibbles(q)), wr.tensor("scales", scales)]
    inputs = ["table", "ids", "scales"]
    zq = None
    if not signed:  # UINT4 zero points, one per block, packed like the table
        zq = rng.integers(0, 16, (rows, blocks))
        inits.append(wr.tensor_raw("zp", [rows, blocks], 21, _nibbles(zq)))
        inputs.append("zp")
    attrs = [wr.attribute_int("bits", 4), wr.attribute_int("block_size", bs), wr.attribute_int("gather_axis", 0),
             wr.attribute_int("quantize_axis", 1)]
    node = wr.node("GatherBlockQuantized", inputs, ["out"], attrs, domain="com.microsoft")
    path = tmp_path / "int4_gather.onnx"
    path.write_bytes(wr.model([node], inits, ["ids"], ["out"]))
    print(f"int4 gather signed={signed} {path}", flush=True)
    model = load(str(path), ctx)
    table = model.params["table"]
    assert isinstance(table, DeviceTensor) and table.dtype == ("s8" if signed else "u8")
    assert table.shape == (rows, cols // 2)
    ids = rng.integers(-rows, rows, (3, 7)).astype(np.int64)
    got = run_nodes(model, {"ids": ctx.put(ids)})["out"].numpy()
    host_table = table.numpy()
    zp_val = model.static.get("zp", model.params.get("zp"))
    zp = zp_val.numpy() if isinstance(zp_val, DeviceTensor) else zp_val
    ref = o.gather_block_quantized(host_table, np.where(ids < 0, ids + rows, ids), scales, zp, bits=4)
    assert got.shape == (3, 7, cols) and got.dtype == np.float16
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    # The values are the integers written to the file.
    want_q = q[np.where(ids < 0, ids + rows, ids)].astype(np.float32)
    want_z = 0.0 if zq is None else np.repeat(zq[np.where(ids < 0, ids + rows, ids)], bs, axis=-1)
    want = ((want_q - want_z) * np.repeat(scales[np.where(ids < 0, ids + rows, ids)].astype(np.float32), bs, axis=-1))
    assert np.array_equal(got, want.astype(np.float16))
