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
