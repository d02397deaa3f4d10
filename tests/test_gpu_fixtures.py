"""The reference's operator fixtures through the HIP operators (ops_test.exs:478-598 on this
backend): graph inputs on the device, initializers as host values, one `quantized.apply` per
node, compared with the ONNX Runtime outputs. Floats within 1e-4 + 1e-3 * max|expected|,
integers exactly; gathered rows and DequantizeLinear values bit-exactly."""

import numpy as np
import pytest

from fixtures import Fixture, max_diff, names, tolerance
from transmuter_amd import quantized

pytestmark = pytest.mark.gpu

SINGLE_NODE = (names("MatMulNBits") + names("GatherBlockQuantized") + names("DequantizeLinear")
               + ["MatMulInteger", "MatMulInteger_k4096_extremes", "MatMulInteger_k4096_signed"]
               + names("DynamicQuantizeLinear"))
BIT_EXACT = ("GatherBlockQuantized", "DequantizeLinear", "MatMulInteger", "DynamicQuantizeLinear")


def run_fixture(ctx, f: Fixture):
    node = f.node
    device_inputs = {name: ctx.put(value) for name, value in f.inputs.items()}
    inputs = [device_inputs.get(n, f.initializers.get(n)) if n else None for n in node.input]
    outs = quantized.apply(node, inputs)
    return {name: out.numpy() for name, out in zip(node.output, outs)}


@pytest.mark.parametrize("name", SINGLE_NODE)
def test_fixture(ctx, name):
    print(f"fixture {name}", flush=True)
    f = Fixture(name)
    got = run_fixture(ctx, f)
    for out_name, expected in f.outputs.items():
        actual = got[out_name]
        assert actual.shape == expected.shape, f"{name}: shape {actual.shape} vs {expected.shape}"
        assert actual.dtype == expected.dtype, f"{name}: dtype {actual.dtype} vs {expected.dtype}"
        if name.startswith(BIT_EXACT):
            assert np.array_equal(actual.reshape(-1).view(np.uint8), expected.reshape(-1).view(np.uint8)), \
                f"{name}: not bit-exact (max diff {max_diff(actual, expected)})"
        else:
            d = max_diff(actual, expected)
            assert d <= tolerance(expected), f"{name}: max difference {d}, tolerance {tolerance(expected)}"
