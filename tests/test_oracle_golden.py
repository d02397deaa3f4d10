"""The oracle against the reference's own operator fixtures (ONNX Runtime outputs).

The fixtures are the reference's test/fixtures/ops/<case> directories (written by its
test/support/make_op_fixtures.py); the comparison rule is its ops_test.exs:569-598: floats
within 1e-4 + 1e-3 * max|expected| (or the fixture's atol), integers exactly. The oracle is
held to more where it must be: gathered rows and DequantizeLinear values bit-exactly.
"""

import numpy as np
import pytest

from fixtures import Fixture, attrs, max_diff, names, tolerance
from oracle import oracle as o


def run_oracle(f: Fixture, node=None, values=None):
    node = node or f.node
    a = attrs(node)
    values = values if values is not None else f.values()
    ins = [values[n] if n else None for n in node.input]
    op = node.op_type
    if op == "MatMulNBits":
        A, B, S, Z, G, bias = (ins + [None] * 6)[:6]
        return [o.matmul_nbits(A, B, S, Z, bias, k=a["K"], n=a["N"], bits=a.get("bits", 4),
                               block_size=a["block_size"], g_idx=G)]
    if op == "GatherBlockQuantized":
        data, idx, s, zp = (ins + [None] * 4)[:4]
        return [o.gather_block_quantized(data, idx, s, zp, bits=a.get("bits", 4),
                                         gather_axis=a.get("gather_axis", 0),
                                         quantize_axis=a.get("quantize_axis", 1))]
    if op == "DequantizeLinear":
        x, s, z = (ins + [None] * 3)[:3]
        return [o.dequantize_linear(x, s, z, axis=a.get("axis", 1), block_size=a.get("block_size", 0))]
    if op == "MatMulInteger":
        A, B, az, bz = (ins + [None] * 4)[:4]
        return [o.matmul_integer(A, B, az, bz)]
    if op == "DynamicQuantizeLinear":
        return list(o.dynamic_quantize_linear(ins[0]))
    if op == "QMoE":
        (x, r, fc1, fc1s, fc1b, fc2, fc2s, fc2b, fc3, fc3s, fc3b, z1, z2, z3) = (ins + [None] * 14)[:14]
        return [o.qmoe(x, r, fc1, fc1s, fc2, fc2s, k=a["k"], bits=a.get("expert_weight_bits", 4),
                       block_size=a.get("block_size", 0), activation=a.get("activation_type", "relu"),
                       swiglu_fusion=a.get("swiglu_fusion", 0), alpha=a.get("activation_alpha", 1.0),
                       beta=a.get("activation_beta", 0.0), limit=a.get("swiglu_limit", 0.0),
                       fc1_bias=fc1b, fc2_bias=fc2b, fc3=fc3, fc3_scales=fc3s, fc3_bias=fc3b,
                       fc1_zp=z1, fc2_zp=z2, fc3_zp=z3)]
    if op == "Cast":
        return [ins[0].astype(np.float32)]
    if op == "Mul":
        return [(np.asarray(ins[0], np.float32) * np.asarray(ins[1], np.float32)).astype(np.float32)]
    raise NotImplementedError(op)


def run_graph(f: Fixture):
    values = f.values()
    for node in f.nodes:
        outs = run_oracle(f, node, values)
        for name, v in zip(node.output, outs):
            values[name] = v
    return {name: values[name] for name in f.outputs}


def assert_same(name, actual, expected, atol=None, exact=False):
    actual = np.asarray(actual)
    assert actual.shape == expected.shape, f"{name}: shape {actual.shape}, expected {expected.shape}"
    if exact or (atol is None and expected.dtype.kind in "iu"):
        assert actual.dtype == expected.dtype, f"{name}: dtype {actual.dtype}, expected {expected.dtype}"
        assert np.array_equal(np.ascontiguousarray(actual).reshape(-1).view(np.uint8),
                              np.ascontiguousarray(expected).reshape(-1).view(np.uint8)), f"{name}: not bit-exact"
        return
    d = max_diff(actual, expected)
    tol = atol if atol is not None else tolerance(expected)
    assert d <= tol, f"{name}: max difference {d}, tolerance {tol}"


@pytest.mark.parametrize("name", names("MatMulNBits"))
def test_matmul_nbits_fixture(name):
    f = Fixture(name)
    (y,) = run_oracle(f)
    assert_same(name, y, f.outputs["Y"])


@pytest.mark.parametrize("name", names("GatherBlockQuantized"))
def test_gather_block_quantized_fixture_bit_exact(name):
    f = Fixture(name)
    (y,) = run_oracle(f)
    assert_same(name, y, f.outputs["Y"], exact=True)


@pytest.mark.parametrize("name", names("DequantizeLinear"))
def test_dequantize_linear_fixture_bit_exact(name):
    f = Fixture(name)
    (y,) = run_oracle(f)
    assert_same(name, y, f.outputs["y"], exact=True)


@pytest.mark.parametrize("name", names("MatMulInteger"))
def test_matmul_integer_fixture_exact(name):
    f = Fixture(name)
    got = run_graph(f)
    for out_name, expected in f.outputs.items():
        assert_same(name, got[out_name], expected, atol=f.atol)


@pytest.mark.parametrize("name", names("DynamicQuantizeLinear"))
def test_dynamic_quantize_linear_fixture_exact(name):
    f = Fixture(name)
    got = run_graph(f)
    for out_name, expected in f.outputs.items():
        assert_same(f"{name} {out_name}", np.asarray(got[out_name]).astype(expected.dtype).reshape(expected.shape),
                    expected, exact=True)


@pytest.mark.parametrize("name", names("QMoE"))
def test_qmoe_fixture(name):
    f = Fixture(name)
    (y,) = run_oracle(f)
    assert_same(name, y, f.outputs["output"], atol=f.atol)


def test_k4096_sums_pass_two_to_the_24():
    """The two k4096 fixtures hold sums beyond 2^24, where an f32 sum stops being exact."""
    for name in ("MatMulInteger_k4096_extremes", "MatMulInteger_k4096_signed"):
        f = Fixture(name)
        assert np.abs(f.outputs["y"].astype(np.int64)).max() > 2 ** 24
