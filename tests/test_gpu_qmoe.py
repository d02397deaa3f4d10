"""QMoE on the GPU: the reference's six QMoE fixtures against their ONNX Runtime outputs, and
seeded cases against the oracle (f32: 1e-4 + 1e-3 * max|ref|; f16: 2e-2 * max|ref|, as the f16
path rounds the expert outputs, the activation and the weighted sum to f16). Shapes and seeds
are printed before each case."""

import zlib

import numpy as np
import pytest

from fixtures import Fixture, max_diff, names, tolerance
from oracle import oracle as o
from transmuter_amd import moe
from transmuter_amd.onnx_wire import ATTR_FLOAT, ATTR_INT, ATTR_STRING, AttributeProto, NodeProto

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", names("QMoE"))
def test_qmoe_fixture(ctx, name):
    print(f"fixture {name}", flush=True)
    f = Fixture(name)
    node = f.node
    values = {**f.initializers, **{n: ctx.put(v) for n, v in f.inputs.items()}}
    inputs = [values[n] if n else None for n in node.input]
    (y,) = moe.apply(node, inputs)
    got = y.numpy()
    expected = f.outputs["output"]
    assert got.shape == expected.shape and got.dtype == expected.dtype
    tol = f.atol if f.atol is not None else tolerance(expected)
    assert max_diff(got, expected) <= tol, f"{name}: max difference {max_diff(got, expected)}"


def _attr(name, value):
    if isinstance(value, str):
        return AttributeProto(name=name, type=ATTR_STRING, s=value.encode())
    if isinstance(value, float):
        return AttributeProto(name=name, type=ATTR_FLOAT, f=value)
    return AttributeProto(name=name, type=ATTR_INT, i=value)


CASES = [
    # dtype, E, k, T, H, N1, act, fusion, fc3, bits, block_size, zero points, bias, limit
    ("f32", 8, 2, 5, 64, 32, "silu", 0, False, 4, 32, False, False, 0.0),
    ("f32", 6, 3, 9, 48, 32, "gelu", 0, False, 8, 16, True, True, 0.0),
    ("f32", 4, 1, 7, 32, 16, "relu", 0, False, 4, 0, True, False, 0.0),         # per-row scales
    ("f32", 4, 2, 3, 32, 32, "swiglu", 1, False, 4, 16, False, True, 7.0),     # interleaved, limit
    ("f16", 16, 4, 40, 128, 64, "swiglu", 0, True, 4, 32, True, False, 0.0),  # gate fc1, linear fc3
    ("f16", 8, 2, 3, 64, 64, "swiglu", 2, False, 4, 0, True, True, 0.0),      # halves, per-row zp
    ("f16", 4, 2, 6, 64, 32, "identity", 0, False, 8, 16, False, True, 0.0),
    ("f16", 128, 8, 16, 512, 256, "swiglu", 0, True, 4, 32, False, False, 0.0),  # 128 experts, top-8
    ("f16", 64, 8, 70, 256, 128, "silu", 0, False, 2, 32, True, False, 0.0),      # 2-bit, rows past 32
]


def _weights(rng, e, n, k, bits, bs, zp, dtype):
    packed = rng.integers(0, 256, (e, n, k * bits // 8), dtype=np.uint8)
    npdt = np.float16 if dtype == "f16" else np.float32
    if bs > 0:
        blocks = -(-k // bs)
        scales = (np.abs(rng.standard_normal((e, n, blocks))) * 0.02 + 1e-3).astype(npdt)
        zero = rng.integers(0, 256, (e, n, -(-blocks * bits // 8)), dtype=np.uint8) if zp else None
    else:
        scales = (np.abs(rng.standard_normal((e, n))) * 0.02 + 1e-3).astype(npdt)
        zero = rng.integers(0, 256, (e, -(-n * bits // 8)), dtype=np.uint8) if zp else None
    return packed, scales, zero


@pytest.mark.parametrize("case", CASES, ids=lambda c: "{}_E{}_k{}_T{}_H{}_N{}_{}{}".format(*c[:8]))
def test_qmoe_matches_oracle(ctx, case):
    dtype, e, k, t, h, n1, act, fusion, fc3, bits, bs, zp, bias, limit = case
    print(f"qmoe {case}", flush=True)
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    npdt = np.float16 if dtype == "f16" else np.float32
    inter = n1 if (act != "swiglu" or fc3) else n1 // 2
    x = rng.standard_normal((t, h)).astype(npdt)
    router = rng.standard_normal((t, e)).astype(np.float32)
    w1, s1, z1 = _weights(rng, e, n1, h, bits, bs, zp, dtype)
    w2, s2, z2 = _weights(rng, e, h, inter, bits, bs, zp, dtype)
    w3, s3, z3 = _weights(rng, e, n1, h, bits, bs, zp, dtype) if fc3 else (None, None, None)
    b1 = (rng.standard_normal((e, n1)) * 0.1).astype(npdt) if bias else None
    b2 = (rng.standard_normal((e, h)) * 0.1).astype(npdt) if bias else None
    attrs = [_attr("k", k), _attr("expert_weight_bits", bits), _attr("block_size", bs), _attr("activation_type", act),
             _attr("swiglu_fusion", fusion), _attr("swiglu_limit", limit)]
    node = NodeProto(op_type="QMoE", input=[], output=["y"], attribute=attrs)
    inputs = [ctx.put(x), ctx.put(router), w1, s1, b1, w2, s2, b2, w3, s3, None, z1, z2, z3]
    (y,) = moe.apply(node, inputs)
    got = y.numpy().astype(np.float64)
    ref = o.qmoe(x.astype(np.float32), router, w1, s1, w2, s2, k=k, bits=bits, block_size=bs, activation=act,
                 swiglu_fusion=fusion, limit=limit, fc1_bias=b1, fc2_bias=b2, fc3=w3, fc3_scales=s3,
                 fc1_zp=z1, fc2_zp=z2, fc3_zp=z3).astype(np.float64)
    scale = np.abs(ref).max()
    tol = 2e-2 * scale if dtype == "f16" else 1e-4 + 1e-3 * scale
    assert np.abs(got - ref).max() <= tol, f"max difference {np.abs(got - ref).max()} (max |ref| {scale})"
