"""QMoE on the GPU: the reference's six QMoE fixtures against their ONNX Runtime outputs, and
seeded cases against the oracle (f32: 1e-4 + 1e-3 * max|ref|; f16: 1e-2 * max|ref| against the
oracle's f16 mode, which rounds the dequantized weights, expert products, activation steps and
weighted outputs to f16 as the reference's Nx ops do). Shapes and seeds are printed before each
case."""

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
    ("f16", 200, 8, 24, 64, 32, "silu", 0, False, 4, 32, False, False, 0.0),       # 4 router keys per lane
    ("f32", 600, 16, 8, 32, 16, "relu", 0, False, 4, 32, False, True, 0.0),        # 16 per lane, top-16
    ("f16", 16, 8, 600, 64, 32, "silu", 0, False, 4, 32, False, False, 0.0),       # 4800 rows: plan reloads ids
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
    print(f"qmoe {case}", flush=True)
    _check_qmoe(ctx, case)


def _draw_qmoe(seed):
    """A seeded random QMoE layer: f32 or f16, 1-64 experts, top-1..8, up to 80 tokens (experts
    with no rows among them), 2/4/8-bit weights, per-row or block-wise (16-128) parameters, with
    and without zero points and biases, every activation and swiglu layout."""
    rng = np.random.default_rng(5000 + seed)
    dtype = str(rng.choice(["f32", "f16"]))
    e = int(rng.integers(1, 65))
    k = int(rng.integers(1, min(8, e) + 1))
    t = int(rng.integers(1, 81))
    h = 16 * int(rng.integers(1, 17))
    act = str(rng.choice(["relu", "gelu", "silu", "identity", "swiglu", "swiglu"]))
    fusion, fc3, limit = 0, False, 0.0
    if act == "swiglu":
        fusion, fc3 = [(0, True), (1, False), (2, False)][int(rng.integers(0, 3))]
        limit = float(rng.choice([0.0, 7.0]))
    n1 = (32 if act == "swiglu" and not fc3 else 16) * int(rng.integers(1, 9))
    bits = int(rng.choice([2, 4, 4, 8]))
    bs = int(rng.choice([0, 16, 32, 64, 128]))
    return (dtype, e, k, t, h, n1, act, fusion, fc3, bits, bs, bool(rng.random() < 0.5), bool(rng.random() < 0.3),
            limit)


@pytest.mark.parametrize("seed", range(24))
def test_random_qmoe(ctx, seed):
    case = _draw_qmoe(seed)
    print(f"random qmoe seed={seed} {case}", flush=True)
    _check_qmoe(ctx, case)


def _check_qmoe(ctx, case):
    dtype, e, k, t, h, n1, act, fusion, fc3, bits, bs, zp, bias, limit = case
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
    ref = o.qmoe(x, router, w1, s1, w2, s2, k=k, bits=bits, block_size=bs, activation=act,
                 swiglu_fusion=fusion, limit=limit, fc1_bias=b1, fc2_bias=b2, fc3=w3, fc3_scales=s3,
                 fc1_zp=z1, fc2_zp=z2, fc3_zp=z3).astype(np.float64)
    scale = np.abs(ref).max()
    tol = 1e-2 * scale if dtype == "f16" else 1e-4 + 1e-3 * scale
    assert np.abs(got - ref).max() <= tol, f"max difference {np.abs(got - ref).max()} (max |ref| {scale})"


# Several groups of eight output tiles per workgroup, one after the other in one chunk pipeline
# (TMH_MOE_GPW; by default the stored products of 16 groups or more run four): groups that do not
# divide evenly, a last group with idle wavefronts (tiles per expert not a multiple of 8), every
# epilogue (swiglu of fc1 and fc3, an activation, the stored fc2).
GPW_CASES = [
    ("f16", 16, 4, 40, 176, 64, "swiglu", 0, True, 4, 32, True, False, 0.0),
    ("f16", 8, 2, 70, 400, 208, "gelu", 0, False, 4, 32, False, True, 0.0),
    ("f16", 12, 3, 33, 272, 96, "silu", 0, False, 8, 64, True, False, 0.0),
]


@pytest.mark.parametrize("gpw", [2, 3])
@pytest.mark.parametrize("case", GPW_CASES, ids=lambda c: "{}_E{}_k{}_T{}_H{}_N{}_{}".format(*c[:7]))
def test_qmoe_several_tile_groups_per_workgroup(ctx, monkeypatch, case, gpw):
    monkeypatch.setenv("TMH_MOE_GPW", str(gpw))
    print(f"qmoe {gpw} tile groups per workgroup {case}", flush=True)
    _check_qmoe(ctx, case)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_qmoe_routing_ties(ctx, dtype):
    """Tied router values, +0 and -0 among them: the lower expert index wins the tie
    (MoE.topk/2, moe.ex:157-165). Experts differ strongly, so a different choice shows in y."""
    print(f"qmoe routing ties {dtype}", flush=True)
    rng = np.random.default_rng(8)
    npdt = np.float16 if dtype == "f16" else np.float32
    e, k, h, n1 = 4, 2, 32, 16
    router = np.array([[0.5, 0.5, 0.5, 0.1], [0.0, -0.0, 0.0, -1.0], [-0.0, 0.0, 1.0, 1.0],
                       [2.0, 3.0, 3.0, 2.0], [0.0, 0.0, 0.0, 0.0], [-0.0, -0.0, -0.0, -0.0]], np.float32)
    t = router.shape[0]
    w1, s1, _ = _weights(rng, e, n1, h, 4, 32, False, dtype)
    w2, s2, _ = _weights(rng, e, h, n1, 4, 32, False, dtype)
    s2 = (s2 * np.arange(1, e + 1, dtype=np.float32)[:, None, None]).astype(npdt)  # expert e scaled by e+1
    x = rng.standard_normal((t, h)).astype(npdt)
    node = NodeProto(op_type="QMoE", input=[], output=["y"],
                     attribute=[_attr("k", k), _attr("block_size", 32), _attr("activation_type", "silu")])
    (y,) = moe.apply(node, [ctx.put(x), ctx.put(router), w1, s1, None, w2, s2, None])
    got = y.numpy().astype(np.float64)
    ref = o.qmoe(x, router, w1, s1, w2, s2, k=k, bits=4, block_size=32, activation="silu").astype(np.float64)
    _vals, idx = o.topk_stable(router, k)
    assert idx.tolist() == [[0, 1], [0, 1], [2, 3], [1, 2], [0, 1], [0, 1]]
    scale = np.abs(ref).max()
    tol = 1e-2 * scale if dtype == "f16" else 1e-4 + 1e-3 * scale
    assert np.abs(got - ref).max() <= tol, f"max difference {np.abs(got - ref).max()} (max |ref| {scale})"


@pytest.mark.parametrize("e", [200, 1000])
def test_qmoe_routing_ties_among_many_experts(ctx, e):
    """Ties across the 64-expert groups that routing holds per lane: equal values at experts far
    apart, +0 beside -0 over every expert, and a maximum held by the last expert only."""
    print(f"qmoe routing ties E={e}", flush=True)
    rng = np.random.default_rng(9)
    k, h, n1 = 3, 32, 16
    router = np.full((4, e), -1.0, np.float32)
    router[0, [e - 1, 130, 65, 64]] = 2.0                       # four-way tie: 64, 65, 130
    router[1, :] = -0.0
    router[1, ::7] = 0.0                                        # all equal: 0, 1, 2
    router[2, e - 1] = 5.0
    router[2, [3, e // 2]] = 4.0                                # e-1, then 3 before e/2
    router[3, :] = np.linspace(-1.0, 1.0, e, dtype=np.float32)  # the three last experts, largest first
    t = router.shape[0]
    w1, s1, _ = _weights(rng, e, n1, h, 4, 32, False, "f16")
    w2, s2, _ = _weights(rng, e, h, n1, 4, 32, False, "f16")
    x = rng.standard_normal((t, h)).astype(np.float16)
    node = NodeProto(op_type="QMoE", input=[], output=["y"],
                     attribute=[_attr("k", k), _attr("block_size", 32), _attr("activation_type", "silu")])
    (y,) = moe.apply(node, [ctx.put(x), ctx.put(router), w1, s1, None, w2, s2, None])
    got = y.numpy().astype(np.float64)
    ref = o.qmoe(x, router, w1, s1, w2, s2, k=k, bits=4, block_size=32, activation="silu").astype(np.float64)
    _vals, idx = o.topk_stable(router, k)
    assert idx.tolist() == [[64, 65, 130], [0, 1, 2], [e - 1, 3, e // 2], [e - 1, e - 2, e - 3]]
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 1e-2 * scale, f"max difference {np.abs(got - ref).max()} (max |ref| {scale})"


def test_qmoe_fc3_without_zero_points_beside_fc1_with_them(ctx):
    """fc1 with packed zero points and fc3 without (each QMoE input has its own, moe.ex:45): the
    swiglu product must read each weight with its own layout."""
    print("qmoe fc1 zp, fc3 none", flush=True)
    rng = np.random.default_rng(9)
    e, k, t, h, n1 = 8, 2, 20, 64, 32
    w1, s1, z1 = _weights(rng, e, n1, h, 4, 32, True, "f16")
    w3, s3, _ = _weights(rng, e, n1, h, 4, 32, False, "f16")
    w2, s2, z2 = _weights(rng, e, h, n1, 4, 32, True, "f16")
    x = rng.standard_normal((t, h)).astype(np.float16)
    router = rng.standard_normal((t, e)).astype(np.float32)
    node = NodeProto(op_type="QMoE", input=[], output=["y"],
                     attribute=[_attr("k", k), _attr("block_size", 32), _attr("activation_type", "swiglu"),
                                _attr("swiglu_fusion", 0)])
    inputs = [ctx.put(x), ctx.put(router), w1, s1, None, w2, s2, None, w3, s3, None, z1, z2, None]
    (y,) = moe.apply(node, inputs)
    got = y.numpy().astype(np.float64)
    ref = o.qmoe(x, router, w1, s1, w2, s2, k=k, bits=4, block_size=32, activation="swiglu", fc3=w3, fc3_scales=s3,
                 fc1_zp=z1, fc2_zp=z2).astype(np.float64)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 1e-2 * scale, f"max difference {np.abs(got - ref).max()} (max |ref| {scale})"


@pytest.mark.parametrize("n1,h", [(24, 32), (32, 24)], ids=["fc1_rows_24", "hidden_24"])
def test_qmoe_rejects_expert_rows_off_the_16_row_tiles(ctx, n1, h):
    """Weights packed by tmh_weight_upload_nbits may hold any E*N rows; tmh_qmoe needs whole
    16-row tiles per expert (fc1 and fc3 rows, and H for fc2) and says so instead of mixing
    experts' rows."""
    from synth import nbits_weight
    from transmuter_amd import PackedWeight
    from transmuter_amd._lib import ERR_UNSUPPORTED, F16, F32, lib

    print(f"qmoe rows per expert n1={n1} h={h}", flush=True)
    rng = np.random.default_rng(10)
    e, t = 4, 3
    fc1 = PackedWeight.upload(ctx, *nbits_weight(rng, h, e * n1, 4, 16), k=h, n=e * n1, bits=4, block_size=16,
                              weight_dtype="f16")
    fc2 = PackedWeight.upload(ctx, *nbits_weight(rng, n1, e * h, 4, 16), k=n1, n=e * h, bits=4, block_size=16,
                              weight_dtype="f16")
    x = ctx.put(rng.standard_normal((t, h)).astype(np.float16))
    router = ctx.put(rng.standard_normal((t, e)).astype(np.float32))
    y = ctx.empty((t, h), "f16")
    status = lib().tmh_qmoe(ctx.handle, x.ptr, F16, t, h, router.ptr, F32, e, 2, fc1.handle, None, fc2.handle, None,
                            None, None, F16, 2, 0, 1.0, 0.0, 0.0, y.ptr, None)
    message = lib().tmh_last_error(ctx.handle).decode()
    assert status == ERR_UNSUPPORTED and "multiples of 16" in message, message
    fc1.free()
    fc2.free()
