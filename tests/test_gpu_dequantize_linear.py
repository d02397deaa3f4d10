"""DequantizeLinear on the GPU against the oracle, bit-exactly, on seeded random inputs: each
parameter layout of expand_quant_param/3 (one value, one per axis entry, blocks along the axis),
every integer value type and float values, f32/f16/bf16 scales, with and without zero points,
shapes whose inner extent is not a multiple of the kernel's four elements per thread, 1-byte
values with per-tensor or last-axis parameters (the vectorized kernel), the 2048 x 2048 u8
tensor of the int8 benchmark, and 32 seeded random draws over all of these."""

import zlib

import numpy as np
import pytest

from oracle import oracle as o
from transmuter_amd import quantized
from transmuter_amd.onnx_wire import ATTR_INT, AttributeProto, NodeProto

pytestmark = pytest.mark.gpu

CASES = [
    # shape, axis, block_size, layout ("tensor" / "axis" / "blocked"), x type, scale type, zero point
    ((2048, 2048), 1, 0, "axis", "u8", "f32", True),
    ((3, 257, 5), 1, 0, "axis", "s8", "f16", True),
    ((4, 100, 6), 1, 16, "blocked", "u8", "bf16", True),
    ((7, 130), 0, 3, "blocked", "s8", "f32", False),
    ((1000,), 0, 0, "tensor", "s32", "f32", True),
    ((33, 65), 1, 0, "axis", "s16", "f16", True),
    ((5, 3, 9), 2, 0, "axis", "u16", "bf16", False),
    ((9, 31), 1, 0, "axis", "f32", "f32", True),
    ((6, 7), 1, 0, "tensor", "f16", "f16", True),
    ((), 0, 0, "tensor", "u8", "f32", True),
    ((2, 3, 1023), 2, 256, "blocked", "u8", "f16", True),
    # 1-byte x, per tensor or along the last axis (a multiple of 4): four elements per 4-byte load
    ((16, 64), 1, 0, "axis", "s8", "bf16", True),
    ((8, 32), 1, 0, "axis", "u8", "f16", False),
    ((4, 6, 8), 2, 0, "axis", "s8", "f32", False),
    ((1024,), 0, 0, "tensor", "s8", "f16", True),
    ((12, 20), 0, 0, "tensor", "u8", "f32", False),
    ((2, 8), 0, 0, "tensor", "u8", "bf16", True),
]

INT_RANGES = {"u8": (0, 256), "s8": (-128, 128), "u16": (0, 65536), "s16": (-32768, 32768),
              "s32": (-2**31, 2**31)}
NP = {"u8": np.uint8, "s8": np.int8, "u16": np.uint16, "s16": np.int16, "s32": np.int32, "f32": np.float32,
      "f16": np.float16}


def _values(rng, shape, dtype):
    if dtype in INT_RANGES:
        lo, hi = INT_RANGES[dtype]
        return rng.integers(lo, hi, shape, dtype=np.int64).astype(NP[dtype])
    return (rng.standard_normal(shape) * 4).astype(NP[dtype])


def _scales(rng, shape, dtype):
    s = (np.abs(rng.standard_normal(shape)) * 0.02 + 1e-3).astype(np.float32)
    if dtype == "bf16":
        return o.bf16_round(s)
    return s.astype(NP[dtype])


@pytest.mark.parametrize("case", CASES, ids=lambda c: "{}_{}_{}{}_{}".format("x".join(map(str, c[0])) or "scalar",
                                                                              c[3], c[4], "_zp" if c[6] else "", c[5]))
def test_dequantize_linear_matches_oracle(ctx, case):
    print(f"dequantize_linear {case}", flush=True)
    _check(ctx, case)


def _draw(seed):
    """A seeded random DequantizeLinear: rank 0-3, every parameter layout, integer and float
    values, every scale type, with and without zero points."""
    rng = np.random.default_rng(6000 + seed)
    rank = int(rng.integers(0, 4))
    shape = tuple(int(x) for x in rng.integers(1, 300 if rank < 3 else 40, size=rank))
    layout = str(rng.choice(["tensor", "axis", "blocked"])) if rank else "tensor"
    axis = int(rng.integers(0, rank)) if rank else 0
    bs = int(rng.integers(1, 70)) if layout == "blocked" else 0
    xdt = str(rng.choice(["u8", "u8", "s8", "s8", "u16", "s16", "s32", "f32", "f16"]))
    sdt = "f16" if xdt == "f16" else ("f32" if xdt == "f32" else str(rng.choice(["f32", "f16", "bf16"])))
    with_zero = bool(rng.random() < 0.6)
    return (shape, axis, bs, layout, xdt, sdt, with_zero)


@pytest.mark.parametrize("seed", range(32))
def test_random_dequantize_linear(ctx, seed):
    case = _draw(seed)
    print(f"random dequantize_linear seed={seed} {case}", flush=True)
    _check(ctx, case)


def _check(ctx, case):
    shape, axis, bs, layout, xdt, sdt, with_zero = case
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    x = _values(rng, shape, xdt)
    if layout == "tensor":
        pshape = ()
    elif layout == "axis":
        pshape = (shape[axis],)
    else:
        pshape = tuple(shape[:axis]) + (-(-shape[axis] // bs),) + tuple(shape[axis + 1:])
    scale = _scales(rng, pshape, sdt)
    zero = _values(rng, pshape, xdt) if with_zero else None
    attrs = [AttributeProto(name="axis", type=ATTR_INT, i=axis)]
    if bs:
        attrs.append(AttributeProto(name="block_size", type=ATTR_INT, i=bs))
    node = NodeProto(op_type="DequantizeLinear", input=["x", "s", "z" if with_zero else ""], output=["y"],
                     attribute=attrs)
    inputs = [ctx.put(x), ctx.put(scale, "bf16" if sdt == "bf16" else None)]
    if with_zero:
        inputs.append(ctx.put(zero))
    got = quantized.apply(node, inputs)[0].numpy()
    ref = o.dequantize_linear(x, scale, zero, axis=axis, block_size=bs)
    assert got.shape == ref.shape and got.dtype == ref.dtype
    assert np.array_equal(got.reshape(-1).view(np.uint8), np.ascontiguousarray(ref).reshape(-1).view(np.uint8))
