"""GatherBlockQuantized on the GPU against the oracle, bit-exactly, over the kernel's variants:
4-byte and 1-byte row units, one or several quantization blocks per thread, vector or scalar
stores; u8 and s8 data; no, packed (u8 / s8) and float zero points; f32, f16 and bf16 scales;
negative ids (counted from the end); s64 and s32 ids; and the multi-slice kernel of rows of whole
256-byte slices (4- and 8-bit data, no or packed zero points, slice counts that leave the last
wavefront partly empty), with 32 seeded random draws over all of these. Seeds and shapes are
printed before each case."""

import zlib

import numpy as np
import pytest

from oracle import oracle as o
from transmuter_amd import quantized
from transmuter_amd.onnx_wire import ATTR_INT, AttributeProto, NodeProto

pytestmark = pytest.mark.gpu

CASES = [
    # bits, rows, row_bytes, blocks, data type, zero points, scale type, ids shape
    (4, 300, 512, 32, "u8", "u8", "f16", (8, 64)),     # bs 32: one block per thread, 16-byte stores
    (4, 50, 12, 6, "u8", None, "f32", (37,)),          # bs 4: two blocks per thread
    (4, 40, 10, 5, "u8", "u8", "bf16", (3, 5)),        # odd row bytes: 1-byte units
    (4, 64, 64, 8, "s8", None, "f16", (20,)),          # signed nibbles, zero point 0
    (4, 64, 64, 8, "s8", "s8", "bf16", (20,)),         # signed packed zero points
    (8, 100, 256, 8, "s8", "float", "f32", (2, 33)),   # float zero points, 16-byte f32 stores
    (8, 30, 12, 3, "u8", "u8", "f16", (11,)),          # rows of 24 bytes out: scalar stores
    (2, 64, 64, 16, "u8", "u8", "f16", (9, 7)),        # q2, bs 16: 32-byte stores
    (2, 16, 4, 1, "u8", None, "f32", (5,)),
    # rows of whole 256-byte slices: several slices per wavefront
    (8, 200, 256, 8, "u8", "u8", "bf16", (13,), np.int32),   # q8, 13 slices: a partial last wavefront
    (4, 100, 768, 48, "s8", "s8", "f32", (7, 3), np.int32),  # 3 slices per row, signed data and zero points
    (8, 64, 512, 16, "s8", None, "f16", (5,)),               # q8 signed, no zero points
    (4, 500, 256, 16, "u8", None, "bf16", (1,)),             # one id, one slice
    # the same kernel's packed-f16 arithmetic: every signedness of data and zero points
    (4, 100, 512, 32, "s8", "s8", "f16", (9, 3), np.int32),  # signed nibbles and zero points
    (4, 100, 256, 16, "s8", None, "f16", (7,)),              # signed nibbles, zero point 0
    (4, 100, 256, 8, "u8", "s8", "f16", (5,)),               # unsigned nibbles, signed zero points
    (8, 100, 512, 16, "u8", "u8", "f16", (6,)),              # q8 with zero points
    (8, 100, 256, 4, "s8", "u8", "f16", (5,)),               # signed bytes, unsigned zero points
    (8, 100, 256, 8, "u8", None, "f16", (3, 3)),             # q8, default zero point 128
]


def _scales(rng, shape, dtype):
    s = (np.abs(rng.standard_normal(shape)) * 0.05 + 1e-3).astype(np.float32)
    return o.bf16_round(s) if dtype == "bf16" else s.astype(np.float16 if dtype == "f16" else np.float32)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "b{}_r{}_B{}_blk{}_{}_{}_{}".format(*c[:7]) +
                         ("_ids32" if len(c) > 8 else ""))
def test_gather_matches_oracle(ctx, case):
    print(f"gather {case}", flush=True)
    _check_gather(ctx, case)


def _check_gather(ctx, case):
    bits, rows, row_bytes, blocks, dtype, zp, sdt, ids_shape = case[:8]
    ids_dtype = case[8] if len(case) > 8 else np.int64
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    data = rng.integers(0, 256, (rows, row_bytes), dtype=np.uint8)
    if dtype == "s8":
        data = data.view(np.int8)
    scales = _scales(rng, (rows, blocks), sdt)
    zrow = -(-blocks * bits // 8)
    if zp is None:
        zero = None
    elif zp == "float":
        zero = rng.integers(-3, 4, (rows, blocks)).astype(np.float32)
    else:
        zero = rng.integers(0, 256, (rows, zrow), dtype=np.uint8)
        zero = zero.view(np.int8) if zp == "s8" else zero
    ids = rng.integers(-rows, rows, ids_shape, dtype=np.int64).astype(ids_dtype)
    node = NodeProto(op_type="GatherBlockQuantized", input=["data", "ids", "scales"] + (["zp"] if zp else []),
                     output=["out"], attribute=[AttributeProto(name="bits", type=ATTR_INT, i=bits)])
    sc_in = ctx.put(scales, sdt) if sdt == "bf16" else ctx.put(scales)
    args = [ctx.put(data), ctx.put(ids), sc_in] + ([ctx.put(zero)] if zp else [])
    got = quantized.apply(node, args)[0].numpy()
    ref = o.gather_block_quantized(data, ids, scales, zero, bits=bits)  # bf16 as uint16 bits
    assert got.shape == ids_shape + (row_bytes * 8 // bits,)
    assert np.array_equal(np.ascontiguousarray(got).view(np.uint8), np.ascontiguousarray(ref).view(np.uint8))


@pytest.mark.parametrize("zp", [False, True], ids=["no_zp", "packed_zp"])
def test_gather_vocab_table(ctx, zp):
    """The tied-embedding lookup at its benchmark shape: a 151936 x 1024 q4 table, block 32, f16
    scales, ids [8, 512] uniform over the whole table (its first and last rows included), with
    and without packed zero points."""
    print(f"gather vocab 151936x1024 ids [8,512] zp={zp}", flush=True)
    rng = np.random.default_rng(5)
    rows, d, bs = 151936, 1024, 32
    data = rng.integers(0, 256, (rows, d // 2), dtype=np.uint8)
    scales = _scales(rng, (rows, d // bs), "f16")
    zero = rng.integers(0, 256, (rows, d // bs // 2), dtype=np.uint8) if zp else None
    ids = np.concatenate([[0, rows - 1, -1], rng.integers(0, rows, 8 * 512 - 3)]).astype(np.int64).reshape(8, 512)
    node = NodeProto(op_type="GatherBlockQuantized", input=["data", "ids", "scales"] + (["zp"] if zp else []),
                     output=["out"], attribute=[AttributeProto(name="bits", type=ATTR_INT, i=4)])
    args = [ctx.put(data), ctx.put(ids), ctx.put(scales)] + ([ctx.put(zero)] if zp else [])
    got = quantized.apply(node, args)[0].numpy()
    ref = o.gather_block_quantized(data, ids, scales, zero, bits=4)
    assert got.shape == (8, 512, d)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_f16_extreme_scales(ctx, bits):
    """f16 scales at the edges of the format (zero, both signs, subnormals, the largest finite
    value, whose products overflow to infinity) through the multi-slice kernel's packed-f16
    arithmetic: the one rounding of (q - zero) * scale matches the oracle's bit for bit."""
    print(f"gather f16 extreme scales bits={bits}", flush=True)
    rng = np.random.default_rng(31 + bits)
    rows, row_bytes = 64, 512
    d = row_bytes * 8 // bits
    blocks = d // 32
    special = np.array([0.0, -0.0, 6e-8, -6e-8, 3e-5, 6.1e-5, 1.0, -0.5, 65504.0, -65504.0, 0.33325, 1e-3],
                       np.float16)
    scales = rng.choice(special, (rows, blocks)).astype(np.float16)
    data = rng.integers(0, 256, (rows, row_bytes), dtype=np.uint8)
    zero = rng.integers(0, 256, (rows, -(-blocks * bits // 8)), dtype=np.uint8)
    ids = rng.integers(0, rows, (40,), dtype=np.int64)
    node = NodeProto(op_type="GatherBlockQuantized", input=["data", "ids", "scales", "zp"], output=["out"],
                     attribute=[AttributeProto(name="bits", type=ATTR_INT, i=bits)])
    got = quantized.apply(node, [ctx.put(data), ctx.put(ids), ctx.put(scales), ctx.put(zero)])[0].numpy()
    ref = o.gather_block_quantized(data, ids, scales, zero, bits=bits)
    bits16 = ref.view(np.uint16)
    assert np.isinf(ref.astype(np.float32)).any() and (((bits16 & 0x7C00) == 0) & ((bits16 & 0x3FF) != 0)).any()
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def _draw_gather(seed):
    """A seeded random gather: 2-, 4- or 8-bit rows, half of them whole 256-byte slices (the
    multi-slice kernel), power-of-two blocks of at least 16 values, every zero-point kind and
    scale type, s32 or s64 ids with negatives."""
    rng = np.random.default_rng(7000 + seed)
    bits = int(rng.choice([2, 4, 4, 8, 8]))
    per = 8 // bits
    if rng.random() < 0.5:
        row_bytes = 256 * int(rng.integers(1, 9))
    else:
        row_bytes = int(rng.integers(1, 200)) * (4 if rng.random() < 0.7 else 1)
    d = row_bytes * per
    sizes = [b for b in (16, 32, 64, 128, 256) if d % b == 0]
    bs = int(rng.choice(sizes)) if sizes else d
    blocks = d // bs
    dtype = str(rng.choice(["u8", "s8"]))
    zp = rng.choice([None, "u8", "s8", "float"])
    sdt = str(rng.choice(["f16", "f16", "f32", "bf16"]))
    rows = int(rng.integers(1, 3000))
    shape = tuple(int(x) for x in rng.integers(1, 40, size=int(rng.integers(1, 3))))
    ids_dtype = np.int32 if rng.random() < 0.4 else np.int64
    return (bits, rows, row_bytes, blocks, dtype, None if zp is None else str(zp), sdt, shape, ids_dtype)


@pytest.mark.parametrize("seed", range(32))
def test_random_gather(ctx, seed):
    case = _draw_gather(seed)
    print(f"random gather seed={seed} {case}", flush=True)
    _check_gather(ctx, case)
