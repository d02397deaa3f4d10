"""Checks that pin the oracle where the fixtures leave it open: closed forms, brute force on
tiny inputs, invariants, and mutations of the oracle that those checks (or the fixtures)
catch. A mutation is planted in a copy of the oracle on the CPU, never in the product."""

import zlib

import numpy as np
import pytest

from fixtures import Fixture, max_diff, tolerance
from oracle import oracle as o
from synth import nbits_weight, pack


# ---------------------------------------------------------------- unpack


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_pack_unpack_round_trip(bits):
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 2 ** bits, (5, 64))
    assert np.array_equal(o.unpack(pack(q, bits), bits), q)


def test_unpack_every_byte_low_bits_first():
    """Brute force over all 256 bytes: element 2i is the low nibble of byte i (packed.ex:3)."""
    b = np.arange(256, dtype=np.uint8)[:, None]
    v4 = o.unpack(b, 4)
    v2 = o.unpack(b, 2)
    for byte in range(256):
        assert list(v4[byte]) == [byte & 15, byte >> 4]
        assert list(v2[byte]) == [(byte >> s) & 3 for s in (0, 2, 4, 6)]


def test_unpack_signed_int4():
    """int4 data loads as s8 bytes and sign extends: 0xF0 holds 0 then -1; 0x87 holds 7 then -8."""
    data = np.array([[-16, -121]], dtype=np.int8)  # 0xF0, 0x87
    assert o.unpack_signed(data, 4).tolist() == [[0, -1, 7, -8]]
    # u8 data never sign extends.
    assert o.unpack_signed(data.view(np.uint8), 4).tolist() == [[0, 15, 7, 8]]


# ---------------------------------------------------------------- dequantize


def test_dequantize_weight_closed_forms():
    rng = np.random.default_rng(1)
    k, n, bits, bs = 64, 3, 4, 16
    b, s, _ = nbits_weight(rng, k, n, bits, bs, zp="none", scale_dtype=np.float32)
    w = o.dequantize_weight(b, s, None, k, n, bits, bs, o.F32)
    q = o.unpack(b.reshape(n, -1), bits).astype(np.float64)
    expect = (q - 8) * np.repeat(s.reshape(n, -1), bs, axis=1)
    assert np.array_equal(w, expect.astype(np.float32))
    # A zero point equal to every value gives zeros.
    q_const = np.full((n, k), 5)
    zp = pack(np.full((n, 4), 5), bits).reshape(-1)
    w0 = o.dequantize_weight(pack(q_const, bits).reshape(n, 4, 8), s, zp, k, n, bits, bs, o.F32)
    assert not np.any(w0)


def test_dequantize_weight_f16_rounds_once():
    """(q - z) is exact in f16 and the product rounds once: compare with a direct RNE of the
    exact f64 product."""
    rng = np.random.default_rng(2)
    k, n, bits, bs = 256, 8, 4, 32
    b, s, zp = nbits_weight(rng, k, n, bits, bs, zp="packed")
    w = o.dequantize_weight(b, s, zp, k, n, bits, bs, o.F16)
    q = o.unpack(b.reshape(n, -1), bits).astype(np.float64)
    z = o.unpack(zp.reshape(n, -1), bits)[:, : k // bs].astype(np.float64)
    exact = (q - np.repeat(z, bs, axis=1)) * np.repeat(s.reshape(n, -1).astype(np.float64), bs, axis=1)
    assert np.array_equal(w, exact.astype(np.float16))


def test_packed_zero_point_rows_are_padded():
    """K=72, block 32: 3 blocks per row take 2 bytes of 4-bit zero points (quantized.ex:316-323)."""
    rng = np.random.default_rng(3)
    k, n, bits, bs = 72, 5, 4, 32
    b, s, zp = nbits_weight(rng, k, n, bits, bs, zp="packed", scale_dtype=np.float32)
    assert zp.size == n * 2
    w = o.dequantize_weight(b, s, zp, k, n, bits, bs, o.F32)
    zrows = o.unpack(zp.reshape(n, 2), bits)
    for row in range(n):
        for blk in range(3):
            cols = slice(blk * bs, min(k, (blk + 1) * bs))
            q = o.unpack(b[row].reshape(-1), bits)[cols]
            expect = ((q - zrows[row, blk]) * s[row * 3 + blk]).astype(np.float32)
            assert np.array_equal(w[row, cols], expect)


def brute_matmul_nbits(a, b, scales, zp, k, n, bits, bs):
    """Element by element with Python integers: W[j][c] from byte c*bits//8 of row j."""
    blocks = -(-k // bs)
    row_bytes = blocks * bs * bits // 8
    zrow = -(-blocks * bits // 8)
    flat_b = b.reshape(n, row_bytes)
    y = np.zeros((a.shape[0], n))
    for j in range(n):
        for c in range(k):
            byte = int(flat_b[j, c * bits // 8])
            q = (byte >> ((c * bits) % 8)) & ((1 << bits) - 1)
            blk = c // bs
            if zp is None:
                z = 1 << (bits - 1)
            else:
                zb = int(zp[j * zrow + blk * bits // 8])
                z = (zb >> ((blk * bits) % 8)) & ((1 << bits) - 1)
            w = float(np.float32(q - z) * np.float32(scales[j * blocks + blk]))
            for i in range(a.shape[0]):
                y[i, j] += float(a[i, c]) * w
    return y


@pytest.mark.parametrize("bits,bs,zp,k", [(4, 16, "packed", 40), (8, 32, "none", 64), (2, 16, "packed", 48),
                                          (4, 32, "none", 72)])
def test_matmul_nbits_brute_force(bits, bs, zp, k):
    rng = np.random.default_rng(bits * 100 + k)
    n = 6
    b, s, z = nbits_weight(rng, k, n, bits, bs, zp=zp, scale_dtype=np.float32)
    a = rng.standard_normal((3, k)).astype(np.float32)
    y = o.matmul_nbits(a, b, s, z, k=k, n=n, bits=bits, block_size=bs)
    ref = brute_matmul_nbits(a, b, s, z, k, n, bits, bs)
    assert np.abs(y - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


def test_matmul_nbits_linear_in_a():
    rng = np.random.default_rng(4)
    k, n = 128, 16
    b, s, z = nbits_weight(rng, k, n, 4, 32, scale_dtype=np.float32)
    a1 = rng.standard_normal((2, k)).astype(np.float32)
    a2 = rng.standard_normal((2, k)).astype(np.float32)
    y = lambda a: o.matmul_nbits(a, b, s, z, k=k, n=n, bits=4, block_size=32).astype(np.float64)
    assert np.allclose(y(a1 + a2), y(a1) + y(a2), atol=1e-5)


def test_moved_weight_type_is_the_scales_type():
    """f32 A with f16 scales: the moved path dequantizes in f16 and gives f32 outputs."""
    rng = np.random.default_rng(5)
    b, s, z = nbits_weight(rng, 64, 8, 4, 32)
    a = rng.standard_normal((1, 64)).astype(np.float32)
    y = o.matmul_nbits(a, b, s, z, k=64, n=8, bits=4, block_size=32, weight_dtype=o.F16)
    assert y.dtype == np.float32
    w16 = o.dequantize_weight(b, s, z, 64, 8, 4, 32, o.F16)
    assert np.allclose(y, a.astype(np.float64) @ w16.astype(np.float64).T, rtol=1e-6, atol=1e-6)


def test_bf16_rounding_is_nearest_even():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.00390625, np.inf, 3.0e38], dtype=np.float32)
    bits = o.bf16_round(x)
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: it rounds to the even 1.0.
    assert o.bf16_to_f32(bits).tolist()[:4] == [1.0, 1.0, 1.015625, -2.0]
    assert np.isinf(o.bf16_to_f32(bits)[4])


def test_bf16_rounding_keeps_the_shape():
    """A 0-d value stays 0-d (a scalar DequantizeLinear scale), and the dequantized scalar with it;
    NaN keeps its quiet pattern whatever the shape."""
    assert o.bf16_round(np.float32(0.5)).shape == ()
    assert o.bf16_round(np.zeros((3, 0, 2), np.float32)).shape == (3, 0, 2)
    assert o.bf16_round(np.full((2, 3), np.nan, np.float32)).tolist() == [[0x7FC0] * 3] * 2
    y = o.dequantize_linear(np.array(7, np.uint16), o.bf16_round(np.float32(0.5)), axis=0)
    assert y.shape == () and o.bf16_to_f32(y) == 3.5


# ---------------------------------------------------------------- other operators


def test_matmul_integer_small_brute_force():
    rng = np.random.default_rng(6)
    a = rng.integers(0, 256, (2, 3, 7)).astype(np.uint8)
    b = rng.integers(-128, 128, (7, 4)).astype(np.int8)
    az = rng.integers(0, 256, (3,)).astype(np.uint8)
    bz = rng.integers(-128, 128, (4,)).astype(np.int8)
    y = o.matmul_integer(a, b, az, bz)
    for bt in range(2):
        for m in range(3):
            for nn in range(4):
                s = sum((int(a[bt, m, kk]) - int(az[m])) * (int(b[kk, nn]) - int(bz[nn])) for kk in range(7))
                assert y[bt, m, nn] == s


def test_matmul_integer_wraps_like_s32():
    a = np.full((1, 70000), 255, np.uint8)
    b = np.full((70000, 1), 255, np.uint8)
    exact = 70000 * 255 * 255
    assert o.matmul_integer(a, b)[0, 0] == np.int64(exact).astype(np.int32)


def test_dequantize_linear_blocked_closed_form():
    x = np.arange(10, dtype=np.uint8).reshape(2, 5)
    s = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    z = np.array([[1, 0], [0, 2]], np.uint8)
    y = o.dequantize_linear(x, s, z, axis=1, block_size=3)
    expect = np.array([[-1, 0, 1, 6, 8], [15, 18, 21, 24, 28]], np.float32)
    assert np.array_equal(y, expect)


def test_gather_matches_dequantized_table():
    """A gathered row is the dequantized table row: gather == take(dequantize(table))."""
    rng = np.random.default_rng(7)
    data = pack(rng.integers(0, 16, (20, 64)), 4)
    scales = (rng.random((20, 4)) * 0.1).astype(np.float16)
    zp = pack(rng.integers(0, 16, (20, 4)), 4)
    ids = np.array([[3, 19, 0, 3]])
    y = o.gather_block_quantized(data, ids, scales, zp, bits=4)
    table = o.dequantize(o.cast(o.unpack(data, 4).astype(np.float32), o.F16),
                         o.block_zero_points(zp, (20, 4), 4, o.F16), scales, o.F16)
    assert np.array_equal(y, table[ids])


# ---------------------------------------------------------------- mutations


def _fails(fn) -> bool:
    try:
        fn()
    except AssertionError:
        return True
    return False


def test_mutation_high_nibble_first_is_caught():
    f = Fixture("GatherBlockQuantized_b4")
    data, ids, s, zp = (f.values()[n] for n in f.node.input)

    def swapped(packed, bits):
        v = o.unpack(packed, bits)
        return v.reshape(*v.shape[:-1], -1, 2)[..., ::-1].reshape(v.shape)

    q = swapped(np.take(data, ids, axis=0), 4).astype(np.float32)
    zero = o.unpack(np.take(zp, ids, axis=0), 4)[..., :4].astype(np.float32)
    y = o.dequantize(q, zero, np.take(s, ids, axis=0), o.F32)
    assert not np.array_equal(y, f.outputs["Y"])


def test_mutation_default_zero_point_is_caught():
    f = Fixture("MatMulNBits_b4_bs32_none_bias")
    A, B, S = (f.values()[n] for n in f.node.input[:3])
    bias = f.values()["bias"]
    w = o.dequantize(o.unpack(B.reshape(16, -1), 4).astype(np.float32), np.float32(0), S.reshape(16, 3), o.F32)[:, :72]
    y = A.astype(np.float64) @ w.T.astype(np.float64) + bias
    assert max_diff(y, f.outputs["Y"]) > tolerance(f.outputs["Y"])


def test_mutation_transposed_zero_points_is_caught():
    f = Fixture("MatMulNBits_b4_bs16_packed")
    A, B, S, Z = (f.values()[n] for n in f.node.input[:4])
    n, blocks = 24, 4
    zero = o.unpack(Z.reshape(n, -1), 4)[:, :blocks].astype(np.float32)
    zero_t = zero.reshape(-1).reshape(blocks, n).T
    w = o.dequantize(o.unpack(B.reshape(n, -1), 4).astype(np.float32), zero_t, S.reshape(n, blocks), o.F32)
    y = A.astype(np.float64) @ w.T.astype(np.float64)
    assert max_diff(y, f.outputs["Y"]) > tolerance(f.outputs["Y"])


def test_mutation_f16_product_is_caught():
    f = Fixture("DequantizeLinear_int32_f16_scale")
    x, s, z = (f.values()[n] for n in f.node.input)
    y = ((x.astype(np.int64) - z).astype(np.float16) * s).astype(np.float16)
    assert not np.array_equal(y, f.outputs["y"])


def test_mutation_missing_zero_shift_is_caught():
    f = Fixture("MatMulInteger_k4096_signed")
    a = f.inputs["a"]
    b = f.initializers["b"]
    y = o.matmul_integer(a, b)  # zero points dropped
    assert not np.array_equal(y, f.outputs["y"])


# ---------------------------------------------------------------- QMoE in f16


def _qmoe_exact_case(k, router):
    """Two experts of identity MLPs whose every value is exact in f16: 4-bit weights in 6..10
    with per-row scale 0.5 and the default zero 8 give weights in {-1, -0.5, 0, 0.5, 1}; inputs
    in {-1, 0, 1}. fc1 sums stay at most 16 (multiples of 0.5), fc2 sums at most 256 (multiples
    of 0.25), and 0.5-weighted pairs of those multiples of 0.125 below 256: all exact in f16."""
    rng = np.random.default_rng(11)
    e, h, n1 = 2, 16, 16
    q1 = rng.integers(6, 11, (e, n1, h))
    q2 = rng.integers(6, 11, (e, h, n1))
    x = rng.integers(-1, 2, (len(router), h)).astype(np.float16)
    s1 = np.full((e, n1), 0.5, np.float16)
    s2 = np.full((e, h), 0.5, np.float16)
    y = o.qmoe(x, np.asarray(router, np.float32), pack(q1.reshape(e * n1, h), 4).reshape(e, n1, h // 2), s1,
               pack(q2.reshape(e * h, n1), 4).reshape(e, h, n1 // 2), s2, k=k, bits=4, block_size=0,
               activation="identity")
    w1 = (q1 - 8) * 0.5
    w2 = (q2 - 8) * 0.5
    return x.astype(np.float64), w1, w2, y


def test_qmoe_f16_closed_form_top1():
    """k = 1: each token's output is its one expert's MLP, weight softmax([v]) = 1 exactly."""
    router = [[1.0, 0.0], [0.0, 2.0], [-3.0, 5.0], [4.0, 4.0]]
    x, w1, w2, y = _qmoe_exact_case(1, router)
    assert y.dtype == np.float16
    for t, row in enumerate(router):
        e = int(np.argmax(row))  # stable: expert 0 for the tie of token 3
        assert np.array_equal(y[t].astype(np.float64), (x[t] @ w1[e].T) @ w2[e].T)


def test_qmoe_f16_closed_form_top2_ties():
    """k = 2 of 2 with equal router values: weights 0.5 and 0.5, y = (mlp_0 + mlp_1) / 2."""
    router = [[0.25, 0.25], [-1.0, -1.0], [3.0, 3.0]]
    x, w1, w2, y = _qmoe_exact_case(2, router)
    for t in range(len(router)):
        want = 0.5 * ((x[t] @ w1[0].T) @ w2[0].T) + 0.5 * ((x[t] @ w1[1].T) @ w2[1].T)
        assert np.array_equal(y[t].astype(np.float64), want)


@pytest.mark.parametrize("act,fusion,fc3,bs", [("silu", 0, False, 32), ("swiglu", 0, True, 32),
                                               ("swiglu", 2, False, 0), ("gelu", 0, False, 16)])
def test_qmoe_f16_agrees_with_f32_within_f16_rounding(act, fusion, fc3, bs):
    """The f16 mode rounds the weights, products, activation steps and weighted outputs to f16:
    it must stay within 4 f16 ulps of the largest output (2^-11 relative each; about 1.5 are
    seen) of the f32 mode on the same values, and the rounding must be visible."""
    rng = np.random.default_rng(zlib.crc32(repr((act, fusion, fc3, bs)).encode()))
    e, k, t, h, n1 = 8, 2, 12, 64, 32
    inter = n1 if (act != "swiglu" or fc3) else n1 // 2

    def weight(n, kk):
        packed = rng.integers(0, 256, (e, n, kk // 2), dtype=np.uint8)
        shape = (e, n, kk // bs) if bs else (e, n)
        return packed, (np.abs(rng.standard_normal(shape)) * 0.02 + 1e-3).astype(np.float16)

    w1, s1 = weight(n1, h)
    w2, s2 = weight(h, inter)
    w3, s3 = weight(n1, h) if fc3 else (None, None)
    x = rng.standard_normal((t, h)).astype(np.float16)
    router = rng.standard_normal((t, e)).astype(np.float32)
    kw = dict(k=k, bits=4, block_size=bs, activation=act, swiglu_fusion=fusion, fc3=w3, fc3_scales=s3)
    y16 = o.qmoe(x, router, w1, s1, w2, s2, **kw).astype(np.float64)
    y32 = o.qmoe(x.astype(np.float32), router, w1, s1, w2, s2, **kw).astype(np.float64)
    scale = np.abs(y32).max()
    diff = np.abs(y16 - y32).max()
    assert 0 < diff <= 4 * 2.0 ** -11 * scale, (diff, scale)


def test_routing_ties_keep_the_lower_expert_first():
    """`MoE.topk/2` (moe.ex:157-165): a stable descending sort, so among equal router values the
    lower expert index comes first; +0 and -0 compare equal."""
    probs = np.array([[0.5, 0.5, 0.5, 0.1],
                      [0.0, -0.0, 0.0, -1.0],
                      [-0.0, 0.0, 1.0, 1.0],
                      [2.0, 3.0, 3.0, 2.0]], np.float32)
    vals, idx = o.topk_stable(probs, 3)
    assert idx.tolist() == [[0, 1, 2], [0, 1, 2], [2, 3, 0], [1, 2, 0]]
    assert np.array_equal(np.take_along_axis(probs, idx, axis=1), vals)
