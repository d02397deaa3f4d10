"""CPU oracle for the quantized-weight operators: a numpy restatement of the reference's algorithm.

TEST INFRASTRUCTURE ONLY. Nothing in the product imports this module: only tests/, the
smoke check of __graft_entry__.py and the CPU-baseline leg of bench.py use it, and only as
the checker. The HIP library never calls into it and has no CPU fallback.

Each function follows the Elixir source cited in its docstring (paths are into the
georgeguimaraes/transmuter repository). Floating-point rounding follows Nx's types: an f16
or bf16 operation computes in f32 and rounds once to the narrow type (numpy's float16 ufuncs
do exactly that; bf16 is emulated with round-to-nearest-even on the f32 bits). Matmul sums
accumulate in f64 and round once to the output type, so the oracle is at least as accurate as
the reference's f32 dot; parity for matmul outputs is a tolerance, never bits.

How each function is pinned (tests/test_oracle_golden.py, tests/test_oracle_math.py):
- unpack / unpack_signed: the reference's low-bits-first rule (packed.ex:3), pack/unpack
  round trip, brute force per byte, and the GatherBlockQuantized fixtures (bit-exact).
- block_zero_points / dequantize / dequantize_weight: the GatherBlockQuantized_b4/_b8 ORT
  fixtures (bit-exact), the six MatMulNBits ORT fixtures through matmul_nbits, and closed
  forms (q == zero gives 0; no zero point gives (q - 2^(bits-1)) * s).
- matmul_nbits: six ORT fixtures (bits 2/4/8, block 16/32/256, zero points none, packed,
  float, a bias, K=72 not a multiple of the block) at 1e-4 + 1e-3 * max|Y|, and an
  element-by-element brute force on tiny shapes.
- gather_block_quantized: two ORT fixtures, bit-exact.
- dequantize_linear: four ORT fixtures (per tensor, per axis, blocked, int32 with an f16
  scale), bit-exact.
- matmul_integer: four ORT fixtures, exact, including two sums past 2^24.
- qmoe: six ORT QMoE fixtures (4 and 8 bits, block and per-row scales, per-row zero points,
  silu and interleaved swiglu, k = 1 and 2) at the fixtures' tolerance.
- dynamic_quantize_linear: three ORT fixtures, bit-exact.
A mutated copy of each function (wrong nibble order, wrong default zero point, missing sign
extension, transposed zero points, f16 instead of f32 product) fails those checks.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------- dtypes

F32, F16, BF16 = "f32", "f16", "bf16"


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Rounds f32 values to bf16 (nearest even), returned as uint16 bit patterns of x's shape
    (a 0-d input stays 0-d)."""
    x = np.asarray(x, dtype=np.float32)
    flat = np.ascontiguousarray(x.reshape(-1))
    u = flat.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(flat), np.uint16(0x7FC0), rounded).astype(np.uint16).reshape(x.shape)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def cast(x, dtype: str) -> np.ndarray:
    """`Nx.as_type/2` to a float type, rounding to nearest even. f16 values are numpy float16;
    bf16 values are f32 arrays that hold exact bf16 numbers."""
    x = np.asarray(x)
    if dtype == F32:
        return x.astype(np.float32)
    if dtype == F16:
        return x.astype(np.float16)
    if dtype == BF16:
        return bf16_to_f32(bf16_round(x.astype(np.float32)))
    raise ValueError(dtype)


def _narrow(x, dtype: str) -> np.ndarray:
    """Rounds the result of one operation (f32, or f64 for a sum) to dtype."""
    x = np.asarray(x)
    if dtype == F32:
        return x.astype(np.float32)
    if dtype == F16:
        return x.astype(np.float16)
    return bf16_to_f32(bf16_round(x.astype(np.float32)))


def _op(a, b, fn, dtype):
    """One elementwise operation in dtype: computed in f32, rounded once to dtype."""
    return _narrow(fn(np.asarray(a, dtype=np.float32), np.asarray(b, dtype=np.float32)), dtype)


def export(x: np.ndarray, dtype: str) -> np.ndarray:
    """The array a caller sees: bf16 values as uint16 bit patterns, others as they are."""
    return bf16_round(x) if dtype == BF16 else x


def floats(x) -> tuple[np.ndarray, str]:
    """A float input and its type: float16, float32, or uint16 bit patterns of bf16."""
    x = np.asarray(x)
    if x.dtype == np.float16:
        return x, F16
    if x.dtype == np.float32:
        return x, F32
    if x.dtype == np.uint16:
        return bf16_to_f32(x), BF16
    raise ValueError(f"not a float array: {x.dtype}")


def merge_types(*dtypes: str) -> str:
    """Nx.Type.merge/2 for the float types: f16 with f16 is f16, bf16 with bf16 is bf16,
    any other mix is f32."""
    ds = set(dtypes)
    if ds == {F16}:
        return F16
    if ds == {BF16}:
        return BF16
    return F32


# ---------------------------------------------------------------- unpack / dequantize


def unpack(packed: np.ndarray, bits: int) -> np.ndarray:
    """`Packed.unpack/2` (lib/transmuter/ops/packed.ex:9-23): the `bits`-wide unsigned values of
    the bytes on the last axis, lowest bits first; element i*per + j is bits j*bits.. of byte i.
    8-bit values stay as they are."""
    if bits == 8:
        return np.asarray(packed)
    per = 8 // bits
    mask = (1 << bits) - 1
    b = np.asarray(packed).astype(np.int16) & 0xFF
    shifts = np.arange(per, dtype=np.int16) * bits
    values = (b[..., None] >> shifts) & mask
    return values.reshape(*b.shape[:-1], b.shape[-1] * per)


def unpack_signed(packed: np.ndarray, bits: int) -> np.ndarray:
    """`Quantized.unpack/2` (lib/transmuter/ops/quantized.ex:294-300): int4 tensors load as s8
    bytes (ops.ex:632-639) and their values are sign extended; other data stays unsigned."""
    values = unpack(packed, bits)
    if bits < 8 and np.asarray(packed).dtype == np.int8:
        values = values - (values >= (1 << (bits - 1))).astype(values.dtype) * (1 << bits)
    return values


def block_zero_points(zero, shape, bits: int, dtype: str, signed: bool = False) -> np.ndarray:
    """`Quantized.block_zero_points/5` (quantized.ex:306-325): per-block zero points of `shape`
    in dtype. None: 0 for signed data, else 2^(bits-1). Float zero points reshape and cast.
    Integer zero points are packed along each row: rows of ceil(blocks*bits/8) bytes, unpacked
    (sign extended when s8) and cut to the first `blocks` values."""
    if zero is None:
        return cast(np.float32(0.0 if signed else 2 ** (bits - 1)), dtype)
    zero = np.asarray(zero)
    if zero.dtype.kind == "f":
        return cast(zero.reshape(shape), dtype)
    blocks = shape[-1]
    rows = zero.reshape(*shape[:-1], -1)
    return cast(unpack_signed(rows, bits)[..., :blocks].astype(np.float32), dtype)


def dequantize(q, zero, scales, dtype: str) -> np.ndarray:
    """`Packed.dequantize/3` (lib/transmuter/ops/packed.ex:28-36): (q - zero) * scales for each
    block of the last axis, each operation in dtype."""
    q = np.asarray(q)
    scales = np.asarray(scales)
    blocks = q.reshape(*scales.shape, -1)
    zero = np.asarray(zero)
    z = zero[..., None] if zero.ndim else zero
    diff = _op(blocks, z, np.subtract, dtype)
    out = _op(diff, scales[..., None], np.multiply, dtype)
    return out.reshape(q.shape)


def nbits_sizes(attrs: dict) -> tuple[int, int, int, int]:
    """`Quantized.nbits_sizes/1` (quantized.ex:226-228): {K, N, bits (4 by default), block_size}."""
    return attrs["K"], attrs["N"], attrs.get("bits", 4), attrs["block_size"]


def dequantize_weight(b, scales, zero_points, k: int, n: int, bits: int, block_size: int,
                      dtype: str) -> np.ndarray:
    """`Quantized.dequantize_weight/4` (quantized.ex:234-240): the {N, K} weights in dtype.
    B unpacks to {N, blocks*block_size}, scales reshape to {N, blocks}, the block zero points
    follow block_zero_points, and the dequantized values are cut to K columns."""
    blocks = (k + block_size - 1) // block_size
    q = cast(unpack_signed(np.asarray(b), bits).reshape(n, blocks * block_size).astype(np.float32), dtype)
    s = cast(np.asarray(scales).reshape(n, blocks), dtype)
    zero = block_zero_points(zero_points, (n, blocks), bits, dtype)
    return dequantize(q, zero, s, dtype)[:, :k]


def _dot_last(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Nx.dot(a, [-1], w, [1]) accumulated in f64."""
    return np.asarray(a, dtype=np.float64) @ np.asarray(w, dtype=np.float64).T


def matmul_nbits(a, b, scales, zero_points=None, bias=None, *, k: int, n: int, bits: int = 4,
                 block_size: int, weight_dtype: str | None = None, g_idx=None) -> np.ndarray:
    """MatMulNBits (quantized.ex:30-46): Y = A . W^T (+ bias).

    The in-graph path dequantizes W in A's type (:42); the moved path of `Transmuter.move/2`
    dequantizes it once in the scales' type after :compute_type (lib/transmuter.ex:1230-1240).
    `weight_dtype` selects the latter. Y has the merged type of A and W, then of the bias.
    """
    if g_idx is not None:
        raise ValueError("MatMulNBits with the g_idx input is not supported")
    a, a_type = floats(a)
    wtype = weight_dtype or a_type
    if np.asarray(b).shape == (n, k):
        w, wtype = floats(b)
    else:
        if np.asarray(scales).dtype == np.uint16:
            scales = bf16_to_f32(scales)
        w = dequantize_weight(b, scales, zero_points, k, n, bits, block_size, wtype)
    out_type = merge_types(a_type, wtype)
    acc = _dot_last(a, w)
    if bias is not None:
        bias, bias_type = floats(bias)
        y = _narrow(acc, out_type)
        out_type = merge_types(out_type, bias_type)
        return export(_op(y, bias, np.add, out_type), out_type)
    return export(_narrow(acc, out_type), out_type)


# ---------------------------------------------------------------- GatherBlockQuantized


def gather_block_quantized(data, indices, scales, zero_points=None, *, bits: int = 4,
                           gather_axis: int = 0, quantize_axis: int = 1) -> np.ndarray:
    """GatherBlockQuantized (quantized.ex:49-66): take rows of data, unpack (sign extended for
    s8 data), cast to the scales' type, and dequantize with the taken zero points and scales.
    Only gather_axis 0 with the quantize axis last is supported (:53-57)."""
    data = np.asarray(data)
    rank = data.ndim
    qa = quantize_axis + rank if quantize_axis < 0 else quantize_axis
    if gather_axis != 0 or qa != rank - 1:
        raise ValueError("GatherBlockQuantized supports gather_axis 0 and quantize_axis on the last axis")
    scales, dtype = floats(scales)
    idx = np.asarray(indices).astype(np.int64)
    taken = np.take(data, idx, axis=0)
    q = cast(unpack_signed(taken, bits).astype(np.float32), dtype)
    shape = q.shape[:-1] + (scales.shape[-1],)
    zp = None if zero_points is None else np.take(np.asarray(zero_points), idx, axis=0)
    zero = block_zero_points(zp, shape, bits, dtype, signed=data.dtype == np.int8)
    return export(dequantize(q, zero, np.take(scales, idx, axis=0), dtype), dtype)


# ---------------------------------------------------------------- DequantizeLinear


def _on_axis(t: np.ndarray, rank: int, axis: int) -> np.ndarray:
    """`Ops.on_axis/3` (ops.ex:440-443): a 1-D tensor laid along one axis of a rank-r value."""
    shape = [1] * rank
    shape[axis] = -1
    return t.reshape(shape)


def expand_quant_param(param: np.ndarray, x: np.ndarray, axis: int = 1, block_size: int = 0) -> np.ndarray:
    """`Quantized.expand_quant_param/3` (quantized.ex:328-353): per tensor (one value), blocked
    along the axis (each value repeated block_size times, cut to the axis size), or per axis."""
    rank = x.ndim
    axis = axis + rank if axis < 0 else axis
    param = np.asarray(param)
    if param.size == 1:
        return param.reshape(())
    if block_size > 0:
        rep = np.repeat(param, block_size, axis=axis)
        return np.take(rep, np.arange(x.shape[axis]), axis=axis)
    return _on_axis(param, rank, axis)


def dequantize_linear(x, scale, zero=None, *, axis: int = 1, block_size: int = 0) -> np.ndarray:
    """DequantizeLinear (quantized.ex:70-84): integer x subtracts the zero point in s32 (float x
    in f32), converts to f32, multiplies by the f32 scale, and rounds to the scale's type."""
    x = np.asarray(x)
    scale, out_type = floats(scale)
    if x.dtype.kind in "iu":
        shifted = x.astype(np.int64)
        if zero is not None:
            z = expand_quant_param(np.asarray(zero).astype(np.int64), x, axis, block_size)
            shifted = shifted - z
        shifted = ((shifted + 2**31) % 2**32 - 2**31).astype(np.int32)  # s32 wraps
        as_f32 = shifted.astype(np.float32)
    else:
        as_f32 = x.astype(np.float32)
        if zero is not None:
            z = expand_quant_param(np.asarray(zero).astype(np.float32), x, axis, block_size)
            as_f32 = (as_f32 - z).astype(np.float32)
    s = expand_quant_param(scale.astype(np.float32), x, axis, block_size)
    return export(_narrow((as_f32 * s).astype(np.float32), out_type), out_type)


# ---------------------------------------------------------------- MatMulInteger


def _per_axis(t, rank: int, axis: int) -> np.ndarray:
    """`Quantized.per_axis/3` (quantized.ex:288-291): a scalar, or a 1-D tensor on one axis."""
    t = np.asarray(t).astype(np.int64)
    return t.reshape(()) if t.size == 1 else _on_axis(t, rank, axis)


def matmul_integer(a, b, a_zero=None, b_zero=None) -> np.ndarray:
    """MatMulInteger (quantized.ex:105-110): the exact s32 sums of (a - a_zero)(b - b_zero).
    a_zero lies along A's rows (axis rank-2), b_zero along B's columns (axis rank-1). The
    reference sums f32 products in chunks of 256 (each exact, 256*255^2 < 2^24) and adds the
    chunks in s32 (lib/transmuter/ops/nn.ex:537-555); the exact integer sum wrapped to s32 is
    the same value. Batch axes broadcast as `Ops.matmul/2` does (ops.ex:465-491)."""
    a = np.asarray(a).astype(np.int64)
    b = np.asarray(b).astype(np.int64)
    if a_zero is not None:
        a = a - _per_axis(a_zero, a.ndim, a.ndim - 2 if a.ndim >= 2 else 0)
    if b_zero is not None:
        b = b - _per_axis(b_zero, b.ndim, b.ndim - 1)
    acc = np.matmul(a, b)
    return ((acc + 2**31) % 2**32 - 2**31).astype(np.int32)


# ---------------------------------------------------------------- DynamicQuantizeLinear


def _round_half_even(x: np.ndarray) -> np.ndarray:
    return np.round(x)  # numpy rounds half to even


def dynamic_quantize_linear(x) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """DynamicQuantizeLinear (quantized.ex:94-103): scale = (max(x,0) - min(x,0)) / 255 in f32
    (1 for a constant x), zero = saturate(round(-low / scale)), y = saturate(round(x / scale) + zero)."""
    x = np.asarray(x, dtype=np.float32)
    low = np.minimum(x.min(), np.float32(0))
    high = np.maximum(x.max(), np.float32(0))
    scale = np.float32(np.float32(high - low) / np.float32(255))
    if scale == 0:
        scale = np.float32(1)
    zero = np.clip(_round_half_even(np.float32(-low) / scale), 0, 255).astype(np.uint8)
    y = np.clip(_round_half_even((x / scale).astype(np.float32)) + np.float32(zero), 0, 255).astype(np.uint8)
    return y, np.float32(scale), zero


# ---------------------------------------------------------------- QMoE


def _softmax_last(x: np.ndarray) -> np.ndarray:
    """`Ops.softmax_last/1`: exp(x - max) / sum, in f32."""
    x = x.astype(np.float32)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def topk_stable(probs: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """`MoE.topk/2` (lib/transmuter/ops/moe.ex:158-165): a stable descending sort, so the lower
    expert index comes first among equal values."""
    idx = np.argsort(-probs, axis=1, kind="stable")[:, :k]
    return np.take_along_axis(probs, idx, axis=1), idx


def qmoe_dequant(packed, scales, zp, bits: int, block_size: int, dtype: str = F32) -> np.ndarray:
    """`MoE.dequant/6` (moe.ex:216-253): {E, N, K} weights. Block scales work in f32 with K padded
    to whole blocks; per-row scales {E, N} or {E, N, 1} use zero points packed along N."""
    q = unpack(np.asarray(packed), bits).astype(np.float32)
    e, n, k = q.shape
    default_zero = 2 ** (bits - 1)
    if block_size > 0 and scales is not None:
        scales = np.asarray(scales, dtype=np.float32)
        blocks = scales.shape[2]
        padded = blocks * block_size
        if padded > k:
            q = np.pad(q, ((0, 0), (0, 0), (0, padded - k)))
        if zp is not None:
            zero = unpack(np.asarray(zp), bits)[..., :blocks].astype(np.float32)
        else:
            zero = np.float32(default_zero)
        w = dequantize(q, zero, scales, F32)[..., :k]
        return cast(w, dtype)
    zero = unpack(np.asarray(zp), bits).astype(np.float32).reshape(e, n, 1) if zp is not None \
        else np.float32(default_zero)
    q_sub = cast(q, dtype).astype(np.float32) - zero
    q_sub = cast(q_sub, dtype)
    if scales is None:
        return q_sub
    s = cast(np.asarray(scales).reshape(e, n, 1), dtype)
    return _op(q_sub, s, np.multiply, dtype)


def _sigmoid(x):
    return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


def _swiglu_gate(g, lin, alpha, beta, limit):
    """`MoE.swiglu_gate/3` (moe.ex:199-206)."""
    if limit != 0:
        g = np.minimum(g, limit)
        lin = np.clip(lin, -limit, limit)
    return (g * _sigmoid(alpha * g) * (lin + beta)).astype(np.float32)


def _activate(h, activation, fusion, alpha, beta, limit):
    """`MoE.activate/2` (moe.ex:176-196)."""
    if activation == "relu":
        return np.maximum(h, 0)
    if activation == "silu":
        return (h * _sigmoid(h)).astype(np.float32)
    if activation == "identity":
        return h
    if activation == "gelu":
        from math import erf, sqrt
        verf = np.vectorize(erf)
        return (h * 0.5 * (1 + verf(h / sqrt(2)))).astype(np.float32)
    if activation == "swiglu":
        if fusion == 2:
            inter = h.shape[1] // 2
            return _swiglu_gate(h[:, :inter], h[:, inter:], alpha, beta, limit)
        pairs = h.reshape(h.shape[0], -1, 2)
        return _swiglu_gate(pairs[..., 0], pairs[..., 1], alpha, beta, limit)
    raise ValueError(activation)


def _narrow_activate(h, activation, fusion, alpha, beta, limit, dtype):
    """`MoE.activate/2` and `swiglu_gate/3` (moe.ex:176-206) on values of a narrow type: every Nx
    operation computes in f32 and rounds once to `dtype` (f16 or bf16), as each Nx op returns a
    tensor of its inputs' type (a Elixir float scalar takes the tensor's type)."""
    r = lambda v: _narrow(v, dtype).astype(np.float32)  # noqa: E731
    h = np.asarray(h, dtype=np.float32)

    def sigmoid(v):
        return r(1.0 / (1.0 + np.exp(-v.astype(np.float64))))

    def gate(g, lin):
        if limit != 0:
            g = np.minimum(g, np.float32(limit))
            lin = np.clip(lin, -np.float32(limit), np.float32(limit))
        return r(r(g * sigmoid(r(np.float32(alpha) * g))) * r(lin + np.float32(beta)))

    if activation == "relu":
        return np.maximum(h, 0)
    if activation == "silu":
        return r(h * sigmoid(h))
    if activation == "identity":
        return h
    if activation == "gelu":
        from math import erf, sqrt
        verf = np.vectorize(erf)
        inner = r(verf(r(h * np.float32(1.0 / sqrt(2)))))
        return r(h * r(np.float32(0.5) * r(np.float32(1.0) + inner)))
    if activation == "swiglu":
        if fusion == 2:
            inter = h.shape[1] // 2
            return gate(h[:, :inter], h[:, inter:])
        pairs = h.reshape(h.shape[0], -1, 2)
        return gate(pairs[..., 0], pairs[..., 1])
    raise ValueError(activation)


def qmoe(x, router, fc1, fc1_scales, fc2, fc2_scales, *, k: int, bits: int = 4, block_size: int = 0,
         activation: str = "relu", swiglu_fusion: int = 0, alpha: float = 1.0, beta: float = 0.0,
         limit: float = 0.0, fc1_bias=None, fc2_bias=None, fc3=None, fc3_scales=None, fc3_bias=None,
         fc1_zp=None, fc2_zp=None, fc3_zp=None) -> np.ndarray:
    """QMoE (moe.ex:42-61, 64-102), with the routed math: each token runs its top-k experts
    (top-k router values, then a softmax over those k values) and adds their outputs with the
    routing weights.

    The arithmetic follows the input's type (`type = Nx.type(input)`, moe.ex:47):
    - f32 input (numpy float32): expert products accumulate in f64, the sums in f64, one
      rounding to f32 at the end (the f32 arithmetic the ORT fixtures pin);
    - f16 input (numpy float16; or bf16 as uint16 bit patterns): as the reference computes it.
      The dequantized expert weights are cast to the input type (moe.ex:53, 225-253). Each
      expert product is one dot of input-type operands, accumulated exactly and rounded once
      to the input type (Nx.dot of f16 x f16 is f16). Bias adds, every operation of the
      activation, the routing weights (Nx.as_type(type), moe.ex:90) and each weighted output
      (Nx.multiply, moe.ex:97) each round to the input type. The slot sum (Nx.sum, moe.ex:99)
      adds exactly and rounds once.
    How the reference's backend orders and rounds its dot and sum accumulations is not fixed by
    Nx: with t*k >= E it sums over all E experts in expert order with weight 0 for the others
    (moe.ex:108-138), otherwise over the k slots. Parity for f16 is therefore a tolerance."""
    x, xt = floats(x)
    h = x.shape[-1]
    x2 = x.reshape(-1, h).astype(np.float32)
    top_vals, top_idx = topk_stable(np.asarray(router, dtype=np.float32), k)
    weights = _softmax_last(top_vals)
    narrow = xt in (F16, BF16)
    wtype = xt if narrow else F32

    def expert(fc, scales, zp, e):  # expert e's {N, K} weights: dequant/6 on its slice
        def part(t):
            return None if t is None else np.asarray(t)[e:e + 1]
        return np.asarray(qmoe_dequant(part(fc), part(scales), part(zp), bits, block_size, wtype)[0], np.float64)

    def rnd(v, *types):  # one operation's result in the merged type of its operands
        return _narrow(v, merge_types(*types)).astype(np.float64) if narrow else np.asarray(v, np.float64)

    def bias_row(b, e):
        b, bt = floats(np.asarray(b)[e])
        return b.astype(np.float64), bt

    n_tok = x2.shape[0]
    outs = np.zeros((n_tok, k, h), dtype=np.float64)
    for e in np.unique(top_idx):
        rows_t, rows_j = np.nonzero(top_idx == e)
        xe = x2[rows_t].astype(np.float64)
        h1 = rnd(xe @ expert(fc1, fc1_scales, fc1_zp, e).T, xt)
        if not narrow:
            h1 = h1.astype(np.float32)
        if fc1_bias is not None:
            b, bt = bias_row(fc1_bias, e)
            h1 = rnd(h1 + b, xt, bt) if narrow else (h1 + b.astype(np.float32)).astype(np.float32)
        if activation == "swiglu" and swiglu_fusion == 0 and fc3 is not None:
            h3 = rnd(xe @ expert(fc3, fc3_scales, fc3_zp, e).T, xt)
            if not narrow:
                h3 = h3.astype(np.float32)
            if fc3_bias is not None:
                b, bt = bias_row(fc3_bias, e)
                h3 = rnd(h3 + b, xt, bt) if narrow else (h3 + b.astype(np.float32)).astype(np.float32)
            if narrow:
                act = _narrow_activate(np.concatenate([h1, h3], axis=1), "swiglu", 2, alpha, beta, limit, xt)
            else:
                act = _swiglu_gate(h1, h3, alpha, beta, limit)
        elif narrow:
            act = _narrow_activate(h1, activation, swiglu_fusion, alpha, beta, limit, xt)
        else:
            act = _activate(h1, activation, swiglu_fusion, alpha, beta, limit)
        o = np.asarray(act, np.float64) @ expert(fc2, fc2_scales, fc2_zp, e).T
        if narrow:
            o = rnd(o, xt)
        if fc2_bias is not None:
            b, bt = bias_row(fc2_bias, e)
            o = rnd(o + b, xt, bt) if narrow else o + b
        outs[rows_t, rows_j] = o
    out = np.zeros_like(x2, dtype=np.float64)
    wts = rnd(weights, xt) if narrow else weights.astype(np.float64)
    for j in range(k):
        wt = wts[:, j]
        live = wt != 0
        term = wt[live, None] * outs[live, j]
        out[live] += rnd(term, xt) if narrow else term
    return export(_narrow(out, xt), xt).reshape(x.shape) if narrow else out.astype(np.float32).reshape(x.shape)
