"""The benchmark workloads at their full sizes against the oracle: the single op of the CPU
path (f32 A [1, 1024], q4 block 32 B [3072, 32, 16], f32 scales, no zero points; f32 Y within
1e-3), the Qwen3-0.6B decode projections (q4, block 32, packed zero points, M in {1, 4, 8,
16}), the SmolLM3-3B prefill
projections (q4, block 128, M in {256, 2048}), the 151936 x 1024 lm_head (M = 1 and 8) and the
Qwen3-30B-A3B QMoE layer (128 experts, top-8, 2048/768, swiglu, 512 tokens). Outputs within
max|Y - Y_ref| / max|Y_ref| <= 1e-2 (f16 activations); QMoE (f16) within 1e-2 * max|ref| of the oracle's f16 mode; the
dequantized decode weights bit-exactly. Shapes and seeds are printed before each case."""

import zlib

import numpy as np
import pytest

from oracle import oracle as o
from synth import nbits_weight
from transmuter_amd import PackedWeight, moe
from transmuter_amd.onnx_wire import ATTR_INT, ATTR_STRING, AttributeProto, NodeProto
from transmuter_amd.quantized import matmul_nbits

pytestmark = pytest.mark.gpu

QWEN3_0_6B = [("q", 1024, 2048), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 2048, 1024),
              ("gate", 1024, 3072), ("up", 1024, 3072), ("down", 3072, 1024)]
SMOLLM3_3B = [("attn", 2048, 2048), ("mlp_up", 2048, 11008), ("mlp_down", 11008, 2048)]


def rel_err(y, ref):
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def check_matmul(ctx, name, k, n, bs, ms, scale_mul):
    rng = np.random.default_rng(zlib.crc32(f"{name}/{k}/{n}/{bs}".encode()))
    b, s, z = nbits_weight(rng, k, n, 4, bs, zp="packed", scale_mul=scale_mul)
    w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=4, block_size=bs, weight_dtype="f16")
    wf = o.dequantize_weight(b, s, z, k, n, 4, bs, o.F16).astype(np.float64)
    try:
        for m in ms:
            print(f"{name} K={k} N={n} block={bs} M={m}", flush=True)
            a = rng.standard_normal((m, k)).astype(np.float16)
            y = matmul_nbits(ctx.put(a), w).numpy()
            assert y.dtype == np.float16 and y.shape == (m, n)
            ref = a.astype(np.float64) @ wf.T
            err = rel_err(y.astype(np.float64), ref)
            assert err <= 1e-2, f"{name} M={m}: relative error {err}"
    finally:
        w.free()


def test_single_op_f32(ctx):
    k, n = 1024, 3072
    print(f"single op f32 K={k} N={n} M=1", flush=True)
    rng = np.random.default_rng(1)
    b, s, z = nbits_weight(rng, k, n, 4, 32, zp="none", scale_dtype=np.float32)
    w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=4, block_size=32, weight_dtype="f32")
    try:
        a = rng.standard_normal((1, k)).astype(np.float32)
        y = matmul_nbits(ctx.put(a), w).numpy()
    finally:
        w.free()
    ref = o.matmul_nbits(a, b, s, z, k=k, n=n, bits=4, block_size=32)
    assert y.dtype == np.float32 and ref.dtype == np.float32 and y.shape == (1, n)
    err = rel_err(y.astype(np.float64), ref.astype(np.float64))
    assert err <= 1e-3, f"relative error {err}"


@pytest.mark.parametrize("proj", QWEN3_0_6B, ids=lambda p: p[0])
def test_decode_projection(ctx, proj):
    name, k, n = proj
    check_matmul(ctx, name, k, n, 32, [1, 4, 8, 16], 0.01)


def test_decode_weight_dequantizes_bit_exactly(ctx):
    k, n = 3072, 1024
    print(f"dequantize down K={k} N={n}", flush=True)
    rng = np.random.default_rng(7)
    b, s, z = nbits_weight(rng, k, n, 4, 32, zp="packed")
    w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=4, block_size=32, weight_dtype="f16")
    try:
        got = w.dequantize().numpy()
    finally:
        w.free()
    ref = o.export(o.dequantize_weight(b, s, z, k, n, 4, 32, o.F16), o.F16)
    assert np.array_equal(got.view(np.uint16), np.ascontiguousarray(ref).view(np.uint16))


@pytest.mark.parametrize("proj", SMOLLM3_3B, ids=lambda p: p[0])
def test_prefill_projection(ctx, proj):
    name, k, n = proj
    check_matmul(ctx, name, k, n, 128, [256, 2048], 0.005)


@pytest.mark.parametrize("adt", ["f32", "bf16"])
@pytest.mark.parametrize("proj", SMOLLM3_3B, ids=lambda p: p[0])
def test_prefill_projection_f32_and_bf16(ctx, proj, adt):
    """The SmolLM3-3B prefill projections with f32 activations and weights (scales f32: the
    reference's :compute_type f32 after move/2, lib/transmuter.ex:49-93 and :1230-1233) within 1e-3,
    and with bf16 activations and weights within 2e-2, at M = 256 and 2048, against the oracle's
    dequantized weights in that type."""
    from transmuter_amd.device import bf16_bits_to_f32, f32_to_bf16_bits

    name, k, n = proj
    rng = np.random.default_rng(zlib.crc32(f"{name}/{k}/{n}/{adt}".encode()))
    b, s, z = nbits_weight(rng, k, n, 4, 128, zp="packed", scale_mul=0.005, scale_dtype=np.float32)
    if adt == "bf16":
        sw = o.bf16_round(s)
        w = PackedWeight.upload(ctx, b, sw, z, k=k, n=n, bits=4, block_size=128, weight_dtype="bf16",
                                scales_dtype="bf16")
        wf = o.dequantize_weight(b, o.bf16_to_f32(sw), z, k, n, 4, 128, o.BF16)  # exact bf16 values
    else:
        w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=4, block_size=128, weight_dtype="f32")
        wf = o.dequantize_weight(b, s, z, k, n, 4, 128, o.F32)
    wf = np.asarray(wf, np.float64)
    try:
        for m in (256, 2048):
            print(f"{name} {adt} K={k} N={n} block=128 M={m}", flush=True)
            a32 = rng.standard_normal((m, k)).astype(np.float32)
            if adt == "bf16":
                bits = f32_to_bf16_bits(a32)
                a_d, a64 = ctx.put(bits, "bf16"), bf16_bits_to_f32(bits).astype(np.float64)
            else:
                a_d, a64 = ctx.put(a32), a32.astype(np.float64)
            y = matmul_nbits(a_d, w)
            assert y.dtype == adt and y.shape == (m, n)
            got = y.numpy()
            got = bf16_bits_to_f32(got).astype(np.float64) if adt == "bf16" else got.astype(np.float64)
            ref = a64 @ wf.T
            err = rel_err(got, ref)
            assert err <= (1e-3 if adt == "f32" else 2e-2), f"{name} {adt} M={m}: relative error {err}"
    finally:
        w.free()


def test_lm_head(ctx):
    check_matmul(ctx, "lm_head", 1024, 151936, 32, [1, 8], 0.01)


def _attr(name, value):
    if isinstance(value, str):
        return AttributeProto(name=name, type=ATTR_STRING, s=value.encode())
    return AttributeProto(name=name, type=ATTR_INT, i=value)


def test_qmoe_layer(ctx):
    experts, k, hidden, inter, tokens = 128, 8, 2048, 768, 512
    print(f"qmoe E={experts} k={k} H={hidden} I={inter} T={tokens}", flush=True)
    rng = np.random.default_rng(6)

    def weight(n, kk):
        packed = rng.integers(0, 256, (experts, n, kk // 2), dtype=np.uint8)
        scales = (np.abs(rng.standard_normal((experts, n, kk // 32))) * 0.01 + 1e-4).astype(np.float16)
        return packed, scales

    (w1, s1), (w3, s3), (w2, s2) = weight(inter, hidden), weight(inter, hidden), weight(hidden, inter)
    x = rng.standard_normal((tokens, hidden)).astype(np.float16)
    router = rng.standard_normal((tokens, experts)).astype(np.float32)
    node = NodeProto(op_type="QMoE", input=[], output=["y"],
                     attribute=[_attr("k", k), _attr("expert_weight_bits", 4), _attr("block_size", 32),
                                _attr("activation_type", "swiglu"), _attr("swiglu_fusion", 0)])
    (y,) = moe.apply(node, [ctx.put(x), ctx.put(router), w1, s1, None, w2, s2, None, w3, s3, None, None, None, None])
    got = y.numpy().astype(np.float64)
    ref = o.qmoe(x, router, w1, s1, w2, s2, k=k, bits=4, block_size=32, activation="swiglu",
                 swiglu_fusion=0, fc3=w3, fc3_scales=s3).astype(np.float64)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 1e-2 * scale, f"max difference {np.abs(got - ref).max()} (max |ref| {scale})"
