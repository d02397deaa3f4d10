"""MatMulNBits on the GPU against the oracle: dequantized weights bit-exactly, Y within the
stated tolerance (max |Y - Y_ref| / max |Y_ref|: 1e-3 for f32 A, 1e-2 for f16 A, 2e-2 for bf16
A, whose output rounds to 8 significant bits). Seeds and shapes are printed before each case."""

import zlib

import numpy as np
import pytest

from oracle import oracle as o
from synth import nbits_weight
from transmuter_amd import PackedWeight
from transmuter_amd.quantized import matmul_nbits

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-3, "f16": 1e-2, "bf16": 2e-2}
NP = {"f32": np.float32, "f16": np.float16}


def host_float(x, dtype):
    return o.bf16_round(x) if dtype == "bf16" else np.asarray(x).astype(NP[dtype])


def as_f64(x, dtype):
    return o.bf16_to_f32(x).astype(np.float64) if dtype == "bf16" else np.asarray(x, np.float64)


def rel_err(y, ref):
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


DEQUANT_CASES = [
    # bits, block, zp kind, K, N, scale type, weight type
    (4, 32, "packed", 1024, 40, "f16", "f16"),
    (4, 32, "none", 72, 17, "f32", "f32"),
    (4, 16, "packed", 96, 33, "f16", "f16"),
    (4, 16, "float", 64, 8, "f32", "f16"),
    (4, 128, "packed", 1000, 24, "f16", "f16"),
    (4, 256, "packed", 512, 40, "f32", "f32"),
    (8, 32, "packed", 256, 19, "f16", "f16"),
    (8, 128, "none", 384, 16, "f32", "bf16"),
    (8, 16, "float", 48, 5, "f16", "f32"),
    (2, 16, "packed", 64, 9, "f32", "f32"),
    (2, 64, "none", 320, 31, "f16", "f16"),
    (4, 64, "packed", 200, 50, "bf16", "bf16"),
]


@pytest.mark.parametrize("case", DEQUANT_CASES, ids=lambda c: "b{}_bs{}_{}_K{}_N{}_{}_{}".format(*c))
def test_dequantize_bit_exact(ctx, case):
    bits, bs, zp, k, n, sdt, wdt = case
    print(f"dequant {case}", flush=True)
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    b, s32, z = nbits_weight(rng, k, n, bits, bs, zp=zp, scale_dtype=np.float32)
    scales = host_float(s32, sdt)
    w = PackedWeight.upload(ctx, b, scales, z, k=k, n=n, bits=bits, block_size=bs, weight_dtype=wdt,
                            scales_dtype=sdt)
    got = w.dequantize().numpy()
    ref = o.dequantize_weight(b, as_f64(scales, sdt).astype(np.float32), z, k, n, bits, bs, wdt)
    ref = o.export(ref, wdt)
    assert got.shape == (n, k)
    assert np.array_equal(got.view(np.uint8), np.ascontiguousarray(ref).view(np.uint8))
    w.free()


@pytest.mark.parametrize("case", DEQUANT_CASES, ids=lambda c: "b{}_bs{}_{}_K{}_N{}_{}_{}".format(*c))
def test_device_packing_equals_host_packing(ctx, case):
    """tmh_weight_pack_nbits repacks B, scales and zero points that are already on the device;
    the weight must be the host packing's, bit for bit: the same dequantized values and the same
    products."""
    bits, bs, zp, k, n, sdt, wdt = case
    print(f"device packing {case}", flush=True)
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()) + 1)
    b, s32, z = nbits_weight(rng, k, n, bits, bs, zp=zp, scale_dtype=np.float32)
    scales = host_float(s32, sdt)
    host = PackedWeight.upload(ctx, b, scales, z, k=k, n=n, bits=bits, block_size=bs, weight_dtype=wdt,
                               scales_dtype=sdt)
    dev = PackedWeight.pack_device(ctx, ctx.put(b), ctx.put(scales, sdt), None if z is None else ctx.put(z), k=k, n=n,
                                   bits=bits, block_size=bs, weight_dtype=wdt)
    assert np.array_equal(dev.dequantize().numpy().view(np.uint8), host.dequantize().numpy().view(np.uint8))
    adt = "f16" if wdt == "f16" else "f32"
    a = ctx.put(rng.standard_normal((3, k)).astype(NP[adt]))
    assert np.array_equal(matmul_nbits(a, dev).numpy().view(np.uint8), matmul_nbits(a, host).numpy().view(np.uint8))
    host.free()
    dev.free()


def test_in_graph_matmul_nbits_packs_on_the_device(ctx):
    """A MatMulNBits node that move/2 did not rewrite, with B on the device and small host scales
    and zero points (static values), runs through the device packing and matches the oracle."""
    from transmuter_amd import quantized
    from transmuter_amd.onnx_wire import ATTR_INT, AttributeProto, NodeProto

    print("in-graph MatMulNBits, device B", flush=True)
    rng = np.random.default_rng(77)
    k, n, bits, bs = 512, 48, 4, 32
    b, s, z = nbits_weight(rng, k, n, bits, bs)
    attrs = [AttributeProto(name=name, type=ATTR_INT, i=v) for name, v in (("K", k), ("N", n), ("bits", bits),
                                                                              ("block_size", bs))]
    node = NodeProto(op_type="MatMulNBits", input=["a", "b", "s", "z"], output=["y"], attribute=attrs)
    a = rng.standard_normal((2, 3, k)).astype(np.float16)
    (y,) = quantized.apply(node, [ctx.put(a), ctx.put(b), s, z])
    ref = o.matmul_nbits(a, b, s, z, k=k, n=n, bits=bits, block_size=bs).astype(np.float64)
    assert y.shape == (2, 3, n) and y.dtype == "f16"
    assert rel_err(y.numpy().astype(np.float64), ref) <= TOL["f16"]


MATMUL_CASES = [
    # bits, block, zp, K, N, M list, A type, scale type, bias
    (4, 32, "packed", 1024, 96, [1, 2, 5, 16, 17, 31, 33, 64, 65, 130], "f16", "f16", None),
    (4, 32, "packed", 72, 16, [1, 6, 70], "f16", "f16", "f16"),
    (4, 16, "packed", 256, 40, [1, 16, 40, 100], "f16", "f16", None),
    (4, 128, "packed", 2048, 64, [1, 8, 256], "f16", "f16", "f32"),
    (4, 256, "none", 512, 40, [3, 129], "f16", "f16", None),
    (8, 32, "packed", 512, 48, [1, 4, 66], "f16", "f16", None),
    (8, 128, "none", 1000, 20, [2, 200], "f16", "f16", "f16"),
    (2, 16, "packed", 256, 24, [1, 20, 80], "f16", "f16", None),
    (4, 32, "none", 1024, 48, [1, 3, 20], "f32", "f32", None),
    (4, 32, "float", 64, 8, [6, 17], "f32", "f32", "f32"),
    (4, 64, "packed", 192, 30, [1, 9], "bf16", "bf16", "bf16"),
    (4, 32, "packed", 128, 16, [1, 5], "f32", "f16", None),
    (8, 16, "packed", 64, 8, [4], "f16", "f32", None),
    (4, 32, "float", 256, 32, [1, 18], "f16", "f16", None),
    # too few output tiles for the GPU: K splits across workgroups, partial sums reduce
    (4, 128, "packed", 2048, 2048, [256, 300], "f16", "f16", None),
    (4, 128, "packed", 2048, 1000, [260], "f16", "f16", "f16"),
    (8, 64, "none", 1024, 520, [100], "f16", "f16", "f32"),
    # decode GEMVs with K not a multiple of a chunk (128 q4 / 64 q8 values): the last chunk's A
    # reads must stop at K, also for rows of A followed by other rows
    (4, 32, "packed", 200, 40, [1, 5, 16], "f16", "f16", None),
    (8, 32, "packed", 72, 24, [2, 9], "f16", "f16", None),
    (4, 16, "none", 1000, 56, [3, 12], "f16", "f16", None),
    (4, 32, "packed", 200, 40, [1, 3, 4], "f32", "f32", None),
    (8, 32, "none", 1000, 24, [2, 4], "f32", "f32", None),
    # 16 wavefronts with A staged through LDS (M > 4), partial sums in the wavefronts' A areas:
    # one round (16 chunks) and two rounds (24 chunks), 4- and 8-bit
    (4, 32, "packed", 2048, 48, [6, 16], "f16", "f16", None),
    (4, 32, "packed", 3072, 40, [8], "f16", "f16", None),
    (8, 32, "none", 1024, 40, [12], "f16", "f16", None),
    # block 256 over K = 104: the second chunk lies wholly past K
    (4, 256, "packed", 104, 40, [1, 5, 16], "f16", "f16", None),
    (4, 256, "none", 104, 24, [2], "f32", "f32", None),
    # K beyond one round of wavefronts: 86 and 128 chunks per row
    (4, 128, "packed", 11008, 64, [1, 20, 70], "f16", "f16", None),
    (8, 32, "packed", 8192, 24, [1, 33], "f16", "f16", "f16"),
    (2, 32, "packed", 4096, 40, [1, 9], "f16", "f16", None),
    # more tiles than the GPU holds wavefronts at once: 2 and 4 tiles per workgroup, last group partial
    (4, 32, "packed", 1024, 16400, [1, 16], "f16", "f16", None),
    (4, 32, "packed", 1024, 30008, [1, 7, 16], "f16", "f16", None),
    (8, 128, "none", 256, 50008, [1, 16], "f16", "f16", None),
    (4, 32, "packed", 4096, 12000, [1, 9], "f16", "f16", None),
    (4, 16, "packed", 512, 40000, [1, 5], "f16", "f16", None),
    # prefill tile shapes with a ragged last m-block: 256x256 tiles over 8-bit weights, and a
    # whole-GPU 256x256 grid over 4-bit weights
    (8, 32, "packed", 2048, 8192, [300], "f16", "f16", None),
    (4, 128, "packed", 4096, 8192, [2011], "f16", "f16", "f16"),
    # the bf16 prefill path (bf16 A and weights): K splits, a bias, 8-bit, K off a chunk
    (4, 128, "packed", 2048, 1000, [65, 260], "bf16", "bf16", "bf16"),
    (8, 64, "none", 1024, 520, [100, 300], "bf16", "bf16", None),
    (4, 32, "packed", 200, 40, [70], "bf16", "bf16", None),
    (2, 64, "packed", 512, 96, [100], "bf16", "bf16", None),
    # the split path (A and weights as bf16 hi + lo, three MFMAs): f32 A and weights, mixed types,
    # float zero points, 2- and 8-bit, K off a chunk, ragged M and N
    (4, 128, "packed", 2048, 2048, [256, 300], "f32", "f32", None),
    (4, 32, "none", 200, 40, [70, 129], "f32", "f32", "f32"),
    (4, 32, "float", 1024, 520, [100, 300], "f16", "f16", None),
    (4, 32, "packed", 1024, 96, [130], "f32", "f16", None),
    (4, 32, "packed", 1024, 96, [130], "bf16", "f32", None),
    (4, 32, "packed", 1024, 96, [130], "f16", "bf16", "f16"),
    (8, 32, "float", 512, 48, [66], "bf16", "bf16", None),
    (8, 128, "packed", 1024, 200, [300], "f32", "f32", None),
    (2, 64, "none", 512, 96, [100], "f32", "f32", None),
    # 2-bit weights on the LDS-tiled f16 GEMM (64- and 128-row tiles; 512-byte rows of A)
    (2, 32, "packed", 1024, 200, [80, 300], "f16", "f16", None),
    (2, 64, "none", 512, 96, [100, 257], "f16", "f16", "f16"),
]


@pytest.mark.parametrize("case", MATMUL_CASES, ids=lambda c: "b{}_bs{}_{}_K{}_N{}_{}_{}_{}".format(
    c[0], c[1], c[2], c[3], c[4], c[6], c[7], c[8]))
def test_matmul_matches_oracle(ctx, case):
    bits, bs, zp, k, n, ms, adt, sdt, bias_dt = case
    rng = np.random.default_rng(zlib.crc32(repr(case[:5]).encode()))
    b, s32, z = nbits_weight(rng, k, n, bits, bs, zp=zp, scale_dtype=np.float32)
    scales = host_float(s32, sdt)
    w = PackedWeight.upload(ctx, b, scales, z, k=k, n=n, bits=bits, block_size=bs, weight_dtype=sdt,
                            scales_dtype=sdt)
    bias = host_float(rng.standard_normal(n).astype(np.float32), bias_dt) if bias_dt else None
    for m in ms:
        print(f"matmul {case} M={m}", flush=True)
        a = host_float(rng.standard_normal((m, k)).astype(np.float32), adt)
        a_d = ctx.put(a, adt)
        bias_d = ctx.put(bias, bias_dt) if bias is not None else None
        y = matmul_nbits(a_d, w, bias_d)
        got = as_f64(y.numpy(), y.dtype)
        ref = o.matmul_nbits(a, b, as_f64(scales, sdt).astype(np.float32), z, bias, k=k, n=n, bits=bits,
                             block_size=bs, weight_dtype=sdt)
        ref_dtype = "bf16" if ref.dtype == np.uint16 else ("f16" if ref.dtype == np.float16 else "f32")
        assert y.dtype == ref_dtype
        err = rel_err(got, as_f64(ref, ref_dtype))
        assert err <= TOL[adt], f"M={m}: relative error {err}"
    w.free()


def test_matmul_f16_fast_path_is_near_exact(ctx):
    """The MFMA path sums exact f16 products in f32: against the f64 sum of the same f16
    weights its error is a few f16 output roundings, far inside the 1e-2 bar."""
    rng = np.random.default_rng(11)
    k, n, m = 3072, 256, 16
    b, s, z = nbits_weight(rng, k, n, 4, 32, zp="packed")
    w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=4, block_size=32, weight_dtype="f16")
    a = rng.standard_normal((m, k)).astype(np.float16)
    y = matmul_nbits(ctx.put(a), w).numpy().astype(np.float64)
    wf = o.dequantize_weight(b, s, z, k, n, 4, 32, o.F16).astype(np.float64)
    ref = a.astype(np.float64) @ wf.T
    assert np.abs(y - ref).max() <= 2 * np.abs(ref).max() * 2.0 ** -11


def test_matmul_zero_rows_is_a_no_op(ctx):
    rng = np.random.default_rng(12)
    b, s, z = nbits_weight(rng, 64, 16, 4, 32)
    w = PackedWeight.upload(ctx, b, s, z, k=64, n=16, bits=4, block_size=32, weight_dtype="f16")
    y = matmul_nbits(ctx.put(np.zeros((0, 64), np.float16)), w)
    assert y.shape == (0, 16)


def test_lda_ldy_strides(ctx):
    """Rows of A and Y with gaps (lda > K, ldy > N) through the C ABI."""
    import ctypes

    from transmuter_amd._lib import F16, lib

    rng = np.random.default_rng(13)
    k, n, m, lda, ldy = 200, 32, 5, 264, 40  # K past the last full chunk: A's padding must not count
    b, s, z = nbits_weight(rng, k, n, 4, 32)
    w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=4, block_size=32, weight_dtype="f16")
    a_full = rng.standard_normal((m, lda)).astype(np.float16)
    a_d = ctx.put(a_full)
    y_d = ctx.put(np.full((m, ldy), 7, np.float16))
    ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, a_d.ptr, F16, m, lda, None, 0, y_d.ptr, F16, ldy, None))
    y = y_d.numpy()
    ref = o.matmul_nbits(a_full[:, :k], b, s, z, k=k, n=n, bits=4, block_size=32)
    assert rel_err(y[:, :n].astype(np.float64), ref.astype(np.float64)) <= 1e-2
    assert np.all(y[:, n:] == 7)
    del ctypes


def test_y_type_must_follow_the_reference(ctx):
    from transmuter_amd._lib import F32, TmhArgumentError, lib

    rng = np.random.default_rng(14)
    b, s, z = nbits_weight(rng, 64, 16, 4, 32)
    w = PackedWeight.upload(ctx, b, s, z, k=64, n=16, bits=4, block_size=32, weight_dtype="f16")
    a_d = ctx.put(np.zeros((1, 64), np.float16))
    y_d = ctx.empty((1, 16), "f32")
    with pytest.raises(TmhArgumentError, match="Y must be f16"):
        ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, a_d.ptr, 10, 1, 64, None, 0, y_d.ptr, F32, 16, None))


# Every prefill tile shape (BM x 64*WN: 256x128, 256x256, 128x128, 128x256, 64x128, 64x256, and
# 128x128 and 64x128 with each k-block's steps split between two wavefronts), with and without K
# splits, forced through TMH_GEMM_PLAN, over ragged M, N and K (a partial last k-block) and a bias.
PLAN_CASES = [
    # bits, block, zp, K, N, M list, bias
    (4, 32, "packed", 1000, 1000, [200, 300], "f16"),
    (4, 128, "packed", 2048, 520, [129], None),
    (8, 64, "none", 768, 520, [130, 257], "f32"),
    (4, 16, "packed", 512, 300, [100], None),  # blocks of 16: parameters per MFMA step
]
# (bm, wn, splits[, 2]): a fourth field 2 splits each k-block's steps between two wavefronts
PLANS = [(256, 2, 1), (256, 4, 1), (128, 2, 1), (128, 4, 1), (256, 2, 3), (128, 2, 2), (128, 4, 4), (128, 2, 1, 2),
         (128, 2, 3, 2), (64, 2, 1), (64, 4, 1), (64, 2, 3), (64, 4, 2), (64, 2, 1, 2), (64, 2, 2, 2)]


@pytest.mark.parametrize("plan", PLANS, ids=lambda p: "bm{}_wn{}_s{}".format(*p) + ("_ks2" if len(p) > 3 else ""))
@pytest.mark.parametrize("case", PLAN_CASES, ids=lambda c: "b{}_bs{}_{}_K{}_N{}".format(*c[:5]))
def test_matmul_every_gemm_plan(ctx, monkeypatch, case, plan):
    bits, bs, zp, k, n, ms, bias_dt = case
    monkeypatch.setenv("TMH_GEMM_PLAN", ",".join(map(str, plan)))
    rng = np.random.default_rng(zlib.crc32(repr(case[:5]).encode()))
    b, s32, z = nbits_weight(rng, k, n, bits, bs, zp=zp, scale_dtype=np.float32)
    scales = s32.astype(np.float16)
    w = PackedWeight.upload(ctx, b, scales, z, k=k, n=n, bits=bits, block_size=bs, weight_dtype="f16",
                            scales_dtype="f16")
    bias = host_float(rng.standard_normal(n).astype(np.float32), bias_dt) if bias_dt else None
    for m in ms:
        print(f"matmul plan {plan} {case} M={m}", flush=True)
        a = rng.standard_normal((m, k)).astype(np.float16)
        y = matmul_nbits(ctx.put(a), w, ctx.put(bias, bias_dt) if bias is not None else None)
        got = as_f64(y.numpy(), y.dtype)
        ref = o.matmul_nbits(a, b, scales.astype(np.float32), z, bias, k=k, n=n, bits=bits, block_size=bs,
                             weight_dtype="f16")
        err = rel_err(got, np.asarray(ref, np.float64))
        assert err <= TOL["f16"], f"M={m}: relative error {err}"
    w.free()


# The bf16 and split prefill paths run the 128x128 and 64x128 tiles on eight wavefronts, and 2-bit
# weights the 64- and 128-row f16 tiles: each forced, with and without K splits, over ragged M, N, K.
MODE_PLAN_CASES = [
    # bits, block, zp, K, N, M, A type, weight type, bias
    (4, 32, "packed", 1000, 1000, 200, "bf16", "bf16", "bf16"),
    (8, 64, "none", 768, 520, 130, "bf16", "bf16", None),
    (4, 32, "packed", 1000, 1000, 200, "f32", "f32", "f32"),
    (4, 64, "float", 768, 300, 257, "f32", "f16", None),
    (8, 32, "packed", 512, 300, 100, "f16", "bf16", None),
    (2, 64, "packed", 1024, 300, 150, "f16", "f16", None),
    (2, 16, "none", 512, 200, 100, "f16", "f16", "f16"),
]
MODE_PLANS = [(128, 2, 1, 2), (128, 2, 3, 2), (64, 2, 1, 2), (64, 2, 2, 2), (128, 4, 2), (64, 4, 1)]


@pytest.mark.parametrize("plan", MODE_PLANS, ids=lambda p: "bm{}_wn{}_s{}".format(*p) + ("_ks2" if len(p) > 3 else ""))
@pytest.mark.parametrize("case", MODE_PLAN_CASES, ids=lambda c: "b{}_bs{}_{}_K{}_N{}_M{}_{}_{}".format(*c[:8]))
def test_matmul_float_and_2bit_gemm_plans(ctx, monkeypatch, case, plan):
    bits, bs, zp, k, n, m, adt, wdt, bias_dt = case
    monkeypatch.setenv("TMH_GEMM_PLAN", ",".join(map(str, plan)))
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    b, s32, z = nbits_weight(rng, k, n, bits, bs, zp=zp, scale_dtype=np.float32)
    scales = host_float(s32, wdt)
    w = PackedWeight.upload(ctx, b, scales, z, k=k, n=n, bits=bits, block_size=bs, weight_dtype=wdt, scales_dtype=wdt)
    bias = host_float(rng.standard_normal(n).astype(np.float32), bias_dt) if bias_dt else None
    print(f"matmul mode plan {plan} {case}", flush=True)
    a = host_float(rng.standard_normal((m, k)).astype(np.float32), adt)
    y = matmul_nbits(ctx.put(a, adt), w, ctx.put(bias, bias_dt) if bias is not None else None)
    ref = o.matmul_nbits(a, b, as_f64(scales, wdt).astype(np.float32), z, bias, k=k, n=n, bits=bits, block_size=bs,
                         weight_dtype=wdt)
    ref_dtype = "bf16" if ref.dtype == np.uint16 else ("f16" if ref.dtype == np.float16 else "f32")
    assert y.dtype == ref_dtype
    err = rel_err(as_f64(y.numpy(), y.dtype), as_f64(ref, ref_dtype))
    assert err <= TOL[adt], f"relative error {err}"
    w.free()


# One row of A (decode at M = 1) over a streaming grid goes to the dot-product GEMV (4- and 8-bit
# weights with one parameter entry per lane) or, forced with TMH_GEMV_PLAN=mfma, to the MFMA GEMV;
# resident grids take the MFMA GEMV either way. Both against the oracle, over resident and
# streaming grids, ragged K, a chunk wholly past K, many chunk rounds and rows of A with padding
# (lda > K).
ONE_ROW_CASES = [
    # bits, block, zp, K, N, lda
    (4, 32, "packed", 1024, 96, 1024),
    (4, 32, "none", 200, 40, 264),
    (4, 128, "packed", 2048, 64, 2048),
    (4, 256, "packed", 104, 40, 112),
    (4, 64, "packed", 11008, 48, 11008),
    (4, 32, "packed", 1024, 30008, 1024),
    (4, 32, "none", 2000, 16000, 2008),
    (4, 128, "packed", 4096, 12000, 4096),
    (4, 32, "packed", 1024, 40008, 1024),  # thousands of tiles: four per workgroup, a ragged last one
    (8, 32, "packed", 512, 48, 512),
    (8, 128, "none", 1000, 20, 1000),
    (8, 32, "none", 72, 24, 80),
    (8, 128, "none", 256, 50008, 256),
    (4, 16, "packed", 256, 40, 256),  # a lane's values span two blocks: MFMA kernel either way
    (2, 16, "packed", 256, 24, 256),
]


@pytest.mark.parametrize("plan", ["dot", "mfma"])
@pytest.mark.parametrize("case", ONE_ROW_CASES, ids=lambda c: "b{}_bs{}_{}_K{}_N{}_lda{}".format(*c))
def test_one_row_both_kernels(ctx, monkeypatch, case, plan):
    import ctypes

    from transmuter_amd._lib import F16, lib

    bits, bs, zp, k, n, lda = case
    if plan == "mfma":
        monkeypatch.setenv("TMH_GEMV_PLAN", "mfma")
    else:
        monkeypatch.delenv("TMH_GEMV_PLAN", raising=False)
    print(f"one row {plan} {case}", flush=True)
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    b, s, z = nbits_weight(rng, k, n, bits, bs, zp=zp)
    w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=bits, block_size=bs, weight_dtype="f16")
    a_full = rng.standard_normal((1, lda)).astype(np.float16)
    y_d = ctx.empty((1, n), "f16")
    ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, ctx.put(a_full).ptr, F16, 1, lda, None, 0, y_d.ptr, F16, n,
                                     None))
    ref = o.matmul_nbits(a_full[:, :k], b, s, z, k=k, n=n, bits=bits, block_size=bs).astype(np.float64)
    err = rel_err(y_d.numpy().astype(np.float64), ref)
    assert err <= TOL["f16"], f"relative error {err}"
    w.free()
    del ctypes


# Decode with an f16 bias (Y = the f16 dot + bias, rounded to f16: quantized.ex:44-45) on the
# decode GEMVs: one-shot grids with A direct (M <= 4) and through LDS (M > 4), K past one round of
# wavefronts, streaming grids of two and four tiles per workgroup, a ragged last tile whose last
# columns store one at a time, and parameters that span two blocks per lane; M = 1 on both the
# dot-product and the MFMA kernel.
BIAS_DECODE_CASES = [
    # bits, block, zp, K, N, M list
    (4, 32, "packed", 1024, 96, [1, 3, 4, 6, 16]),
    (4, 32, "packed", 3072, 40, [1, 8]),
    (4, 32, "packed", 1024, 30008, [1, 7, 16]),
    (4, 32, "packed", 1024, 16400, [1, 2]),
    (8, 32, "none", 512, 42, [1, 3, 9]),
    (4, 16, "packed", 256, 40, [1, 5]),
]


@pytest.mark.parametrize("plan", ["dot", "mfma"])
@pytest.mark.parametrize("case", BIAS_DECODE_CASES, ids=lambda c: "b{}_bs{}_{}_K{}_N{}".format(*c[:5]))
def test_decode_gemv_with_bias(ctx, monkeypatch, case, plan):
    """Against the oracle, and bit for bit against the same kernel's output without the bias with
    the bias then added on the host in f32 and rounded to f16."""
    bits, bs, zp, k, n, ms = case
    if plan == "mfma":
        monkeypatch.setenv("TMH_GEMV_PLAN", "mfma")
    else:
        monkeypatch.delenv("TMH_GEMV_PLAN", raising=False)
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()) + 3)
    b, s, z = nbits_weight(rng, k, n, bits, bs, zp=zp)
    w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=bits, block_size=bs, weight_dtype="f16")
    bias = rng.standard_normal(n).astype(np.float16)
    bias_d = ctx.put(bias)
    for m in ms:
        print(f"decode bias {plan} {case} M={m}", flush=True)
        a = rng.standard_normal((m, k)).astype(np.float16)
        a_d = ctx.put(a)
        y = matmul_nbits(a_d, w, bias_d).numpy()
        y0 = matmul_nbits(a_d, w).numpy()
        assert np.array_equal(y.view(np.uint16), (y0.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
                              .view(np.uint16)), f"M={m}"
        ref = o.matmul_nbits(a, b, s, z, bias, k=k, n=n, bits=bits, block_size=bs).astype(np.float64)
        err = rel_err(y.astype(np.float64), ref)
        assert err <= TOL["f16"], f"M={m}: relative error {err}"
    w.free()


def test_one_row_dot_kernel_is_near_exact(ctx, monkeypatch):
    """The dot-product GEMV (one row of A over more tiles than the GPU holds at once) sums exact
    products (q + 1024) * a in f32 and removes the offsets per lane: against the f64 sum over the
    exact weights (q - zero) * scale its error is about one f16 output rounding."""
    monkeypatch.delenv("TMH_GEMV_PLAN", raising=False)
    rng = np.random.default_rng(15)
    k, n = 1024, 12800
    b, s, z = nbits_weight(rng, k, n, 4, 32, zp="packed")
    w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=4, block_size=32, weight_dtype="f16")
    a = rng.standard_normal((1, k)).astype(np.float16)
    y = matmul_nbits(ctx.put(a), w).numpy().astype(np.float64)
    q = o.unpack(b.reshape(n, -1), 4)[:, :k].astype(np.float64)
    zq = o.unpack(z.reshape(n, -1), 4)[:, : k // 32].astype(np.float64)
    wx = (q - np.repeat(zq, 32, axis=1)) * np.repeat(s.reshape(n, -1).astype(np.float64), 32, axis=1)
    ref = a.astype(np.float64) @ wx.T
    assert np.abs(y - ref).max() <= 2 * np.abs(ref).max() * 2.0 ** -11
