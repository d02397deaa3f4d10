"""Seeded random MatMulNBits configurations on the GPU against the oracle: bits 2/4/8, block
sizes 16-256, zero points none/packed/float, f16/f32/bf16 activations, ragged K and N, with
and without bias, and M spread over the decode GEMV, small-M and prefill GEMM paths (24 of the
64 seeds draw the f16 prefill GEMM: tile shapes, split K, ragged last m-blocks and K past the
last whole chunk). Tolerances as in test_gpu_nbits.py. Each case prints its parameters before
it runs."""

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


def draw(seed):
    """Seeds below 40 spread over every path; seeds from 40 on draw the f16 prefill GEMM (4- and
    8-bit weights, M > 64)."""
    rng = np.random.default_rng(seed)
    prefill = seed >= 40
    bits = int(rng.choice([4, 8] if prefill else [2, 4, 4, 4, 8, 8]))
    bs = int(rng.choice([16, 32, 64, 128, 256]))
    k = int(rng.choice([bs * int(rng.integers(1, 24)), 8 * int(rng.integers(2, 300))]))
    n = int(rng.integers(1, 3000))
    if prefill:
        m = int(rng.integers(65, 1100))
    else:
        m = int(rng.choice([1, int(rng.integers(2, 17)), int(rng.integers(17, 65)), int(rng.integers(65, 700))]))
    zp = str(rng.choice(["none", "packed"] if prefill else ["none", "packed", "float"]))
    adt = "f16" if prefill else str(rng.choice(["f16", "f16", "f32", "bf16"]))
    bias = bool(rng.random() < 0.3)
    return bits, bs, k, n, m, zp, adt, bias


@pytest.mark.parametrize("seed", range(64))
def test_random_matmul(ctx, seed):
    bits, bs, k, n, m, zp, adt, with_bias = draw(seed)
    print(f"random seed={seed} bits={bits} block={bs} K={k} N={n} M={m} zp={zp} A={adt} bias={with_bias}",
          flush=True)
    rng = np.random.default_rng(1000 + seed)
    b, s32, z = nbits_weight(rng, k, n, bits, bs, zp=zp, scale_dtype=np.float32)
    sdt = adt
    scales = host_float(s32, sdt)
    w = PackedWeight.upload(ctx, b, scales, z, k=k, n=n, bits=bits, block_size=bs, weight_dtype=sdt,
                            scales_dtype=sdt)
    try:
        bias = host_float(rng.standard_normal(n).astype(np.float32), adt) if with_bias else None
        a = host_float(rng.standard_normal((m, k)).astype(np.float32), adt)
        y = matmul_nbits(ctx.put(a, adt), w, ctx.put(bias, adt) if bias is not None else None)
        got = as_f64(y.numpy(), y.dtype)
    finally:
        w.free()
    ref = o.matmul_nbits(a, b, as_f64(scales, sdt).astype(np.float32), z, bias, k=k, n=n, bits=bits,
                         block_size=bs, weight_dtype=sdt)
    ref_dtype = "bf16" if ref.dtype == np.uint16 else ("f16" if ref.dtype == np.float16 else "f32")
    assert y.dtype == ref_dtype
    err = float(np.abs(got - as_f64(ref, ref_dtype)).max() / max(np.abs(as_f64(ref, ref_dtype)).max(), 1e-30))
    assert err <= TOL[adt], f"seed {seed}: relative error {err}"
