"""The C restatement (oracle/oracle.c) against the numpy oracle and the reference fixtures."""

import numpy as np
import pytest

from fixtures import Fixture, names
from oracle import coracle
from oracle import oracle as o
from synth import nbits_weight


def test_f16_conversion_matches_numpy_everywhere():
    """Every f16 value and the midpoints between neighbours (ties to even), plus extremes."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    finite = h[np.isfinite(h)].astype(np.float32)
    assert np.array_equal(coracle.f32_to_f16(finite).view(np.uint16), finite.astype(np.float16).view(np.uint16))
    pos = np.sort(np.unique(np.abs(finite)))
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    assert np.array_equal(coracle.f32_to_f16(mids).view(np.uint16), mids.astype(np.float16).view(np.uint16))
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(100000) * np.exp(rng.uniform(-20, 12, 100000))).astype(np.float32)
    x = np.concatenate([x, [65504, 65519.9, 65520, 1e9, -1e9, 1e-9, 5.96e-8, 2.98e-8, 2.9802322e-08]]).astype(np.float32)
    assert np.array_equal(coracle.f32_to_f16(x).view(np.uint16), x.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("bits,bs,zp,k", [(4, 32, "packed", 1024), (4, 32, "none", 72), (8, 16, "float", 64),
                                          (2, 64, "packed", 320)])
@pytest.mark.parametrize("out_f16", [False, True])
def test_dequantize_matches_numpy_oracle(bits, bs, zp, k, out_f16):
    rng = np.random.default_rng(bits + k)
    n = 12
    b, s, z = nbits_weight(rng, k, n, bits, bs, zp=zp, scale_dtype=np.float32)
    got = coracle.dequantize_nbits(b, s, z, k, n, bits, bs, out_f16=out_f16)
    ref = o.dequantize_weight(b, s, z, k, n, bits, bs, o.F16 if out_f16 else o.F32)
    assert np.array_equal(got.view(np.uint8), ref.view(np.uint8))


@pytest.mark.parametrize("threads", [1, 3])
def test_gemm_matches_f64(threads):
    rng = np.random.default_rng(threads)
    a = rng.standard_normal((3, 300)).astype(np.float32)
    w = rng.standard_normal((37, 300)).astype(np.float32)
    ref = a.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(coracle.gemm(a, w, threads) - ref).max() < 1e-4
    assert np.abs(coracle.gemm(a, w.astype(np.float16), threads)
                  - a.astype(np.float64) @ w.astype(np.float16).astype(np.float64).T).max() < 1e-4


@pytest.mark.parametrize("name", [n for n in names("MatMulInteger") if n != "MatMulInteger_dynamic_quant"])
def test_matmul_integer_fixture(name):
    f = Fixture(name)
    a, b, az, bz = f.node_inputs()
    assert np.array_equal(coracle.matmul_integer(a, b, az, bz), f.outputs["y"])


def test_matmul_nbits_fixture_through_c():
    f = Fixture("MatMulNBits_b4_bs256_packed")
    A, B, S, Z = f.node_inputs()
    w = coracle.dequantize_nbits(B, S, Z, 512, 40, 4, 256)
    y = coracle.gemm(A.reshape(-1, 512), w, 2).reshape(2, 3, 40)
    expected = f.outputs["Y"]
    assert np.abs(y - expected).max() <= 1e-4 + 1e-3 * np.abs(expected).max()


@pytest.mark.parametrize("f16,zp,threads", [(True, True, 1), (True, False, 3), (False, True, 2)])
def test_in_graph_matmul_matches_the_numpy_oracle(f16, zp, threads):
    """oracle_matmul_nbits_in_graph (dequantize on every call, then the dot) against
    oracle.matmul_nbits with W in the activations' type."""
    rng = np.random.default_rng(int(f16) * 4 + int(zp) * 2 + threads)
    k, n, m = 200, 37, 3
    b, s, z = nbits_weight(rng, k, n, 4, 32, zp="packed" if zp else "none")
    a = rng.standard_normal((m, k)).astype(np.float16 if f16 else np.float32)
    got = coracle.matmul_nbits_in_graph(a.astype(np.float32), b, s.astype(np.float32), z, k, n, 4, 32, f16, threads)
    want = o.matmul_nbits(a, b, s.astype(np.float16 if f16 else np.float32), z, k=k, n=n, bits=4,
                          block_size=32).astype(np.float64)
    assert np.abs(got - want).max() <= (1e-2 if f16 else 1e-4) * np.abs(want).max()
