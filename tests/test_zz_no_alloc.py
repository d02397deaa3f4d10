"""tmh_matmul_nbits_noalloc, the MatMulNBits entry point that allocates nothing: its split-K
partial sums live in a fixed per-device scratch area. Called through the C ABI, it must give the
bits of tmh_matmul_nbits on the same inputs: on two calls in a row, the second smaller, on a
decode GEMV (no scratch), in a graph captured on a fresh context (whose own workspace is empty),
and where tmh_matmul_nbits's plan keeps more partial sums than the scratch holds it must run a
plan that fits."""

import ctypes

import numpy as np
import pytest

from synth import nbits_weight
from transmuter_amd import Context, PackedWeight
from transmuter_amd._lib import F16, lib

pytestmark = pytest.mark.gpu

def _call(fn, ctx, w, a, m, y):
    return fn(ctx.handle, w.handle, a.ptr, F16, m, w.k, None, 0, y.ptr, F16, w.n, None)


def _pair(ctx, w, a, m):
    """The outputs of tmh_matmul_nbits and of tmh_matmul_nbits_noalloc on the same inputs."""
    y_ref, y = ctx.empty((m, w.n), "f16"), ctx.empty((m, w.n), "f16")
    ctx.check(_call(lib().tmh_matmul_nbits, ctx, w, a, m, y_ref))
    ctx.check(_call(lib().tmh_matmul_nbits_noalloc, ctx, w, a, m, y))
    ctx.synchronize()
    return y_ref.numpy(), y.numpy()


def test_noalloc_matches_matmul_nbits_on_two_calls_the_second_smaller(monkeypatch):
    monkeypatch.delenv("TMH_GEMM_PLAN", raising=False)
    ctx = Context(0)
    try:
        rng = np.random.default_rng(31)
        cases = [(2048, 2048, 256), (2048, 2048, 100)]  # splits K (8 MiB, then 3 MiB of partial sums)
        k, n = 2048, 2048
        w = PackedWeight.upload(ctx, *nbits_weight(rng, k, n, 4, 128), k=k, n=n, bits=4, block_size=128,
                                weight_dtype="f16")
        for _k, _n, m in cases:
            print(f"noalloc M={m} K={k} N={n}", flush=True)
            a = ctx.put(rng.standard_normal((m, k)).astype(np.float16))
            want, got = _pair(ctx, w, a, m)
            assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), m
        w1 = PackedWeight.upload(ctx, *nbits_weight(rng, 1024, 3072, 4, 32), k=1024, n=3072, bits=4, block_size=32,
                                 weight_dtype="f16")
        a1 = ctx.put(rng.standard_normal((1, 1024)).astype(np.float16))
        print("noalloc decode M=1 K=1024 N=3072", flush=True)
        want, got = _pair(ctx, w1, a1, 1)
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    finally:
        ctx.synchronize()
        ctx.close()


def test_noalloc_in_a_graph_on_a_fresh_context(monkeypatch):
    """A fresh context has no workspace, so tmh_matmul_nbits cannot split K during capture;
    the no-alloc variant can. Its replays equal the eager calls of tmh_matmul_nbits."""
    monkeypatch.delenv("TMH_GEMM_PLAN", raising=False)
    ctx = Context(0)
    try:
        rng = np.random.default_rng(32)
        k, n = 3072, 1024
        w = PackedWeight.upload(ctx, *nbits_weight(rng, k, n, 4, 128), k=k, n=n, bits=4, block_size=128,
                                weight_dtype="f16")
        m_big, m_small = 512, 200
        a_big = ctx.put(rng.standard_normal((m_big, k)).astype(np.float16))
        a_small = ctx.put(rng.standard_normal((m_small, k)).astype(np.float16))
        y_big, y_small = ctx.empty((m_big, n), "f16"), ctx.empty((m_small, n), "f16")
        print(f"noalloc graph M={m_big},{m_small} K={k} N={n}", flush=True)
        ctx.check(lib().tmh_graph_begin(ctx.handle, None))
        ctx.check(_call(lib().tmh_matmul_nbits_noalloc, ctx, w, a_big, m_big, y_big))
        ctx.check(_call(lib().tmh_matmul_nbits_noalloc, ctx, w, a_small, m_small, y_small))
        graph = ctypes.c_void_p()
        ctx.check(lib().tmh_graph_end(ctx.handle, None, ctypes.byref(graph)))
        replays = []
        for _ in range(3):
            for y in (y_big, y_small):
                ctx.check(lib().tmh_upload(ctx.handle, y.ptr, np.full(y.size, 7, np.uint16).ctypes.data_as(
                    ctypes.c_void_p), y.nbytes))
            ctx.check(lib().tmh_graph_launch(ctx.handle, graph, None))
            ctx.synchronize()
            replays.append((y_big.numpy(), y_small.numpy()))
        ctx.check(lib().tmh_graph_destroy(ctx.handle, graph))
        want_big, _ = _pair(ctx, w, a_big, m_big)
        want_small, _ = _pair(ctx, w, a_small, m_small)
        for got_big, got_small in replays:
            assert np.array_equal(got_big.view(np.uint16), want_big.view(np.uint16))
            assert np.array_equal(got_small.view(np.uint16), want_small.view(np.uint16))
    finally:
        ctx.synchronize()
        ctx.close()


def test_noalloc_replans_partial_sums_beyond_its_scratch(monkeypatch):
    """Where tmh_matmul_nbits's plan keeps more than 64 MiB of partial sums (11008 -> 2048 at
    M=4096: four K splits, 128 MiB; a forced 16-way split at M=2048: 256 MiB), the no-alloc call
    runs a plan that fits and gives the same sums up to f32 summation order, on two calls in a
    row, the second smaller."""
    ctx = Context(0)
    try:
        rng = np.random.default_rng(33)
        k, n = 11008, 2048
        w = PackedWeight.upload(ctx, *nbits_weight(rng, k, n, 4, 128), k=k, n=n, bits=4, block_size=128,
                                weight_dtype="f16")
        for plan, m in ((None, 4096), ("128,2,16", 2048)):
            if plan:
                monkeypatch.setenv("TMH_GEMM_PLAN", plan)
            else:
                monkeypatch.delenv("TMH_GEMM_PLAN", raising=False)
            print(f"noalloc re-plans M={m} K={k} N={n} plan={plan}", flush=True)
            a = ctx.put(rng.standard_normal((m, k)).astype(np.float16))
            want, got = _pair(ctx, w, a, m)
            want, got = want.astype(np.float64), got.astype(np.float64)
            assert np.isfinite(got).all()
            err = np.abs(got - want).max() / np.abs(want).max()
            assert err <= 2e-3, (m, plan, err)
            a.free()
    finally:
        ctx.synchronize()
        ctx.close()
