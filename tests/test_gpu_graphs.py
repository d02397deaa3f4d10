"""HIP graph capture of the library's calls: every compute call is capture-safe (no
allocation, no memset). A graph is replayed several times with the program's own eager work
and synchronisations between replays, and every replay must equal the eager result."""

import ctypes

import numpy as np
import pytest

from synth import nbits_weight, pack
from transmuter_amd import Context, PackedWeight
from transmuter_amd._lib import F16, S64, U8, lib

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager():
    ctx = Context(0)  # a fresh context: its split-K workspace is empty when capture starts
    try:
        rng = np.random.default_rng(21)
        k, n = 2048, 2048
        b, s, z = nbits_weight(rng, k, n, 4, 128)
        w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=4, block_size=128, weight_dtype="f16")
        w1 = PackedWeight.upload(ctx, *nbits_weight(rng, 1024, 3072, 4, 32), k=1024, n=3072, bits=4, block_size=32,
                                 weight_dtype="f16")
        a = ctx.put(rng.standard_normal((256, k)).astype(np.float16))
        a1 = ctx.put(rng.standard_normal((1, 1024)).astype(np.float16))
        table = pack(rng.integers(0, 16, (500, 64)), 4)
        scales = (rng.random((500, 2)) * 0.1).astype(np.float16)
        zps = pack(rng.integers(0, 16, (500, 2)), 4)
        t_d, s_d, z_d = ctx.put(table), ctx.put(scales), ctx.put(zps)
        ids = ctx.put(rng.integers(0, 500, (64,)).astype(np.int64))
        y, y1, g = ctx.empty((256, n), "f16"), ctx.empty((1, 3072), "f16"), ctx.empty((64, 64), "f16")

        def calls():
            ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, a.ptr, F16, 256, k, None, 0, y.ptr, F16, n, None))
            ctx.check(lib().tmh_matmul_nbits(ctx.handle, w1.handle, a1.ptr, F16, 1, 1024, None, 0, y1.ptr, F16, 3072,
                                             None))
            ctx.check(lib().tmh_gather_block_quantized(ctx.handle, t_d.ptr, U8, 500, 32, ids.ptr, S64, 64, s_d.ptr,
                                                       F16, 2, z_d.ptr, U8, 4, g.ptr, None))

        ctx.check(lib().tmh_graph_begin(ctx.handle, None))
        calls()
        graph = ctypes.c_void_p()
        ctx.check(lib().tmh_graph_end(ctx.handle, None, ctypes.byref(graph)))
        outs = []
        for _ in range(3):
            for t in (y, y1, g):  # scribble between replays
                ctx.check(lib().tmh_upload(ctx.handle, t.ptr, np.full(t.size, 7, np.uint16).ctypes.data_as(
                    ctypes.c_void_p), t.nbytes))
            ctx.check(lib().tmh_graph_launch(ctx.handle, graph, None))
            ctx.synchronize()
            outs.append([t.numpy() for t in (y, y1, g)])
        calls()  # eager, now with a workspace for split K
        eager = [t.numpy() for t in (y, y1, g)]
        for replay in outs:
            for got, want in zip(replay, eager):
                # the graph ran the unsplit path (no workspace during capture): same values within f16
                assert np.allclose(got.astype(np.float32), want.astype(np.float32), rtol=2e-3, atol=2e-3)
        assert np.array_equal(outs[0][1], eager[1]) and np.array_equal(outs[0][2], eager[2])
        ctx.check(lib().tmh_graph_destroy(ctx.handle, graph))
    finally:
        ctx.synchronize()
        ctx.close()


def test_split_k_repeated_calls_and_replays_are_bit_exact(monkeypatch):
    """Split-K GEMMs share the context's workspace of partial sums. Repeated eager calls,
    several splits of one weight in one graph, and replays interleaved with eager calls must all
    give the first call's bits."""
    ctx = Context(0)
    try:
        rng = np.random.default_rng(22)
        k, n, m = 2048, 1000, 300
        b, s, z = nbits_weight(rng, k, n, 4, 128)
        w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=4, block_size=128, weight_dtype="f16")
        a = ctx.put(rng.standard_normal((m, k)).astype(np.float16))
        ys = [ctx.empty((m, n), "f16") for _ in range(3)]
        plans = ["128,2,4", "256,4,3", "128,4,2"]

        def call(i):
            monkeypatch.setenv("TMH_GEMM_PLAN", plans[i])
            ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, a.ptr, F16, m, k, None, 0, ys[i].ptr, F16, n, None))

        for i in range(3):  # eager first: sizes the workspace for the largest split
            call(i)
        ctx.synchronize()
        first = [y.numpy() for y in ys]
        for _ in range(2):
            for i in range(3):
                call(i)
            ctx.synchronize()
            for y, want in zip(ys, first):
                assert np.array_equal(y.numpy(), want)
        ctx.check(lib().tmh_graph_begin(ctx.handle, None))
        for i in (0, 1, 2, 0):
            call(i)
        graph = ctypes.c_void_p()
        ctx.check(lib().tmh_graph_end(ctx.handle, None, ctypes.byref(graph)))
        for _ in range(3):
            for y in ys:
                ctx.check(lib().tmh_upload(ctx.handle, y.ptr, np.full(y.size, 7, np.uint16).ctypes.data_as(
                    ctypes.c_void_p), y.nbytes))
            ctx.check(lib().tmh_graph_launch(ctx.handle, graph, None))
            ctx.synchronize()
            for y, want in zip(ys, first):
                assert np.array_equal(y.numpy(), want)
            call(1)  # eager work on the same workspace between replays
            ctx.synchronize()
            assert np.array_equal(ys[1].numpy(), first[1])
        ctx.check(lib().tmh_graph_destroy(ctx.handle, graph))
    finally:
        ctx.synchronize()
        ctx.close()
