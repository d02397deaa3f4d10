"""HIP graph capture of the library's calls: every compute call is capture-safe (no
allocation, no memset). A graph is replayed several times with the program's own eager work
and synchronisations between replays, and every replay must equal the eager result."""

import ctypes

import numpy as np
import pytest

from synth import nbits_weight, pack
from transmuter_amd import Context, PackedWeight
from transmuter_amd._lib import ERR_UNSUPPORTED, F16, S64, U8, lib

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

        def split_k_call():
            return lib().tmh_matmul_nbits(ctx.handle, w.handle, a.ptr, F16, 256, k, None, 0, y.ptr, F16, n, None)

        def calls():
            ctx.check(split_k_call())
            ctx.check(lib().tmh_matmul_nbits(ctx.handle, w1.handle, a1.ptr, F16, 1, 1024, None, 0, y1.ptr, F16, 3072,
                                             None))
            ctx.check(lib().tmh_gather_block_quantized(ctx.handle, t_d.ptr, U8, 500, 32, ids.ptr, S64, 64, s_d.ptr,
                                                       F16, 2, z_d.ptr, U8, 4, g.ptr, None))

        # A split-K call cannot grow the workspace while the stream is captured: it fails with a
        # message (it never runs unsplit instead, which would give other bits than eager calls).
        ctx.check(lib().tmh_graph_begin(ctx.handle, None))
        status = split_k_call()
        message = lib().tmh_last_error(ctx.handle).decode()
        graph = ctypes.c_void_p()
        ctx.check(lib().tmh_graph_end(ctx.handle, None, ctypes.byref(graph)))
        ctx.check(lib().tmh_graph_destroy(ctx.handle, graph))
        assert status == ERR_UNSUPPORTED and "workspace" in message and "capture" in message, message
        calls()  # eager: sizes the workspace
        ctx.synchronize()
        eager = [t.numpy() for t in (y, y1, g)]
        ctx.check(lib().tmh_graph_begin(ctx.handle, None))
        calls()
        ctx.check(lib().tmh_graph_end(ctx.handle, None, ctypes.byref(graph)))
        for _ in range(3):
            for t in (y, y1, g):  # scribble between replays
                ctx.check(lib().tmh_upload(ctx.handle, t.ptr, np.full(t.size, 7, np.uint16).ctypes.data_as(
                    ctypes.c_void_p), t.nbytes))
            ctx.check(lib().tmh_graph_launch(ctx.handle, graph, None))
            ctx.synchronize()
            for t, want in zip((y, y1, g), eager):
                assert np.array_equal(t.numpy(), want)
        ctx.check(lib().tmh_graph_destroy(ctx.handle, graph))
    finally:
        ctx.synchronize()
        ctx.close()


def test_replays_survive_a_workspace_that_grows_later(monkeypatch):
    """A graph keeps the workspace addresses of its capture. A later, larger eager call grows
    the workspace; the old one stays allocated (until the context ends), so the graph's replays
    still give their bits. Covers split-K partial sums and the QMoE intermediates."""
    from transmuter_amd._lib import F32
    from transmuter_amd.moe import ExpertWeight

    ctx = Context(0)
    try:
        rng = np.random.default_rng(23)
        k, n = 2048, 1000
        w = PackedWeight.upload(ctx, *nbits_weight(rng, k, n, 4, 128), k=k, n=n, bits=4, block_size=128,
                                weight_dtype="f16")
        a_small = ctx.put(rng.standard_normal((300, k)).astype(np.float16))
        a_big = ctx.put(rng.standard_normal((600, k)).astype(np.float16))
        y_small, y_big = ctx.empty((300, n), "f16"), ctx.empty((600, n), "f16")
        e, h, inter = 16, 64, 32
        fc1 = ExpertWeight.upload(ctx, rng.integers(0, 256, (e, inter, h // 2), dtype=np.uint8),
                                  (rng.random((e, inter, h // 32)) * 0.05 + 1e-3).astype(np.float16), None, bits=4,
                                  block_size=32, dtype="f16")
        fc2 = ExpertWeight.upload(ctx, rng.integers(0, 256, (e, h, inter // 2), dtype=np.uint8),
                                  (rng.random((e, h, 1)) * 0.05 + 1e-3).astype(np.float16), None, bits=4,
                                  block_size=32, dtype="f16")
        x_small = ctx.put(rng.standard_normal((8, h)).astype(np.float16))
        x_big = ctx.put(rng.standard_normal((4000, h)).astype(np.float16))
        r_small = ctx.put(rng.standard_normal((8, e)).astype(np.float32))
        r_big = ctx.put(rng.standard_normal((4000, e)).astype(np.float32))
        y_moe, y_moe_big = ctx.empty((8, h), "f16"), ctx.empty((4000, h), "f16")

        def qmoe(x, r, y, t):  # top-2 of 16 experts, silu
            ctx.check(lib().tmh_qmoe(ctx.handle, x.ptr, F16, t, h, r.ptr, F32, e, 2, fc1.handle, None, fc2.handle,
                                     None, None, None, F16, 2, 0, 1.0, 0.0, 0.0, y.ptr, None))

        def small():
            monkeypatch.setenv("TMH_GEMM_PLAN", "128,2,2")
            ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, a_small.ptr, F16, 300, k, None, 0, y_small.ptr,
                                             F16, n, None))
            qmoe(x_small, r_small, y_moe, 8)

        small()  # eager: sizes the workspace for the small calls
        ctx.synchronize()
        want = [y_small.numpy(), y_moe.numpy()]
        ctx.check(lib().tmh_graph_begin(ctx.handle, None))
        small()
        graph = ctypes.c_void_p()
        ctx.check(lib().tmh_graph_end(ctx.handle, None, ctypes.byref(graph)))
        for round_ in range(3):
            if round_ == 1:  # larger eager calls grow the workspace after the capture
                monkeypatch.setenv("TMH_GEMM_PLAN", "128,2,8")
                ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, a_big.ptr, F16, 600, k, None, 0, y_big.ptr,
                                                 F16, n, None))
                qmoe(x_big, r_big, y_moe_big, 4000)
                ctx.synchronize()
            for t in (y_small, y_moe):
                ctx.check(lib().tmh_upload(ctx.handle, t.ptr, np.full(t.size, 7, np.uint16).ctypes.data_as(
                    ctypes.c_void_p), t.nbytes))
            ctx.check(lib().tmh_graph_launch(ctx.handle, graph, None))
            ctx.synchronize()
            assert np.array_equal(y_small.numpy(), want[0]), round_
            assert np.array_equal(y_moe.numpy(), want[1]), round_
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


def test_prepared_matmul_integer_replays_match_eager():
    """MatMulInteger over a prepared B inside a graph: every replay equals the eager call."""
    from transmuter_amd._lib import S32
    from transmuter_amd.packed import Int8Weight

    ctx = Context(0)
    try:
        rng = np.random.default_rng(23)
        m, k, n = 300, 1040, 400
        b = rng.integers(0, 256, (k, n), dtype=np.uint8)
        w = Int8Weight.prepare(ctx, b, rng.integers(0, 256, n, dtype=np.uint8))
        a = ctx.put(rng.integers(0, 256, (m, k), dtype=np.uint8))
        az = ctx.put(np.array([17], np.uint8))
        y = ctx.empty((m, n), "s32")

        def call():
            ctx.check(lib().tmh_matmul_integer_prepared(ctx.handle, a.ptr, U8, az.ptr, 1, 1, m, w.handle, y.ptr, None))

        call()
        want = y.numpy()
        graph = ctypes.c_void_p()
        ctx.check(lib().tmh_graph_begin(ctx.handle, None))
        call()
        ctx.check(lib().tmh_graph_end(ctx.handle, None, ctypes.byref(graph)))
        for _ in range(3):
            ctx.check(lib().tmh_upload(ctx.handle, y.ptr, np.zeros((m, n), np.int32).ctypes.data_as(ctypes.c_void_p),
                                       y.nbytes))
            ctx.check(lib().tmh_graph_launch(ctx.handle, graph, None))
            ctx.synchronize()
            assert np.array_equal(y.numpy(), want)
        ctx.check(lib().tmh_graph_destroy(ctx.handle, graph))
        del S32
        w.free()
    finally:
        ctx.close()
