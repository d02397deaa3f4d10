"""The launch timeline (tmh_timeline_begin / _end): the stamping builds of the decode GEMVs, the
prefill GEMM and its split-K sum, the vocabulary gather, the QMoE kernels and the floors
compute what the ordinary builds compute, bit for bit, and every wavefront of every logged launch
writes a start no later than its end; launches captured into a graph write their slots again at
each replay; launches beyond the slots run unstamped and are counted."""

import ctypes

import numpy as np
import pytest

from synth import nbits_weight
from transmuter_amd import PackedWeight
from transmuter_amd._lib import F16, F32, S64, U8, lib
from transmuter_amd.timeline import Timeline

pytestmark = pytest.mark.gpu


def _matmul(ctx, w, a, m, y):
    ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, a.ptr, F16, m, w.k, None, 0, y.ptr, F16, w.n, None))


def _check_launches(tl, kernels):
    got = [k for k, _first, _waves in tl.log]
    assert got == kernels, got
    for ln in tl.launches():
        assert ln["waves"] > 0, ln
        assert 0 <= ln["us"] < 10_000, ln
        assert ln["ghz"] is None or 0.3 < ln["ghz"] < 4.0, ln


@pytest.mark.parametrize("m,k,n,plan,kernels", [
    (1, 1024, 3072, None, ["k_gemv_dot"]),
    (8, 2048, 1024, None, ["k_gemv_dec"]),
    (1, 1024, 151936, None, ["k_gemv_dot"]),
    (256, 2048, 2048, "128,2,4", ["k_gemm_lds", "k_splitk_reduce"]),
    (300, 1024, 512, "256,4,1", ["k_gemm_lds"]),
])
def test_stamping_builds_compute_the_same_bits(ctx, monkeypatch, m, k, n, plan, kernels):
    if plan:
        monkeypatch.setenv("TMH_GEMM_PLAN", plan)
    else:
        monkeypatch.delenv("TMH_GEMM_PLAN", raising=False)
    rng = np.random.default_rng(m * 7 + n)
    bs = 128 if m > 16 else 32
    w = PackedWeight.upload(ctx, *nbits_weight(rng, k, n, 4, bs), k=k, n=n, bits=4, block_size=bs, weight_dtype="f16")
    a = ctx.put(rng.standard_normal((m, k)).astype(np.float16))
    y0, y1 = ctx.empty((m, n), "f16"), ctx.empty((m, n), "f16")
    print(f"timeline matmul M={m} K={k} N={n} plan={plan}", flush=True)
    _matmul(ctx, w, a, m, y0)
    tl = Timeline(ctx, 1 << 16)
    tl.begin()
    _matmul(ctx, w, a, m, y1)
    tl.end()
    ctx.synchronize()
    assert np.array_equal(y0.numpy().view(np.uint16), y1.numpy().view(np.uint16))
    _check_launches(tl, kernels)
    tl.free()
    w.free()


def test_graph_replays_rewrite_the_slots_and_overflow_is_counted(ctx):
    rng = np.random.default_rng(5)
    k, n = 1024, 2048
    w = PackedWeight.upload(ctx, *nbits_weight(rng, k, n, 4, 32), k=k, n=n, bits=4, block_size=32, weight_dtype="f16")
    a = ctx.put(rng.standard_normal((1, k)).astype(np.float16))
    y = ctx.empty((1, n), "f16")
    sink = ctx.empty((16,), "u8")
    tl = Timeline(ctx, 1 << 16)
    tl.begin()
    ctx.check(lib().tmh_graph_begin(ctx.handle, None))
    _matmul(ctx, w, a, 1, y)
    ctx.check(lib().tmh_floor_empty(ctx.handle, 64, None))
    ctx.check(lib().tmh_floor_read(ctx.handle, w.handle, sink.ptr, None))
    ctx.check(lib().tmh_floor_read_all(ctx.handle, w.handle, sink.ptr, None))
    ctx.check(lib().tmh_floor_write(ctx.handle, y.ptr, y.nbytes, None))
    graph = ctypes.c_void_p()
    ctx.check(lib().tmh_graph_end(ctx.handle, None, ctypes.byref(graph)))
    tl.end()
    print("timeline graph replays", flush=True)
    ends = []
    for _ in range(2):
        ctx.check(lib().tmh_graph_launch(ctx.handle, graph, None))
        ctx.synchronize()
        launches = tl.launches()
        ends.append(tl.stamps()[:, 1].copy())
        _check_launches(tl, ["k_gemv_dot", "k_floor_empty", "k_floor_read", "k_floor_read_all", "k_floor_write"])
        # in order: each launch starts after the previous one started
        starts = [ln["start_us"] for ln in launches]
        assert starts == sorted(starts)
    assert not np.array_equal(ends[0], ends[1])  # the second replay wrote them again
    ctx.check(lib().tmh_graph_destroy(ctx.handle, graph))
    # Too few slots: the launch runs unstamped (the same bits) and is counted.
    small = Timeline(ctx, 4)
    small.begin()
    y2 = ctx.empty((1, n), "f16")
    _matmul(ctx, w, a, 1, y2)
    small.end()
    assert small.log == [] and small.dropped == 1
    _matmul(ctx, w, a, 1, y)
    assert np.array_equal(y.numpy().view(np.uint16), y2.numpy().view(np.uint16))
    small.free()
    tl.free()
    w.free()


def test_gather_and_qmoe_stamping_builds(ctx):
    from oracle import oracle as o

    rng = np.random.default_rng(6)
    rows, hidden = 1000, 1024
    b = rng.integers(0, 256, (rows, hidden // 2), dtype=np.uint8)
    sc = (np.abs(rng.standard_normal((rows, hidden // 32))) * 0.01 + 1e-4).astype(np.float16)
    zp = rng.integers(0, 256, (rows, hidden // 64), dtype=np.uint8)
    ids = rng.integers(0, rows, (4, 33)).astype(np.int64)
    bt, st, zt, it = ctx.put(b), ctx.put(sc), ctx.put(zp), ctx.put(ids)
    out = ctx.empty((4, 33, hidden), "f16")
    tl = Timeline(ctx, 1 << 16)
    tl.begin()
    ctx.check(lib().tmh_gather_block_quantized(ctx.handle, bt.ptr, U8, rows, hidden // 2, it.ptr, S64, ids.size, st.ptr,
                                               F16, hidden // 32, zt.ptr, U8, 4, out.ptr, None))
    tl.end()
    ctx.synchronize()
    print("timeline gather", flush=True)
    ref = o.gather_block_quantized(b, ids, sc, zp, bits=4)
    assert np.array_equal(out.numpy().view(np.uint16), ref.view(np.uint16))
    _check_launches(tl, ["k_gather_bq_rows"])
    tl.free()
    # QMoE: 8 experts, top-2, SwiGLU over fc1 and fc3, f16.
    from transmuter_amd.moe import ExpertWeight

    e, kk, h, inter, t = 8, 2, 256, 128, 64
    ws = []
    for n_, k_ in ((inter, h), (inter, h), (h, inter)):
        packed = rng.integers(0, 256, (e, n_, k_ // 2), dtype=np.uint8)
        scales = (np.abs(rng.standard_normal((e, n_, k_ // 32))) * 0.01 + 1e-4).astype(np.float16)
        ws.append(ExpertWeight.upload(ctx, packed, scales, None, bits=4, block_size=32, dtype="f16"))
    x = ctx.put(rng.standard_normal((t, h)).astype(np.float16))
    router = ctx.put(rng.standard_normal((t, e)).astype(np.float32))
    ys = [ctx.empty((t, h), "f16") for _ in range(2)]
    tl = Timeline(ctx, 1 << 16)
    for i, yy in enumerate(ys):
        if i == 1:
            tl.begin()
        ctx.check(lib().tmh_qmoe(ctx.handle, x.ptr, F16, t, h, router.ptr, F32, e, kk, ws[0].handle, None,
                                 ws[2].handle, None, ws[1].handle, None, F16, 4, 0, 1.0, 0.0, 0.0, yy.ptr, None))
    tl.end()
    ctx.synchronize()
    print("timeline qmoe", flush=True)
    assert np.array_equal(ys[0].numpy().view(np.uint16), ys[1].numpy().view(np.uint16))
    _check_launches(tl, ["k_moe_route", "k_moe_plan", "k_moe_gemm_f16", "k_moe_gemm_f16", "k_moe_combine"])
    tl.free()
    for w in ws:
        w.free()
