"""The asynchronous boundary a NIF uses: compute calls return after enqueueing, an event
recorded after them is the completion fence of their outputs (tmh_event_query polls it without
blocking, tmh_event_synchronize waits for it), and nothing is read before the fence."""

import ctypes

import numpy as np
import pytest

from oracle import oracle as o
from synth import nbits_weight
from transmuter_amd import PackedWeight
from transmuter_amd._lib import F16, lib

pytestmark = pytest.mark.gpu


def test_enqueued_calls_complete_at_their_fence(ctx):
    print("async fence: 64 GEMVs enqueued, then polled", flush=True)
    rng = np.random.default_rng(41)
    k, n = 1024, 3072
    b, s, z = nbits_weight(rng, k, n, 4, 32)
    w = PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=4, block_size=32, weight_dtype="f16")
    a_host = rng.standard_normal((64, 1, k)).astype(np.float16)
    a = [ctx.put(x) for x in a_host]
    y = [ctx.empty((1, n), "f16") for _ in range(64)]
    fence = ctypes.c_void_p()
    ctx.check(lib().tmh_event_create(ctx.handle, ctypes.byref(fence)))
    for ai, yi in zip(a, y):  # enqueue only: no call waits
        ctx.check(lib().tmh_matmul_nbits(ctx.handle, w.handle, ai.ptr, F16, 1, k, None, 0, yi.ptr, F16, n, None))
    ctx.check(lib().tmh_event_record(ctx.handle, fence, None))
    done = ctypes.c_int(-1)
    ctx.check(lib().tmh_event_query(ctx.handle, fence, ctypes.byref(done)))
    assert done.value in (0, 1)
    ctx.check(lib().tmh_event_synchronize(ctx.handle, fence))
    ctx.check(lib().tmh_event_query(ctx.handle, fence, ctypes.byref(done)))
    assert done.value == 1
    wd = o.dequantize_weight(b, s, z, k, n, 4, 32, o.F16).astype(np.float64)
    for x, yi in zip(a_host[::9], y[::9]):
        ref = x.astype(np.float64) @ wd.T
        assert np.abs(yi.numpy().astype(np.float64) - ref).max() <= 1e-2 * np.abs(ref).max()
    ctx.check(lib().tmh_event_destroy(ctx.handle, fence))
    w.free()
