"""Launch timelines of the library's kernels (tmh_timeline_begin / tmh_timeline_end).

While a timeline records, the calls of a context launch the stamping builds of their main
kernels: each wavefront writes the GPU's 100 MHz real-time counter and its shader cycle counter
at its start and end into its own 16-byte slot. Calls captured into HIP graphs keep their slots,
so replaying the graphs measures the kernels where they are timed: inside the replays, with the
next launch's dispatch overlapping the previous kernel's end, which a tracer that launches each
kernel by itself does not see.

    tl = Timeline(ctx, capacity=1 << 20)
    tl.begin()
    graph = capture(...)          # or eager calls
    tl.end()
    replay(graph)
    launches = tl.launches()      # per launch: kernel, start/end (us), duration (us), clock (GHz)
"""

from __future__ import annotations

import ctypes

import numpy as np

from ._lib import TIMELINE_KERNELS, lib

TICK_US = 0.01  # the real-time counter runs at 100 MHz
_MISSING = 0xFFFFFFFF


class Timeline:
    """The slots of one context's launch timeline and the log of its launches."""

    MAX_LAUNCHES = 1 << 20

    def __init__(self, ctx, capacity: int):
        self.ctx = ctx
        self.capacity = int(capacity)
        self.buf = ctx.empty((self.capacity * 4,), "s32")
        self.log: list[tuple[str, int, int]] = []
        self.dropped = 0

    def clear(self) -> None:
        """Marks every slot unwritten (each wavefront that stamps overwrites its own slot)."""
        host = np.full(self.capacity * 4, _MISSING, np.uint32)
        self.ctx.check(lib().tmh_upload(self.ctx.handle, self.buf.ptr, host.ctypes.data_as(ctypes.c_void_p),
                                        host.nbytes))

    def begin(self) -> None:
        self.clear()
        self.ctx.check(lib().tmh_timeline_begin(self.ctx.handle, self.buf.ptr, self.capacity))

    def end(self) -> list[tuple[str, int, int]]:
        """Stops recording. Returns the launches since begin() as (kernel, first slot, wavefronts),
        in launch order; launches beyond the slots (counted in self.dropped) ran unstamped."""
        cap = min(self.capacity, self.MAX_LAUNCHES)
        log = np.zeros(3 * cap, np.int64)
        n, dropped = ctypes.c_int64(), ctypes.c_int64()
        self.ctx.check(lib().tmh_timeline_end(self.ctx.handle, log.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                              cap, ctypes.byref(n), ctypes.byref(dropped)))
        if n.value > cap:
            raise RuntimeError(f"the timeline logged {n.value} launches, more than {cap} read back")
        self.dropped = int(dropped.value)
        self.log = [(TIMELINE_KERNELS.get(int(k), f"kernel {int(k)}"), int(first), int(waves))
                    for k, first, waves in log[: 3 * n.value].reshape(-1, 3)]
        return self.log

    def stamps(self) -> np.ndarray:
        """The slots as u32 [capacity, 4]: real-time start, end; cycle counter start, end."""
        return self.buf.numpy().view(np.uint32).reshape(self.capacity, 4)

    def launches(self) -> list[dict]:
        """Per logged launch: kernel, wavefronts stamped, start and end (us, from the earliest
        stamp of the timeline: the first wavefront's start, the last one's end), duration (us) and
        the shader clock over its wavefronts (GHz: cycles over real time, summed over them)."""
        st = self.stamps().astype(np.int64)
        written = ~np.all(st == _MISSING, axis=1)
        real0 = st[written, 0]
        if real0.size == 0:
            return []
        # Counters are 32-bit: times are taken modulo 2^32 from the earliest start, which holds
        # while the timeline spans less than 42 s.
        ref = int(real0[np.argmin((real0 - real0[0] + (1 << 31)) % (1 << 32))])
        out = []
        for kernel, first, waves in self.log:
            s = st[first:first + waves]
            ok = written[first:first + waves]
            if not ok.any():
                out.append({"kernel": kernel, "waves": 0})
                continue
            s = s[ok]
            t0 = (s[:, 0] - ref) % (1 << 32)
            t1 = (s[:, 1] - ref) % (1 << 32)
            real = (s[:, 1] - s[:, 0]) % (1 << 32)
            cyc = (s[:, 3] - s[:, 2]) % (1 << 32)
            start, end = int(t0.min()), int(t1.max())
            out.append({"kernel": kernel, "waves": int(ok.sum()), "start_us": start * TICK_US,
                        "end_us": end * TICK_US, "us": (end - start) * TICK_US,
                        "ghz": float(cyc.sum()) / float(real.sum()) / 10.0 if real.sum() else None})
        return out

    def free(self) -> None:
        self.buf.free()
