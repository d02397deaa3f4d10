"""The C ABI on a host without a GPU: the library loads, exports every declared entry point,
reports errors without a device, validates MatMulNBits weights, and lays out packed weights
as its header documents (checked against an independent numpy restatement of the layout)."""

import ctypes
import os
import re

import numpy as np
import pytest

from synth import nbits_weight
from transmuter_amd import _lib
from transmuter_amd._lib import lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "transmuter_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tmh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 25
    handle = lib()
    for name in names:
        assert hasattr(handle, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version():
    assert lib().tmh_abi_version() == 1


def test_null_context_errors_do_not_crash():
    assert lib().tmh_synchronize(None, None) == _lib.ERR_INVALID
    assert b"NULL" in lib().tmh_last_error(None)
    assert lib().tmh_matmul_nbits(None, None, None, 1, 1, 1, None, 0, None, 1, 1, None) == _lib.ERR_INVALID
    assert lib().tmh_gather_block_quantized(None, None, 2, 1, 1, None, 7, 1, None, 1, 1, None, 0, 4, None, None) \
        == _lib.ERR_INVALID
    lib().tmh_weight_free(None)
    lib().tmh_ctx_destroy(None)


def test_no_device_is_reported():
    n = ctypes.c_int(-1)
    status = lib().tmh_device_count(ctypes.byref(n))
    if status == _lib.OK:
        pytest.skip("a GPU is visible")
    assert status == _lib.ERR_NO_DEVICE and n.value == 0
    ctx = ctypes.c_void_p()
    assert lib().tmh_ctx_create(0, ctypes.byref(ctx)) == _lib.ERR_NO_DEVICE


def pack_host(b, scales, zp, k, n, bits, bs, sdt=_lib.F16, wdt=_lib.F16, zp_kind=None, zdt=_lib.U8,
              query_only=False):
    b = np.ascontiguousarray(b)
    scales = np.ascontiguousarray(scales)
    if zp_kind is None:
        zp_kind = _lib.ZP_NONE if zp is None else (_lib.ZP_FLOAT if zp.dtype.kind == "f" else _lib.ZP_PACKED)
    zp = None if zp is None else np.ascontiguousarray(zp)
    sizes = [ctypes.c_size_t(0) for _ in range(3)]
    args = [b.ctypes.data_as(ctypes.c_void_p), b.nbytes, scales.ctypes.data_as(ctypes.c_void_p), sdt, scales.size,
            None if zp is None else zp.ctypes.data_as(ctypes.c_void_p), zp_kind, zdt, 0 if zp is None else zp.size,
            k, n, bits, bs, wdt]
    st = lib().tmh_pack_nbits_host(*args, None, ctypes.byref(sizes[0]), None, ctypes.byref(sizes[1]), None,
                                   ctypes.byref(sizes[2]))
    if st != _lib.OK or query_only:
        return st, None
    bufs = [np.zeros(max(1, s.value), np.uint8) for s in sizes]
    st = lib().tmh_pack_nbits_host(*args, bufs[0].ctypes.data_as(ctypes.c_void_p), ctypes.byref(sizes[0]),
                                   bufs[1].ctypes.data_as(ctypes.c_void_p), ctypes.byref(sizes[1]),
                                   bufs[2].ctypes.data_as(ctypes.c_void_p) if sizes[2].value else None,
                                   ctypes.byref(sizes[2]))
    return st, [buf[: s.value] for buf, s in zip(bufs, sizes)]


@pytest.mark.parametrize("kwargs,needle", [
    (dict(bits=3), b"bits must be 2, 4 or 8"),
    (dict(bs=24), b"power of two"),
    (dict(bs=8), b"power of two"),
    (dict(k=0), b"positive"),
    (dict(drop_b=1), b"B holds"),
    (dict(drop_s=1), b"scales hold"),
    (dict(drop_z=1), b"packed zero points hold"),
    (dict(sdt=_lib.S32), b"scales must be"),
    (dict(wdt=_lib.U8), b"weight type must be"),
    (dict(zdt=_lib.F32), b"packed zero points must be u8"),
])
def test_pack_validation(kwargs, needle):
    rng = np.random.default_rng(0)
    k, n, bits, bs = 64, 8, 4, 32
    b, s, z = nbits_weight(rng, k, n, bits, bs)
    if kwargs.pop("drop_b", 0):
        b = b.reshape(-1)[:-1]
    if kwargs.pop("drop_s", 0):
        s = s[:-1]
    if kwargs.pop("drop_z", 0):
        z = z[:-1]
    args = dict(k=k, n=n, bits=bits, bs=bs)
    args.update(kwargs)
    st, _ = pack_host(b, s, z, args["k"], args["n"], args["bits"], args["bs"], sdt=args.get("sdt", _lib.F16),
                      wdt=args.get("wdt", _lib.F16), zdt=args.get("zdt", _lib.U8), query_only=True)
    assert st == _lib.ERR_INVALID
    assert needle in lib().tmh_last_error(None)


def reference_layout(b, scales, zp, k, n, bits, bs):
    """The tiled layout written out from its definition: tiles of 16 rows, chunks of 64 bytes
    per row, lane l = 16g + r holding row r's bytes 16g..16g+15 of the chunk, sub-byte value 2j
    of each 32-bit word at bit j*bits and value 2j+1 at bit 16 + j*bits; parameters per
    (tile, chunk, block-of-chunk j, row), packed zero points `bits` bits each in entry order,
    lowest bits first (rows 2i and 2i+1 of a block share a byte at 4 bits)."""
    blocks = -(-k // bs)
    row_bytes = blocks * bs * bits // 8
    nchunks = -(-row_bytes // 64)
    ntiles = -(-n // 16)
    rows = np.zeros((ntiles * 16, nchunks * 64), np.uint8)
    rows[:n, :row_bytes] = b.reshape(n, row_bytes)
    q = np.zeros((ntiles, nchunks, 64, 16), np.uint8)
    for l in range(64):
        r, g = l % 16, l // 16
        q[:, :, l, :] = rows.reshape(ntiles, 16, nchunks, 64)[:, r, :, 16 * g:16 * g + 16]
    words = q.reshape(-1, 4).copy().view("<u4").reshape(-1).astype(np.uint64)
    if bits < 8:
        per = 32 // bits
        out = np.zeros_like(words)
        for i in range(per):
            v = (words >> np.uint64(i * bits)) & np.uint64((1 << bits) - 1)
            out |= v << np.uint64((i % 2) * 16 + (i // 2) * bits)
        words = out
    q_bytes = words.astype("<u4").view(np.uint8)
    cw = 512 // bits
    bsc = min(bs, cw)
    nbc = cw // bsc
    s = np.zeros((ntiles, nchunks, nbc, 16), np.float16)
    zz = np.full((ntiles, nchunks, nbc, 16), 1 << (bits - 1), np.uint8)
    zrow = -(-blocks * bits // 8)
    for t in range(ntiles):
        for c in range(nchunks):
            for j in range(nbc):
                blk = (c * cw + j * bsc) // bs
                for r in range(16):
                    row = t * 16 + r
                    if row < n and blk < blocks:
                        s[t, c, j, r] = scales[row * blocks + blk]
                        if zp is not None:
                            byte = zp[row * zrow + blk * bits // 8]
                            zz[t, c, j, r] = (byte >> ((blk * bits) % 8)) & ((1 << bits) - 1)
    per = 8 // bits
    entries = zz.reshape(-1, per).astype(np.uint32)
    packed = np.zeros(entries.shape[0], np.uint32)
    for i in range(per):
        packed |= entries[:, i] << np.uint32(i * bits)
    return q_bytes, s.view(np.uint8).reshape(-1), packed.astype(np.uint8)


@pytest.mark.parametrize("bits,bs,k,n", [(4, 32, 1024, 40), (4, 16, 96, 17), (4, 256, 512, 16), (8, 32, 200, 5),
                                         (2, 16, 128, 33), (4, 128, 72, 3)])
def test_packed_layout_matches_its_definition(bits, bs, k, n):
    rng = np.random.default_rng(bits * 1000 + k)
    b, s, z = nbits_weight(rng, k, n, bits, bs, zp="packed")
    st, (q, sc, zz) = pack_host(b, s, z, k, n, bits, bs)
    assert st == _lib.OK, lib().tmh_last_error(None)
    rq, rs, rz = reference_layout(b, s, z, k, n, bits, bs)
    assert np.array_equal(q, rq)
    assert np.array_equal(sc, rs)
    assert np.array_equal(zz, rz)


def test_pack_rejects_a_small_buffer():
    rng = np.random.default_rng(1)
    b, s, z = nbits_weight(rng, 64, 8, 4, 32)
    sizes = [ctypes.c_size_t(1) for _ in range(3)]
    bufs = [np.zeros(4096, np.uint8) for _ in range(3)]
    st = lib().tmh_pack_nbits_host(b.ctypes.data_as(ctypes.c_void_p), b.nbytes, s.ctypes.data_as(ctypes.c_void_p),
                                   _lib.F16, s.size, z.ctypes.data_as(ctypes.c_void_p), _lib.ZP_PACKED, _lib.U8, z.size,
                                   64, 8, 4, 32, _lib.F16, *[x for pair in zip(
                                       [bb.ctypes.data_as(ctypes.c_void_p) for bb in bufs],
                                       [ctypes.byref(sz) for sz in sizes]) for x in pair])
    assert st == _lib.ERR_INVALID and b"too small" in lib().tmh_last_error(None)


def test_qmoe_refuses_more_tokens_than_its_work_items_number():
    """Work items carry their index in 16 bits, at least 32 rows each, and an expert gets at most
    one row per token: more than 2^21 tokens could overflow that field, so the call refuses them
    before it touches a device (here, with no context at all)."""
    args = dict(x_dtype=_lib.F16, H=2048, router_dtype=_lib.F32, E=128, k=1)
    qmoe = lib().tmh_qmoe

    def call(T, k=1):
        return qmoe(None, None, args["x_dtype"], T, args["H"], None, args["router_dtype"], args["E"], k, None, None,
                    None, None, None, None, _lib.F16, 4, 0, 1.0, 0.0, 0.0, None, None)

    assert call((32 << 16) + 1) == _lib.ERR_UNSUPPORTED
    assert b"tokens per call" in lib().tmh_last_error(None)
    assert call(1 << 24, k=1) == _lib.ERR_UNSUPPORTED  # also past the routed-row limit
    # At the limit the sizes pass and the missing context is what fails.
    assert call(32 << 16) == _lib.ERR_INVALID
    assert b"context is NULL" in lib().tmh_last_error(None)
