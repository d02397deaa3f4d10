"""The u8/s8 activation path on the GPU: DynamicQuantizeLinear and MatMulInteger (int8 MFMA with
row/column-sum corrections) against the oracle, bit-exactly, and the reference's
MatMulInteger_dynamic_quant graph (DynamicQuantizeLinear -> MatMulInteger on the device, Cast
and Mul on the host as they stay on the Nx backend) against its ONNX Runtime output."""

import ctypes
import zlib

import numpy as np
import pytest

from fixtures import Fixture, tolerance
from oracle import oracle as o
from transmuter_amd import quantized
from transmuter_amd.onnx_wire import NodeProto

pytestmark = pytest.mark.gpu

MI_CASES = [
    # batch, M, K, N, a type, b type, a_zero (None / "scalar" / "row"), b_zero, b batched
    (1, 1, 64, 16, "u8", "s8", "scalar", None, False),
    (1, 130, 200, 70, "u8", "u8", "row", "col", False),    # ragged tiles and k
    (1, 128, 256, 128, "s8", "s8", None, None, False),
    (1, 33, 4096, 257, "u8", "s8", "scalar", "scalar", False),
    (3, 40, 96, 48, "s8", "u8", "row", "col", True),
    (2, 17, 75, 9, "u8", "u8", "scalar", "col", False),      # K and N off every vector width
    (1, 300, 512, 520, "u8", "s8", "scalar", None, False),
    # K and N multiples of 16 (16-byte buffer loads): ragged M and N tiles, a last k-step of 16
    (1, 200, 272, 208, "u8", "u8", "row", "col", False),
    (2, 129, 1040, 400, "s8", "u8", "scalar", "col", True),
    (1, 513, 2048, 384, "u8", "s8", "scalar", None, False),
    (1, 256, 512, 1024, "u8", "u8", "scalar", "col", False),  # 16 tiles: the XCD tile order
    # 256 rows and more over a shared B with K a multiple of 16: one k-step of 16, N off 16 and
    # off 4 (scalar output stores), a batch of A over one B
    (1, 256, 16, 16, "s8", "u8", "row", "col", False),
    (2, 200, 4096, 257, "u8", "u8", "row", "col", False),
    (1, 384, 1040, 130, "s8", "s8", "scalar", "scalar", False),
    (3, 100, 272, 64, "u8", "s8", None, "col", False),
    (1, 512, 1024, 512, "u8", "u8", "scalar", "col", False),
]


def _ints(rng, shape, dtype):
    return rng.integers(-128, 128, shape, dtype=np.int8) if dtype == "s8" else rng.integers(0, 256, shape, dtype=np.uint8)


@pytest.mark.parametrize("case", MI_CASES, ids=lambda c: "b{}_M{}_K{}_N{}_{}{}".format(*c[:6]))
def test_matmul_integer_matches_oracle(ctx, case):
    print(f"matmul_integer {case}", flush=True)
    _check_plain(ctx, case)


@pytest.mark.parametrize("seed", range(24))
def test_random_matmul_integer(ctx, seed):
    """Seeded random MatMulInteger over B as given: any K, ragged M and N, batched A with a shared
    or batched B, every signedness and zero-point layout."""
    rng = np.random.default_rng(9500 + seed)
    batch = int(rng.choice([1, 1, 1, 2, 3]))
    case = (batch, int(rng.integers(1, 400)), int(rng.integers(1, 1600)), int(rng.integers(1, 400)),
            str(rng.choice(["u8", "s8"])), str(rng.choice(["u8", "s8"])), rng.choice([None, "scalar", "row"]),
            rng.choice([None, "scalar", "col"]), bool(batch > 1 and rng.random() < 0.5))
    print(f"random matmul_integer seed={seed} {case}", flush=True)
    _check_plain(ctx, case)


@pytest.mark.parametrize("seed", range(16))
def test_random_matmul_integer_many_rows(ctx, seed):
    """Seeded random MatMulInteger over B as given with 256 to 700 rows over a shared B and K a
    multiple of 16 (the 16-byte load path over several row tiles): ragged M and N, every
    signedness and zero-point layout."""
    rng = np.random.default_rng(9700 + seed)
    batch = int(rng.choice([1, 1, 2]))
    case = (batch, int(rng.integers(256 // batch, 700 // batch)), 16 * int(rng.integers(1, 100)),
            int(rng.integers(1, 400)), str(rng.choice(["u8", "s8"])), str(rng.choice(["u8", "s8"])),
            rng.choice([None, "scalar", "row"]), rng.choice([None, "scalar", "col"]), False)
    print(f"random matmul_integer (many rows) seed={seed} {case}", flush=True)
    _check_plain(ctx, case)


def test_matmul_integer_extremes_over_row_tiles(ctx):
    """Every product at its largest magnitude over two row tiles (u8 255 x 255 and s8 -128 x -128
    over K = 4096: 266 M, past 2^24), with the zero points at their ends."""
    k, m, n = 4096, 256, 48
    for adt, bdt, av, bv in (("u8", "u8", 255, 255), ("s8", "s8", -128, -128), ("u8", "s8", 255, -128)):
        a = np.full((m, k), av, np.uint8 if adt == "u8" else np.int8)
        b = np.full((k, n), bv, np.uint8 if bdt == "u8" else np.int8)
        az = np.array([0 if adt == "u8" else 127], a.dtype)
        bz = np.full(n, 0 if bdt == "u8" else 127, b.dtype)
        node = NodeProto(op_type="MatMulInteger", input=["a", "b", "az", "bz"], output=["y"])
        got = quantized.apply(node, [ctx.put(a), ctx.put(b), ctx.put(az), ctx.put(bz)])[0].numpy()
        want = k * (int(av) - int(az[0])) * (int(bv) - int(bz[0]))
        assert np.all(got == want), (adt, bdt)


def _check_plain(ctx, case):
    batch, m, k, n, adt, bdt, az, bz, bb = case
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    a = _ints(rng, (batch, m, k) if batch > 1 else (m, k), adt)
    b = _ints(rng, (batch, k, n) if bb else (k, n), bdt)
    a_zero = None if az is None else _ints(rng, (1,) if az == "scalar" else (m,), adt)
    b_zero = None if bz is None else _ints(rng, (1,) if bz == "scalar" else (n,), bdt)
    inputs = [ctx.put(a), ctx.put(b), ctx.put(a_zero) if a_zero is not None else None,
              ctx.put(b_zero) if b_zero is not None else None]
    node = NodeProto(op_type="MatMulInteger", input=["a", "b", "az" if az else "", "bz" if bz else ""], output=["y"])
    got = quantized.apply(node, inputs)[0].numpy()
    ref = o.matmul_integer(a, b, a_zero.reshape(-1) if a_zero is not None else None,
                           b_zero.reshape(-1) if b_zero is not None else None)
    assert got.dtype == np.int32 and got.shape == ref.shape
    assert np.array_equal(got, ref)


def test_matmul_integer_extremes_past_two_to_the_24(ctx):
    """Every product at its largest: 4096 * 255 * 255 is beyond 2^24 (f32-exact) but within s32."""
    k = 4096
    a = np.full((3, k), 255, np.uint8)
    b = np.full((k, 5), 255, np.uint8)
    node = NodeProto(op_type="MatMulInteger", input=["a", "b"], output=["y"])
    got = quantized.apply(node, [ctx.put(a), ctx.put(b)])[0].numpy()
    assert np.all(got == 4096 * 255 * 255)


DQL_CASES = [
    ("normal", 1000), ("normal", 5), ("normal", 300_000), ("positive", 4097), ("negative", 77), ("constant", 64),
    ("zeros", 10), ("ties", 256), ("empty", 0),
    # partial ranges over many workgroups, reduced in the quantize pass; grid-stride rounds and
    # a ragged tail
    ("normal", 2048 * 2048), ("positive", 2_000_003), ("negative", 1_048_577),
]


def _dql_input(rng, kind, n):
    if kind == "normal":
        return rng.standard_normal(n).astype(np.float32) * 3
    if kind == "positive":
        return rng.random(n).astype(np.float32) * 7 + 0.5
    if kind == "negative":
        return -rng.random(n).astype(np.float32) * 2 - 0.25
    if kind == "constant":
        return np.full(n, 2.5, np.float32)
    if kind == "zeros":
        return np.zeros(n, np.float32)
    if kind == "ties":  # x / scale lands on halves: scale is exactly 1 here
        return np.arange(n, dtype=np.float32) - np.float32(127.5)
    return np.zeros(0, np.float32)


@pytest.mark.parametrize("case", DQL_CASES, ids=lambda c: f"{c[0]}_{c[1]}")
def test_dynamic_quantize_linear_matches_oracle(ctx, case):
    kind, n = case
    print(f"dynamic_quantize_linear {case}", flush=True)
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    _check_dql(ctx, _dql_input(rng, kind, n))


@pytest.mark.parametrize("seed", range(24))
def test_random_dynamic_quantize_linear(ctx, seed):
    """Seeded random DynamicQuantizeLinear: rank 1-3 shapes up to about 3 M values, each input
    kind, scaled over magnitudes from 2^-20 to 2^20 and shifted off zero."""
    rng = np.random.default_rng(9700 + seed)
    kind = str(rng.choice(["normal", "positive", "negative", "constant", "zeros", "ties"]))
    rank = int(rng.integers(1, 4))
    shape = tuple(int(x) for x in rng.integers(1, [3_000_000, 2000, 150][rank - 1], size=rank))
    x = _dql_input(rng, kind, int(np.prod(shape))).reshape(shape)
    if kind != "ties":
        x = (x * np.float32(2.0 ** int(rng.integers(-20, 21))) + np.float32(rng.standard_normal())).astype(np.float32)
    print(f"random dynamic_quantize_linear seed={seed} {kind} {shape}", flush=True)
    _check_dql(ctx, x)


def _check_dql(ctx, x):
    n = x.size
    node = NodeProto(op_type="DynamicQuantizeLinear", input=["x"], output=["y", "s", "z"])
    y, s, z = (t.numpy() for t in quantized.apply(node, [ctx.put(x)]))
    if n == 0:  # no range: the scale of a constant (1) and zero point 0
        assert y.shape == (0,) and s == np.float32(1) and z == 0
        return
    ry, rs, rz = o.dynamic_quantize_linear(x)
    assert y.dtype == np.uint8 and y.shape == x.shape
    assert np.array_equal(y, ry)
    assert np.float32(s).view(np.uint32) == np.float32(rs).view(np.uint32)
    assert np.uint8(z) == rz


def test_dynamic_quant_matmul_fixture(ctx):
    """MatMulInteger_dynamic_quant: x -> DynamicQuantizeLinear -> MatMulInteger with the s8
    weights and the activation zero point -> Cast -> Mul by (x scale * w scale)."""
    f = Fixture("MatMulInteger_dynamic_quant")
    values = {name: ctx.put(v) for name, v in f.inputs.items()}
    values.update(f.initializers)
    for node in f.nodes:
        args = [values[name] if name else None for name in node.input]
        if node.op_type in quantized.op_types():
            outs = quantized.apply(node, args)
        elif node.op_type == "Cast":
            outs = [np.asarray(args[0].numpy(), np.float32)]
        else:  # Mul
            host = [a.numpy() if hasattr(a, "numpy") else np.asarray(a) for a in args]
            outs = [(np.asarray(host[0], np.float32) * np.asarray(host[1], np.float32)).astype(np.float32)]
        for name, v in zip(node.output, outs):
            values[name] = v
    got = np.asarray(values["y"])
    expected = f.outputs["y"]
    assert got.shape == expected.shape
    assert np.abs(got - expected).max() <= tolerance(expected)


# MatMulInteger over a B prepared once (tmh_int8_weight_prepare: B transposed to s8 rows of k with
# its column sums and zero points folded in), against the oracle, bit-exactly: u8/s8 on either
# side, every zero-point form, batched A, ragged M and N (N off the 16-byte stores), K a multiple
# of 16 but not of a 128-byte k-step, and one prepared B serving calls of different M.
PREPARED_CASES = [
    # batch, M, K, N, a type, b type, a_zero, b_zero
    (1, 1, 64, 16, "u8", "s8", "scalar", None),
    (1, 130, 272, 70, "u8", "u8", "row", "col"),
    (1, 128, 256, 128, "s8", "s8", None, None),
    (1, 33, 4096, 257, "u8", "s8", "scalar", "scalar"),
    (3, 40, 96, 48, "s8", "u8", "row", "col"),
    (2, 17, 16, 9, "u8", "u8", "scalar", "col"),
    (1, 300, 512, 520, "u8", "s8", "scalar", None),
    (2, 129, 1040, 400, "s8", "u8", "scalar", "col"),
    (1, 513, 2048, 384, "u8", "s8", "scalar", None),
    (1, 256, 512, 1024, "u8", "u8", "scalar", "col"),
]


@pytest.mark.parametrize("case", PREPARED_CASES, ids=lambda c: "b{}_M{}_K{}_N{}_{}{}_{}_{}".format(*c))
def test_matmul_integer_prepared_matches_oracle(ctx, case):
    print(f"matmul_integer prepared {case}", flush=True)
    _check_prepared(ctx, case)


def _draw_prepared(seed):
    """A seeded random MatMulInteger over a prepared B: K a multiple of 16 (what preparation
    takes), M and N ragged against the 128-row tiles, batches, every signedness and zero-point
    layout."""
    rng = np.random.default_rng(9000 + seed)
    batch = int(rng.choice([1, 1, 1, 2, 3]))
    m = int(rng.integers(1, 400))
    k = 16 * int(rng.integers(1, 100))
    n = int(rng.integers(1, 400))
    return (batch, m, k, n, str(rng.choice(["u8", "s8"])), str(rng.choice(["u8", "s8"])),
            rng.choice([None, "scalar", "row"]), rng.choice([None, "scalar", "col"]))


@pytest.mark.parametrize("seed", range(24))
def test_random_matmul_integer_prepared(ctx, seed):
    case = _draw_prepared(seed)
    print(f"random matmul_integer prepared seed={seed} {case}", flush=True)
    _check_prepared(ctx, case)


def _check_prepared(ctx, case):
    from transmuter_amd.packed import Int8Weight

    batch, m, k, n, adt, bdt, az, bz = case
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()) + 7)
    b = _ints(rng, (k, n), bdt)
    b_zero = None if bz is None else _ints(rng, (1,) if bz == "scalar" else (n,), bdt)
    w = Int8Weight.prepare(ctx, b, b_zero)
    for mm in (m, max(1, m // 2 + 1)):
        a = _ints(rng, (batch, mm, k) if batch > 1 else (mm, k), adt)
        a_zero = None if az is None else _ints(rng, (1,) if az == "scalar" else (mm,), adt)
        node = NodeProto(op_type="MatMulInteger", input=["a", "b", "az" if az else "", ""], output=["y"])
        got = quantized.apply(node, [ctx.put(a), w, ctx.put(a_zero) if a_zero is not None else None, None])[0].numpy()
        ref = o.matmul_integer(a, b, a_zero.reshape(-1) if a_zero is not None else None,
                               b_zero.reshape(-1) if b_zero is not None else None)
        assert got.dtype == np.int32 and got.shape == ref.shape
        assert np.array_equal(got, ref), f"M={mm}"
    w.free()


def test_matmul_integer_prepared_extremes_and_full_size(ctx):
    """Every product at its largest (4096 * 255 * 255, beyond 2^24), and the 2048^3 u8 x u8 product
    with zero points equal to the plain MatMulInteger kernel's, bit for bit."""
    from transmuter_amd.packed import Int8Weight

    w = Int8Weight.prepare(ctx, np.full((4096, 5), 255, np.uint8))
    node = NodeProto(op_type="MatMulInteger", input=["a", "b"], output=["y"])
    got = quantized.apply(node, [ctx.put(np.full((3, 4096), 255, np.uint8)), w])[0].numpy()
    assert np.all(got == 4096 * 255 * 255)
    w.free()
    rng = np.random.default_rng(2048)
    a = rng.integers(0, 256, (2048, 2048), dtype=np.uint8)
    b = rng.integers(0, 256, (2048, 2048), dtype=np.uint8)
    az, bz = np.array([131], np.uint8), rng.integers(0, 256, 2048, dtype=np.uint8)
    plain = NodeProto(op_type="MatMulInteger", input=["a", "b", "az", "bz"], output=["y"])
    want = quantized.apply(plain, [ctx.put(a), ctx.put(b), ctx.put(az), ctx.put(bz)])[0].numpy()
    w = Int8Weight.prepare(ctx, b, bz)
    prepared = NodeProto(op_type="MatMulInteger", input=["a", "b", "az", ""], output=["y"])
    got = quantized.apply(prepared, [ctx.put(a), w, ctx.put(az), None])[0].numpy()
    assert np.array_equal(got, want)
    w.free()


@pytest.mark.parametrize("a_shape,b_shape", [((3, 0), (0, 5)), ((2, 3, 0), (0, 5)), ((3, 0), (2, 0, 5)),
                                             ((0, 7), (2, 7, 5)), ((4, 7), (7, 0))])
def test_matmul_integer_empty_operands(ctx, a_shape, b_shape):
    """Empty operands: a contraction over K = 0 gives zeros (A and B hold no device bytes), and no
    rows or no columns give an empty result, for plain A over a batched B too."""
    print(f"matmul_integer empty {a_shape} x {b_shape}", flush=True)
    a = np.zeros(a_shape, np.uint8)
    b = np.zeros(b_shape, np.int8)
    node = NodeProto(op_type="MatMulInteger", input=["a", "b"], output=["y"])
    y = quantized.apply(node, [ctx.put(a), ctx.put(b)])[0]
    ref = o.matmul_integer(a, b)
    got = y.numpy()
    assert got.shape == ref.shape and np.array_equal(got, ref)


def test_matmul_integer_prepare_needs_k_in_sixteens(ctx):
    from transmuter_amd._lib import TmhArgumentError
    from transmuter_amd.packed import Int8Weight

    assert not Int8Weight.supported(75, 9)
    with pytest.raises(TmhArgumentError, match="multiple of 16"):
        Int8Weight.prepare(ctx, np.zeros((75, 9), np.uint8))


def test_dynamic_quant_matmul_fixture_with_b_prepared_at_load(ctx):
    """The MatMulInteger_dynamic_quant graph after the load-time move: its MatMulInteger reads the
    s8 weight initializer prepared as "<B>:int8", and the graph still matches ONNX Runtime."""
    from transmuter_amd import hip
    from transmuter_amd.packed import Int8Weight

    f = Fixture("MatMulInteger_dynamic_quant")
    model = hip.Model(nodes=list(f.nodes), params={}, static=dict(f.initializers), outputs=["y"])
    moved = hip.prepare_matmul_integer(model, ctx)
    mi = [node for node in moved.nodes if node.op_type == "MatMulInteger"]
    assert mi and all(node.input[1].endswith(":int8") for node in mi)
    assert all(isinstance(moved.params[node.input[1]], Int8Weight) for node in mi)
    values = {name: ctx.put(v) for name, v in f.inputs.items()}
    values.update(moved.static)
    values.update(moved.params)
    for node in moved.nodes:
        args = [values[name] if name else None for name in node.input]
        if node.op_type in quantized.op_types():
            outs = quantized.apply(node, args)
        elif node.op_type == "Cast":
            outs = [np.asarray(args[0].numpy(), np.float32)]
        else:  # Mul
            host = [a.numpy() if hasattr(a, "numpy") else np.asarray(a) for a in args]
            outs = [(np.asarray(host[0], np.float32) * np.asarray(host[1], np.float32)).astype(np.float32)]
        for name, v in zip(node.output, outs):
            values[name] = v
    got = np.asarray(values["y"])
    expected = f.outputs["y"]
    assert got.shape == expected.shape
    assert np.abs(got - expected).max() <= tolerance(expected)


def test_prepared_matmul_integer_offset_view_and_row_blocks(ctx, monkeypatch):
    """A prepared MatMulInteger whose A is an offset view (not 16-byte aligned) is copied to an
    aligned buffer first, and an A longer than one launch's 32-bit offsets reach goes in blocks of
    rows per batch (forced here with a small row limit): both bit-exact against the oracle, with
    one a_zero_point per row so the blocks must take their own slice of it."""
    from transmuter_amd import DeviceTensor
    from transmuter_amd.packed import Int8Weight

    rng = np.random.default_rng(77)
    batch, m, k, n = 2, 300, 272, 130
    b = _ints(rng, (k, n), "u8")
    bz = _ints(rng, (n,), "u8")
    w = Int8Weight.prepare(ctx, b, bz)
    a = _ints(rng, (batch, m, k), "u8")
    az = _ints(rng, (m,), "u8")
    ref = o.matmul_integer(a, b, az, bz)
    node = NodeProto(op_type="MatMulInteger", input=["a", "b", "az", ""], output=["y"])
    # A at byte offset 3 inside a larger buffer.
    buf = ctx.put(np.concatenate([np.zeros(3, np.uint8), a.ravel(), np.zeros(13, np.uint8)]))
    view = DeviceTensor(ctx, ctypes.c_void_p(buf.ptr.value + 3), a.shape, "u8", a.nbytes)
    view._owner = False
    assert view.ptr.value % 16 != 0
    for limit in (None, 64):
        monkeypatch.setattr(quantized, "PREPARED_ROW_LIMIT", limit)
        print(f"prepared MatMulInteger offset A, row limit {limit}", flush=True)
        got = quantized.apply(node, [view, w, ctx.put(az), None])[0].numpy()
        assert np.array_equal(got, ref), limit
        aligned = quantized.apply(node, [ctx.put(a), w, ctx.put(az), None])[0].numpy()
        assert np.array_equal(aligned, ref), limit
    w.free()
    buf.free()


def test_prepared_matmul_integer_with_no_rows(ctx):
    """An A of zero rows (no device buffer behind it) gives a [0, N] result over a prepared B, as
    the plain MatMulInteger does, and the same B still serves the next call."""
    from transmuter_amd.packed import Int8Weight

    rng = np.random.default_rng(79)
    b = _ints(rng, (64, 24), "s8")
    w = Int8Weight.prepare(ctx, b)
    node = NodeProto(op_type="MatMulInteger", input=["a", "b"], output=["y"])
    for batch_shape in ((), (3,)):
        print(f"prepared MatMulInteger with no rows, batch {batch_shape}", flush=True)
        got = quantized.apply(node, [ctx.put(np.zeros(batch_shape + (0, 64), np.uint8)), w])[0]
        assert got.shape == batch_shape + (0, 24) and got.dtype == "s32"
    a = _ints(rng, (5, 64), "u8")
    assert np.array_equal(quantized.apply(node, [ctx.put(a), w])[0].numpy(), o.matmul_integer(a, b, None, None))
    w.free()


def test_handlers_defer_freeing_their_uploads(ctx):
    """A handler that uploads host inputs frees them after its work is done, without waiting
    for it: the temporaries wait on an event until the next synchronize or download."""
    rng = np.random.default_rng(78)
    a = _ints(rng, (64, 128), "u8")
    b = _ints(rng, (128, 48), "s8")
    node = NodeProto(op_type="MatMulInteger", input=["a", "b"], output=["y"])
    ctx.synchronize()
    a_t = ctx.put(a)
    y = quantized.apply(node, [a_t, b])[0]  # B is uploaded by the handler
    assert ctx.pending_frees() == 1
    got = y.numpy()  # the download drains the stream: the uploads are freed
    assert ctx.pending_frees() == 0
    assert np.array_equal(got, o.matmul_integer(a, b, None, None))


def _dql_call(ctx, x_dev, n, y, s, z):
    from transmuter_amd._lib import F32, lib
    ctx.check(lib().tmh_dynamic_quantize_linear(ctx.handle, x_dev.ptr, F32, n, y.ptr, s.ptr, z.ptr, None))


def _dql_check(got_y, got_s, got_z, x):
    ry, rs, rz = o.dynamic_quantize_linear(x)
    assert np.array_equal(got_y, ry)
    assert np.float32(got_s).view(np.uint32) == np.float32(rs).view(np.uint32)
    assert np.uint8(got_z) == rz


def test_dynamic_quantize_linear_calls_in_a_row_and_graph_replays():
    """Calls of different sizes in a row on a fresh context (the partial ranges of one call in
    the workspace the previous call sized), then one call captured and replayed with calls of
    other sizes between the replays: every output equals the oracle's."""
    import ctypes
    from transmuter_amd import Context
    from transmuter_amd._lib import lib
    ctx = Context(0)
    try:
        rng = np.random.default_rng(98)
        sizes = (1, 4096, 8193, 2048 * 2048, 33, 3 * 1024 * 1024 + 7)
        xs = [_dql_input(rng, "normal", n) * np.float32(1 + i) for i, n in enumerate(sizes)]
        outs = []
        for x in xs:
            print(f"dynamic_quantize_linear in a row n={x.size}", flush=True)
            xd, y, s, z = ctx.put(x), ctx.empty((x.size,), "u8"), ctx.empty((1,), "f32"), ctx.empty((1,), "u8")
            _dql_call(ctx, xd, x.size, y, s, z)
            outs.append((xd, y, s, z))
        ctx.synchronize()
        for x, (_, y, s, z) in zip(xs, outs):
            _dql_check(y.numpy(), s.numpy()[0], z.numpy()[0], x)
        xd, y, s, z = outs[3]
        graph = ctypes.c_void_p()
        ctx.check(lib().tmh_graph_begin(ctx.handle, None))
        _dql_call(ctx, xd, xs[3].size, y, s, z)
        ctx.check(lib().tmh_graph_end(ctx.handle, None, ctypes.byref(graph)))
        for rep in range(3):
            print(f"dynamic_quantize_linear graph replay {rep}", flush=True)
            ctx.check(lib().tmh_upload(ctx.handle, y.ptr, np.full(y.size, 3, np.uint8).ctypes.data_as(ctypes.c_void_p),
                                       y.nbytes))
            ctx.check(lib().tmh_graph_launch(ctx.handle, graph, None))
            ctx.synchronize()
            _dql_check(y.numpy(), s.numpy()[0], z.numpy()[0], xs[3])
            xo, yo, so, zo = outs[rep % 3]  # an eager call of another size between replays
            _dql_call(ctx, xo, xs[rep % 3].size, yo, so, zo)
            ctx.synchronize()
            _dql_check(yo.numpy(), so.numpy()[0], zo.numpy()[0], xs[rep % 3])
        ctx.check(lib().tmh_graph_destroy(ctx.handle, graph))
    finally:
        ctx.synchronize()
        ctx.close()


def test_dynamic_quantize_linear_large_and_unaligned(ctx):
    """More values than one grid-stride round of either pass covers (8 M + 5), and x at an
    offset that is not a multiple of 16 bytes (the scalar paths of both passes)."""
    from transmuter_amd.device import DeviceTensor
    rng = np.random.default_rng(99)
    big = _dql_input(rng, "normal", 2 * 2048 * 2048 + 5)
    print(f"dynamic_quantize_linear large n={big.size}", flush=True)
    _check_dql(ctx, big)
    x = _dql_input(rng, "positive", 300_001)
    buf = ctx.put(np.concatenate([np.zeros(1, np.float32), x, np.zeros(3, np.float32)]))
    view = DeviceTensor(ctx, ctypes.c_void_p(buf.ptr.value + 4), x.shape, "f32", x.nbytes)
    view._owner = False
    assert view.ptr.value % 16 != 0
    print("dynamic_quantize_linear offset x", flush=True)
    y, s, z = ctx.empty(x.shape, "u8"), ctx.empty((1,), "f32"), ctx.empty((1,), "u8")
    _dql_call(ctx, view, x.size, y, s, z)
    ctx.synchronize()
    _dql_check(y.numpy(), s.numpy()[0], z.numpy()[0], x)
    buf.free()
