"""Load-time packing and merging on the GPU, as the reference tests its move/2 and
Fusion.matmuls/2: a moved MatMulNBits gives the outputs of the dequantization in the graph
(ops_test.exs:182-244), move/2 rewrites the node to read "B:packed" and drops what only it
read (:74-149), and MatMulNBits nodes that read one input merge into one node and a Split
with the same outputs (fusion_test.exs:396-433)."""

import numpy as np
import pytest

from fixtures import Fixture
from oracle import oracle as o
from synth import nbits_weight
from transmuter_amd import PackedWeight
from transmuter_amd.hip import Model, merge_matmuls, move, run_nodes
from transmuter_amd.onnx_wire import ATTR_INT, AttributeProto, NodeProto

pytestmark = pytest.mark.gpu


def fixture_model():
    f = Fixture("MatMulNBits_b4_bs256_packed")
    node = f.node
    # B (>4096 bytes) is a param; the small scales and zero points are static values
    # (lib/transmuter.ex:29-32, :1310-1320; asserted at ops_test.exs:83).
    params = {"B": f.initializers["B"]}
    static = {"scales": f.initializers["scales"], "zp": f.initializers["zp"]}
    return Model(nodes=[node], params=params, static=static, outputs=["Y"]), node


def with_attr(node, name, value):
    attrs = [AttributeProto(name=a.name, type=a.type, i=value) if a.name == name else a for a in node.attribute]
    return NodeProto(input=list(node.input), output=list(node.output), name=node.name, op_type=node.op_type,
                     domain=node.domain, attribute=attrs)


def cases():
    model, node = fixture_model()
    rng = np.random.default_rng(3)
    b8 = rng.integers(0, 256, (40, 2, 256)).astype(np.uint8)
    zp8 = rng.integers(0, 256, (80,)).astype(np.uint8)
    no_zp = NodeProto(input=["A", "B", "scales", ""], output=["Y"], name=node.name, op_type=node.op_type,
                      domain=node.domain, attribute=node.attribute)
    return [
        ("4-bit with zero points", model),
        ("4-bit without zero points", Model(nodes=[no_zp], params=model.params,
                                            static={"scales": model.static["scales"]}, outputs=["Y"])),
        ("8-bit with zero points", Model(nodes=[with_attr(node, "bits", 8)], params={"B": b8},
                                         static={"scales": model.static["scales"], "zp": zp8}, outputs=["Y"])),
        ("f16 scales in f32", Model(nodes=[node], params=model.params,
                                    static={"scales": model.static["scales"].astype(np.float16),
                                            "zp": model.static["zp"]}, outputs=["Y"], compute_type="f32")),
    ]


@pytest.mark.parametrize("name,model", cases(), ids=[c[0] for c in cases()])
def test_moved_matmul_nbits_gives_the_in_graph_outputs(ctx, name, model):
    print(f"move case {name}", flush=True)
    rng = np.random.default_rng(5)
    a = rng.standard_normal((2, 3, 512)).astype(np.float32)
    inputs = {"A": ctx.put(a)}
    in_graph = run_nodes(model, inputs)["Y"].numpy()
    moved = move(model, ctx)
    assert moved.nodes[0].input == ["A", "B:packed", "", ""], name
    assert list(moved.params) == ["B:packed"], name
    weight = moved.params["B:packed"]
    assert isinstance(weight, PackedWeight) and weight.shape == (40, 512)
    assert "scales" not in moved.static and "zp" not in moved.static
    got = run_nodes(moved, inputs)["Y"].numpy()
    # Both run the f32 path over the same f32 weights: equal bits, as on EXLA (:237-239).
    assert got.dtype == np.float32
    assert np.array_equal(got.view(np.uint32), in_graph.view(np.uint32)), name
    # And both match the oracle of the graph.
    node = model.nodes[0]
    bits = next(a.i for a in node.attribute if a.name == "bits")
    values = {**model.static, **model.params}
    zp = values.get(node.input[3]) if len(node.input) > 3 and node.input[3] else None
    ref = o.matmul_nbits(a, values["B"], values["scales"].astype(np.float32), zp, k=512, n=40, bits=bits,
                         block_size=256)
    assert np.abs(got - ref).max() <= 1e-4 + 1e-3 * np.abs(ref).max()
    # A second move leaves the model as it is.
    again = move(moved, ctx)
    assert again.nodes[0].input == moved.nodes[0].input and list(again.params) == ["B:packed"]


def test_move_keeps_raw_values_that_other_nodes_read(ctx):
    """A GatherBlockQuantized of tied embeddings also reads B and the scales: they stay."""
    model, node = fixture_model()
    gather = NodeProto(input=["B", "ids", "scales"], output=["E"], op_type="GatherBlockQuantized")
    m2 = Model(nodes=[node, gather], params=model.params, static=model.static, outputs=["Y", "E"])
    moved = move(m2, ctx)
    assert moved.nodes[0].input == ["A", "B:packed", "", ""]
    assert "B" in moved.params and "scales" in moved.static and "zp" not in moved.static


def nbits_node(a, b, scales, out, n, k=1024, zp="", bits=4):
    attrs = [AttributeProto(name="K", type=ATTR_INT, i=k), AttributeProto(name="N", type=ATTR_INT, i=n),
             AttributeProto(name="bits", type=ATTR_INT, i=bits), AttributeProto(name="block_size", type=ATTR_INT, i=32)]
    inputs = [a, b, scales] + ([zp] if zp else [])
    return NodeProto(input=inputs, output=[out], name=out, op_type="MatMulNBits", domain="com.microsoft",
                     attribute=attrs)


def test_matmul_nbits_nodes_that_read_one_input_merge(ctx):
    """fusion_test.exs:396-433: two MatMulNBits of 4 bits read x; the move merges them into one
    MatMulNBits and a Split, with the outputs of the graph without the rewrite."""
    iota = lambda n, f: (np.arange(n * 32 * 16).reshape(n, 32, 16) * f % 256).astype(np.uint8)
    params = {"bq": iota(32, 7), "sq": np.full(32 * 32, 0.01, np.float32),
              "bk": iota(16, 13), "sk": np.full(16 * 32, 0.02, np.float32)}
    nodes = [nbits_node("x", "bq", "sq", "q", 32), nbits_node("x", "bk", "sk", "k", 16)]
    model = Model(nodes=nodes, params=params, outputs=["q", "k"])
    x = (np.arange(2 * 1024, dtype=np.float32).reshape(1, 2, 1024) % 17.0 - 8.0).astype(np.float32)
    inputs = {"x": ctx.put(x)}
    expected = run_nodes(model, inputs)
    moved = move(model, ctx)
    assert [n.op_type for n in moved.nodes] == ["MatMulNBits", "Split"]
    assert moved.nodes[0].input == ["x", "bq:packed:merged", "", ""]
    got = run_nodes(moved, inputs)
    for name in ("q", "k"):
        assert got[name].shape == expected[name].shape
        assert np.array_equal(got[name].numpy(), expected[name].numpy()), name


@pytest.mark.parametrize("ns,bits,zp", [([2048, 1024, 1024], 4, "packed"), ([40, 8, 24], 4, "packed"),
                                        ([17, 5], 4, "packed"), ([17, 5, 3, 1], 2, "packed"),
                                        ([33, 7, 2], 8, "packed"), ([21, 6], 4, "float"), ([9, 16], 4, "none")])
def test_concat_is_the_rows_of_its_parts(ctx, ns, bits, zp):
    """The merged weight holds every part's rows in order; part boundaries off the 16-row tiles
    move each row's packed zero points (several a byte below 8 bits) to another slot of a byte."""
    print(f"concat ns={ns} bits={bits} zp={zp}", flush=True)
    rng = np.random.default_rng(sum(ns) + bits)
    k = 1024
    parts, raw = [], []
    for n in ns:
        b, s, z = nbits_weight(rng, k, n, bits, 32, zp=zp)
        raw.append((b, s, z))
        parts.append(PackedWeight.upload(ctx, b, s, z, k=k, n=n, bits=bits, block_size=32, weight_dtype="f16"))
    merged = PackedWeight.concat(parts)
    assert merged.shape == (sum(ns), k)
    got = merged.dequantize().numpy()
    want = np.concatenate([o.dequantize_weight(b, s, z, k, n, bits, 32, o.F16) for (b, s, z), n in zip(raw, ns)])
    assert np.array_equal(got, want)
    from transmuter_amd.quantized import matmul_nbits

    a = ctx.put(rng.standard_normal((3, k)).astype(np.float16))
    y = matmul_nbits(a, merged).numpy()
    ys = np.concatenate([matmul_nbits(a, p).numpy() for p in parts], axis=1)
    assert np.array_equal(y, ys)


def test_mixed_precision_matmuls_on_one_input_merge_by_layout(ctx):
    """q and k of 4 bits and v of 8 bits read x (a mixed-precision export): the move merges q
    and k and leaves v alone, since packed weights of different bit widths do not concatenate;
    every output equals the graph's without the rewrite."""
    print("move mixed 4/8-bit", flush=True)
    rng = np.random.default_rng(12)
    params, nodes = {}, []
    for name, n, bits in (("q", 48, 4), ("k", 16, 4), ("v", 32, 8)):
        params["b" + name] = rng.integers(0, 256, (n, 32, 32 * bits // 8), dtype=np.uint8)
        params["s" + name] = (np.abs(rng.standard_normal(n * 32)) * 0.01 + 1e-3).astype(np.float32)
        nodes.append(nbits_node("x", "b" + name, "s" + name, name, n, bits=bits))
    model = Model(nodes=nodes, params=params, outputs=["q", "k", "v"])
    inputs = {"x": ctx.put(rng.standard_normal((2, 1024)).astype(np.float32))}
    expected = run_nodes(model, inputs)
    moved = move(model, ctx)
    assert [n.op_type for n in moved.nodes] == ["MatMulNBits", "Split", "MatMulNBits"]
    assert moved.nodes[0].input == ["x", "bq:packed:merged", "", ""] and moved.nodes[2].input[1] == "bv:packed"
    got = run_nodes(moved, inputs)
    for name in ("q", "k", "v"):
        assert np.array_equal(got[name].numpy(), expected[name].numpy()), name


def test_more_matmuls_on_one_input_than_one_concat_takes(ctx):
    """Ten MatMulNBits on one input merge in runs of at most eight parts."""
    print("move 10 matmuls on one input", flush=True)
    rng = np.random.default_rng(13)
    params, nodes = {}, []
    for i in range(10):
        n = 16 + 8 * i
        params[f"b{i}"] = rng.integers(0, 256, (n, 32, 16), dtype=np.uint8)
        params[f"s{i}"] = (np.abs(rng.standard_normal(n * 32)) * 0.01 + 1e-3).astype(np.float32)
        nodes.append(nbits_node("x", f"b{i}", f"s{i}", f"y{i}", n))
    model = Model(nodes=nodes, params=params, outputs=[f"y{i}" for i in range(10)])
    inputs = {"x": ctx.put(rng.standard_normal((3, 1024)).astype(np.float32))}
    expected = run_nodes(model, inputs)
    moved = move(model, ctx)
    assert [n.op_type for n in moved.nodes] == ["MatMulNBits", "Split", "MatMulNBits", "Split"]
    assert [len(n.output) for n in moved.nodes if n.op_type == "Split"] == [8, 2]
    got = run_nodes(moved, inputs)
    for name in expected:
        assert np.array_equal(got[name].numpy(), expected[name].numpy()), name


def test_bf16_scales_move_and_run(ctx):
    """bf16 scales (BF16Host bit patterns) with bf16 activations: the moved weight dequantizes in
    bf16 (the scales' type, no compute type), as the graph's does in A's type (quantized.ex:42),
    and both agree with each other and with the oracle."""
    from transmuter_amd.device import bf16_host

    print("move bf16 scales", flush=True)
    rng = np.random.default_rng(14)
    n, k = 40, 1024
    b = rng.integers(0, 256, (n, 32, 16), dtype=np.uint8)
    s32 = (np.abs(rng.standard_normal(n * 32)) * 0.01 + 1e-3).astype(np.float32)
    scales = bf16_host(o.bf16_round(s32))
    model = Model(nodes=[nbits_node("x", "B", "scales", "Y", n)], params={"B": b, "scales": scales}, outputs=["Y"])
    a32 = rng.standard_normal((2, k)).astype(np.float32)
    a = ctx.put(o.bf16_round(a32), "bf16")
    expected = run_nodes(model, {"x": a})["Y"]
    moved = move(model, ctx)
    weight = moved.params["B:packed"]
    assert isinstance(weight, PackedWeight) and weight.dtype == "bf16"
    got = run_nodes(moved, {"x": a})["Y"]
    assert got.dtype == "bf16" and expected.dtype == "bf16"
    assert np.array_equal(np.asarray(got.numpy()), np.asarray(expected.numpy()))
    ref = o.bf16_to_f32(o.matmul_nbits(o.bf16_round(a32), b, np.asarray(scales), None, k=k, n=n, bits=4,
                                       block_size=32)).astype(np.float64)  # bf16 A and weights: bf16 Y
    y = o.bf16_to_f32(np.asarray(got.numpy())).astype(np.float64)
    assert np.abs(y - ref).max() <= 2e-2 * np.abs(ref).max()
