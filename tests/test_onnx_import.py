"""ONNX import without the onnx package: the wire-format codec and from_onnx.

The cases mirror the reference's import tests (tests/test_import.py:21-191): symbolic
dimensions and whole input shapes, opset bounds and operator domains, unsupported element types,
undefined values, control flow, the Constant node forms, string attributes, the legacy softmax
axis, optional inputs and unused outputs. The reference builds its models with onnx.helper; here
they come from this build's own writer (``onnx_proto.make_*``), so what pins the decoder to the
real format is the set of files PyTorch's exporter wrote (tests/golden/onnx, see
make_onnx_fixtures.py): libtorch serializes them with its compiled copy of the ONNX schema, and
each is imported and run by the oracle interpreter against PyTorch's own outputs. Field-level
checks against the protobuf runtime's encoder cover the encodings PyTorch does not write
(packed and unpacked lists, negative varints, typed payload fields).
"""

from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import pytest

from ml_graph_compiler import builders
from ml_graph_compiler import onnx_proto as pb
from ml_graph_compiler.cli import main as cli_main
from ml_graph_compiler.errors import ModelImportError, UnsupportedOpError
from ml_graph_compiler.ir import TensorType
from ml_graph_compiler.onnx_export import save_onnx, to_onnx
from ml_graph_compiler.onnx_import import from_onnx, opset_version
from oracle import interpreter as oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "onnx"
MANIFEST = json.loads((GOLDEN / "manifest.json").read_text())


def model_of(nodes, inputs, outputs, inits=(), opset=14, domain=""):
    return pb.make_model(pb.make_graph(nodes, "m", inputs, outputs, list(inits)), opset=opset, domain=domain)


def vi(name, shape, elem=pb.FLOAT):
    return pb.make_value_info(name, elem, shape)


def node(op, inputs, outputs, **attrs):
    return pb.make_node(op, inputs, outputs, **attrs)


def fixture(name):
    z = np.load(GOLDEN / f"{name}.npz")
    feeds = {k[3:]: z[k] for k in z.files if k.startswith("in_")}
    outs = {k[4:]: z[k] for k in z.files if k.startswith("out_")}
    return feeds, outs


# -- files written by PyTorch's exporter -----------------------------------------------------


@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_torch_exported_models_match_torch(name):
    """Decoded, imported and interpreted, each file reproduces PyTorch's float32 outputs."""
    graph = from_onnx(GOLDEN / f"{name}.onnx", dims=MANIFEST[name]["dims"])
    assert graph.opset == MANIFEST[name]["opset"]
    feeds, want = fixture(name)
    got = oracle.run_graph(graph, feeds)
    for k, w in want.items():
        assert got[k].shape == w.shape
        err = float(np.max(np.abs(got[k].astype(np.float64) - w)))
        assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), (k, err)


def test_torch_file_metadata():
    m = pb.load_model(GOLDEN / "encoder_unfolded_dynamic.onnx")
    assert m.producer_name == "pytorch" and m.ir_version >= 7
    assert [(o.domain, o.version) for o in m.opset_import] == [("", 13)]
    (x,) = m.graph.input
    assert x.name == "x" and x.elem_type == pb.FLOAT
    assert [(d.dim_value, d.dim_param) for d in x.shape] == [(None, "batch"), (None, "sequence"), (32, "")]
    consts = [n for n in m.graph.node if n.op_type == "Constant"]
    assert consts and all(a.type == pb.A_TENSOR for n in consts for a in n.attribute)
    gemm = pb.load_model(GOLDEN / "cnn.onnx").graph.node
    attrs = {a.name: pb.attribute_value(a) for n in gemm if n.op_type == "Conv" for a in n.attribute}
    assert attrs["kernel_shape"] == [3, 3] and attrs["pads"] == [1, 1, 1, 1]


def test_torch_shape_arithmetic_is_partially_evaluated():
    """Shape -> Gather -> Unsqueeze -> Concat -> Reshape over the bound dims types every Reshape."""
    graph = from_onnx(GOLDEN / "encoder_unfolded_dynamic.onnx", dims={"batch": 3, "sequence": 5})
    reshapes = [n for n in graph.nodes if n.op == "Reshape"]
    assert len(reshapes) == 4 and all(n.output.type is not None for n in reshapes)
    assert graph.outputs[0].type == TensorType("float32", (3, 5, 32))


def test_legacy_softmax_file_from_torch():
    graph = from_onnx(GOLDEN / "legacy_softmax_opset11.onnx")
    assert graph.opset == 11
    assert [n.attrs["axis"] for n in graph.nodes if n.op in ("Softmax", "LogSoftmax")] == [-1, -1]


# -- the reference's import cases -----------------------------------------------------------


def test_import_from_path(tmp_path):
    path = save_onnx(builders.mlp(), tmp_path / "mlp.onnx")
    graph = from_onnx(path)
    assert graph.inputs[0].type == TensorType("float32", (4, 16))
    assert graph.opset == 14


@pytest.mark.parametrize("name", sorted(builders.SAMPLES))
def test_samples_round_trip_bit_exact(name):
    g = builders.SAMPLES[name]()
    back = from_onnx(to_onnx(g).encode())
    assert [n.op for n in back.nodes if n.op != "Identity"] == [n.op for n in g.nodes]
    feeds = oracle.random_feeds(g, 1, int_high=50)
    want, got = oracle.run_graph(g, feeds), oracle.run_graph(back, feeds)
    assert all(np.array_equal(want[k], got[k]) for k in want)


def test_symbolic_dims_and_input_shapes():
    model = model_of([node("Relu", ["x"], ["y"])], [vi("x", ["batch", 3])], [vi("y", ["batch", 3])])
    with pytest.raises(ModelImportError, match="dynamic dimension 'batch'"):
        from_onnx(model)
    assert from_onnx(model, dims={"batch": 5}).outputs[0].type == TensorType("float32", (5, 3))
    assert from_onnx(model, input_shapes={"x": (7, 3)}).outputs[0].tensor_type.shape == (7, 3)
    with pytest.raises(ModelImportError, match="unknown inputs"):
        from_onnx(model, input_shapes={"nope": (1,)}, dims={"batch": 1})


def test_unknown_dimension_without_name():
    model = model_of([node("Relu", ["x"], ["y"])], [vi("x", [None, 3])], [vi("y", None)])
    with pytest.raises(ModelImportError, match="'\\?'"):
        from_onnx(model)


def test_missing_shape_is_a_scalar():
    model = model_of([node("Relu", ["x"], ["y"])], [vi("x", None)], [vi("y", None)])
    assert from_onnx(model).inputs[0].type == TensorType("float32", ())


def test_opset_bounds_and_domains():
    nodes = [node("Relu", ["x"], ["y"])]
    with pytest.raises(ModelImportError, match="opset 6 is outside the supported range 7..21"):
        from_onnx(model_of(nodes, [vi("x", [2])], [vi("y", [2])], opset=6))
    with pytest.raises(ModelImportError, match="opset 22"):
        from_onnx(model_of(nodes, [vi("x", [2])], [vi("y", [2])], opset=22))
    custom = model_of([pb.make_node("Foo", ["x"], ["y"], domain="com.example")], [vi("x", [2])], [vi("y", [2])])
    custom.opset_import.append(pb.OperatorSetIdProto("com.example", 1))
    with pytest.raises(ModelImportError, match="domain 'com.example' \\(Foo\\)"):
        from_onnx(custom)
    other = model_of(nodes, [vi("x", [2])], [vi("y", [2])], domain="com.example")
    assert opset_version(other) == 21
    assert from_onnx(model_of(nodes, [vi("x", [2])], [vi("y", [2])], domain="ai.onnx", opset=9)).opset == 9


def test_unsupported_input_type_and_undefined_values():
    nodes = [node("Relu", ["x"], ["y"])]
    with pytest.raises(ModelImportError, match="element type 8"):
        from_onnx(model_of(nodes, [vi("x", [2], pb.STRING)], [vi("y", [2])]))
    with pytest.raises(ModelImportError, match="undefined value 'missing'"):
        from_onnx(model_of([node("Relu", ["missing"], ["y"])], [vi("x", [2])], [vi("y", [2])]))
    with pytest.raises(ModelImportError, match="'z' is never defined"):
        from_onnx(model_of(nodes, [vi("x", [2])], [vi("z", [2])]))


def test_unsupported_operator():
    with pytest.raises(UnsupportedOpError):
        from_onnx(model_of([node("NonMaxSuppression", ["x"], ["y"])], [vi("x", [2])], [vi("y", [2])]))


def test_control_flow_is_rejected():
    body = pb.make_graph([], "b", [], [])
    model = model_of([node("If", ["c"], ["y"], then_branch=body, else_branch=body)],
                     [vi("c", [], pb.BOOL)], [vi("y", [2])])
    with pytest.raises(ModelImportError, match="control flow"):
        from_onnx(model.encode())
    loop = model_of([node("Scan", ["c"], ["y"], bodies=[body])], [vi("c", [], pb.BOOL)], [vi("y", [2])])
    with pytest.raises(ModelImportError, match="control flow"):
        from_onnx(loop.encode())


@pytest.mark.parametrize(
    "attr, expected, dtype",
    [
        ({"value": pb.from_array(np.arange(3, dtype=np.float32))}, [0.0, 1.0, 2.0], np.float32),
        ({"value_float": 2.5}, 2.5, np.float32),
        ({"value_floats": [1.0, 2.0]}, [1.0, 2.0], np.float32),
        ({"value_int": 4}, 4, np.int64),
        ({"value_ints": [1, 2]}, [1, 2], np.int64),
    ],
)
def test_constant_node_forms(attr, expected, dtype):
    nodes = [node("Constant", [], ["c"], **attr), node("Identity", ["c"], ["y"])]
    graph = from_onnx(model_of(nodes, [], [vi("y", None)]).encode())
    out = oracle.run_graph(graph, {})["y"]
    assert out.dtype == dtype and out.tolist() == expected


def test_constant_node_unsupported_form():
    with pytest.raises(ModelImportError, match="unsupported Constant attributes \\['value_string'\\]"):
        from_onnx(model_of([node("Constant", [], ["c"], value_string="hi")], [], [vi("c", None)]).encode())


def test_string_and_tensor_list_attributes_import():
    graph = from_onnx(model_of([node("Gelu", ["x"], ["y"], approximate="tanh")], [vi("x", [3])],
                               [vi("y", [3])], opset=20).encode())
    assert graph.nodes[0].attrs["approximate"] == "tanh"
    a = pb.AttributeProto.decode(memoryview(pb.make_attribute("t", [np.ones(2, np.int32), np.zeros((1, 2))]).encode()))
    assert a.type == pb.A_TENSORS and [pb.to_array(t).dtype for t in a.tensors] == [np.int32, np.float64]
    s = pb.AttributeProto.decode(memoryview(pb.make_attribute("s", ["a", "bc"]).encode()))
    assert pb.attribute_value(s) == [b"a", b"bc"]


def test_legacy_softmax_last_axis_and_rejection():
    nodes = [node("Softmax", ["x"], ["y"], axis=1)]
    graph = from_onnx(model_of(nodes, [vi("x", [2, 5])], [vi("y", [2, 5])], opset=11))
    assert graph.nodes[0].attrs["axis"] == -1
    x = np.random.default_rng(0).standard_normal((2, 5)).astype(np.float32)
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    np.testing.assert_allclose(oracle.run_graph(graph, {"x": x})["y"], e / e.sum(1, keepdims=True), rtol=1e-6)
    # the default axis before opset 13 is 1: last axis of a 2-D input, not of a 3-D one
    plain = from_onnx(model_of([node("LogSoftmax", ["x"], ["y"])], [vi("x", [3, 4])], [vi("y", [3, 4])], opset=12))
    assert plain.nodes[0].attrs["axis"] == -1
    with pytest.raises(UnsupportedOpError, match="2-D coercion"):
        from_onnx(model_of(nodes, [vi("x", [2, 3, 4])], [vi("y", [2, 3, 4])], opset=11))
    modern = from_onnx(model_of(nodes, [vi("x", [2, 3, 4])], [vi("y", [2, 3, 4])], opset=13))
    assert modern.nodes[0].attrs["axis"] == 1


def test_optional_inputs_and_unused_outputs():
    nodes = [node("Clip", ["x", "", "hi"], ["c"]), node("Dropout", ["c"], ["y", ""])]
    hi = pb.from_array(np.asarray(0.5, np.float32), "hi")
    graph = from_onnx(model_of(nodes, [vi("x", [4])], [vi("y", [4])], inits=[hi]).encode())
    assert graph.nodes[0].inputs[1] is None
    assert graph.nodes[1].outputs[1].name == "dropout_unused"
    out = oracle.run_graph(graph, {"x": np.asarray([-1, 0, 1, 2], np.float32)})
    assert out["y"].tolist() == [-1, 0, 0.5, 0.5]


def test_initializers_listed_as_inputs():
    """Files before IR version 4 also list every initializer among the graph inputs."""
    w = pb.from_array(np.full((2,), 3.0, np.float32), "w")
    model = model_of([node("Mul", ["x", "w"], ["y"])], [vi("x", [2]), vi("w", [2])], [vi("y", [2])], inits=[w])
    graph = from_onnx(model.encode())
    assert [v.name for v in graph.inputs] == ["x"]
    assert oracle.run_graph(graph, {"x": np.ones(2, np.float32)})["y"].tolist() == [3.0, 3.0]


# -- the wire format --------------------------------------------------------------------------


def _varint_py(n: int) -> bytes:
    n &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = n & 0x7F
        n >>= 7
        out.append(b | (0x80 if n else 0))
        if not n:
            return bytes(out)


def test_packed_varints_against_scalar_decoding():
    rng = np.random.default_rng(3)
    values = [0, 1, 127, 128, 300, 2**31 - 1, -1, -(2**31), 2**63 - 1, -(2**63), 2**35 + 7]
    values += [int(v) for v in rng.integers(-(2**62), 2**62, 200)]
    packed = b"".join(_varint_py(v) for v in values)
    got = pb._packed_varints(memoryview(packed)).view(np.int64).tolist()
    assert got == values
    pos, scalar = 0, []
    while pos < len(packed):
        v, pos = pb._varint_at(memoryview(packed), pos)
        scalar.append(pb._signed(v))
    assert scalar == values
    with pytest.raises(ModelImportError, match="truncated"):
        pb._packed_varints(memoryview(packed[:-1] + b"\x80"))


def test_typed_payload_fields():
    """Tensors whose values sit in the typed fields instead of raw_data, as older writers and
    hand-built models store them; FLOAT16 keeps bit patterns in int32_data."""
    halves = np.array([1.5, -2.0, 65504.0], np.float16)
    cases = [
        (pb.TensorProto("f", [2, 2], pb.FLOAT, float_data=np.array([1, 2, 3, 4], np.float32)), np.arange(1, 5, dtype=np.float32).reshape(2, 2)),
        (pb.TensorProto("d", [2], pb.DOUBLE, double_data=np.array([0.1, -7.0])), np.array([0.1, -7.0])),
        (pb.TensorProto("l", [3], pb.INT64, int64_data=np.array([-5, 0, 2**40])), np.array([-5, 0, 2**40], np.int64)),
        (pb.TensorProto("i", [3], pb.INT32, int32_data=np.array([-7, 0, 2**31 - 1])), np.array([-7, 0, 2**31 - 1], np.int32)),
        (pb.TensorProto("b", [3], pb.INT8, int32_data=np.array([-128, 5, 127])), np.array([-128, 5, 127], np.int8)),
        (pb.TensorProto("u", [2], pb.UINT8, int32_data=np.array([0, 255])), np.array([0, 255], np.uint8)),
        (pb.TensorProto("q", [2], pb.BOOL, int32_data=np.array([1, 0])), np.array([True, False])),
        (pb.TensorProto("h", [3], pb.FLOAT16, int32_data=halves.view(np.uint16).astype(np.int64)), halves),
        (pb.TensorProto("w", [2], pb.UINT64, uint64_data=np.array([2**64 - 1, 3], np.uint64)), np.array([2**64 - 1, 3], np.uint64)),
        (pb.TensorProto("s", [], pb.FLOAT, float_data=np.array([2.5], np.float32)), np.array(2.5, np.float32)),
        (pb.TensorProto("e", [0, 3], pb.FLOAT), np.zeros((0, 3), np.float32)),
    ]
    for tensor, want in cases:
        got = pb.to_array(pb.TensorProto.decode(memoryview(tensor.encode())))
        assert got.dtype == want.dtype and got.shape == want.shape and np.array_equal(got, want), tensor.name
    with pytest.raises(ModelImportError, match="holds 3 values"):
        pb.to_array(pb.TensorProto("x", [2, 2], pb.FLOAT, float_data=np.zeros(3, np.float32)))
    with pytest.raises(ModelImportError, match="raw_data holds 4 bytes"):
        pb.to_array(pb.TensorProto("x", [2], pb.FLOAT, raw_data=b"\0" * 4))
    with pytest.raises(ModelImportError, match="unsupported data type 16"):
        pb.to_array(pb.TensorProto("x", [1], pb.BFLOAT16, raw_data=b"\0\0"))


def test_unpacked_and_packed_lists_decode_alike():
    """proto2 writers emit repeated scalars unpacked unless the field says packed; a parser takes
    both, even mixed within one message."""
    w = pb._Writer()
    w.str(1, "axes")
    w.int(8, 3)
    w.packed_varints(8, [-1, 4])
    w.int(8, 2**33)
    w.float(7, 0.5)
    w.packed(7, np.array([1.25, -3.0], "<f4"))
    w.int(20, pb.A_INTS)
    a = pb.AttributeProto.decode(memoryview(w.done()))
    assert a.ints == [3, -1, 4, 2**33] and a.floats == [0.5, 1.25, -3.0]


def test_missing_attribute_type_is_inferred():
    w = pb._Writer()
    w.str(1, "alpha")
    w.float(2, 0.25)
    a = pb.AttributeProto.decode(memoryview(w.done()))
    assert a.type == pb.A_FLOAT and pb.attribute_value(a) == 0.25


def test_against_protobuf_runtime():
    """The protobuf runtime's own encoder, given a schema with these field numbers, produces
    bytes this decoder reads back (and the reverse): negative int64 and int32 varints, packed
    repeated fields, nested messages, proto2 presence of a zero dim_value."""
    descriptor_pb2 = pytest.importorskip("google.protobuf.descriptor_pb2")
    from google.protobuf import descriptor_pool, message_factory

    F = descriptor_pb2.FieldDescriptorProto
    fdp = descriptor_pb2.FileDescriptorProto(name="mini_onnx.proto", package="mini", syntax="proto2")

    def message(name, fields):
        m = fdp.message_type.add(name=name)
        for fname, number, ftype, label, type_name, packed in fields:
            f = m.field.add(name=fname, number=number, type=ftype, label=label)
            if type_name:
                f.type_name = f".mini.{type_name}"
            if packed:
                f.options.packed = True

    OPT, REP = F.LABEL_OPTIONAL, F.LABEL_REPEATED
    message("Tensor", [("dims", 1, F.TYPE_INT64, REP, "", False), ("data_type", 2, F.TYPE_INT32, OPT, "", False),
                       ("float_data", 4, F.TYPE_FLOAT, REP, "", True), ("int32_data", 5, F.TYPE_INT32, REP, "", True),
                       ("int64_data", 7, F.TYPE_INT64, REP, "", True), ("name", 8, F.TYPE_STRING, OPT, "", False),
                       ("raw_data", 9, F.TYPE_BYTES, OPT, "", False)])
    message("Attr", [("name", 1, F.TYPE_STRING, OPT, "", False), ("f", 2, F.TYPE_FLOAT, OPT, "", False),
                     ("i", 3, F.TYPE_INT64, OPT, "", False), ("t", 5, F.TYPE_MESSAGE, OPT, "Tensor", False),
                     ("ints", 8, F.TYPE_INT64, REP, "", False), ("type", 20, F.TYPE_INT32, OPT, "", False)])
    message("Dim", [("dim_value", 1, F.TYPE_INT64, OPT, "", False), ("dim_param", 2, F.TYPE_STRING, OPT, "", False)])
    pool = descriptor_pool.DescriptorPool()
    pool.Add(fdp)
    cls = {n: message_factory.GetMessageClass(pool.FindMessageTypeByName(f"mini.{n}")) for n in ("Tensor", "Attr", "Dim")}

    t = cls["Tensor"](dims=[2, 3], data_type=pb.INT32, int32_data=[-1, 2, -(2**31), 7, 0, 9], name="t")
    mine = pb.TensorProto.decode(memoryview(t.SerializeToString()))
    assert pb.to_array(mine).tolist() == [[-1, 2, -(2**31)], [7, 0, 9]] and mine.name == "t"
    t64 = cls["Tensor"](dims=[2], data_type=pb.INT64, int64_data=[-(2**63), 2**62])
    assert pb.to_array(pb.TensorProto.decode(memoryview(t64.SerializeToString()))).tolist() == [-(2**63), 2**62]

    a = cls["Attr"](name="a", i=-3, ints=[-1, 0, 5], type=pb.A_INTS)
    a.t.CopyFrom(cls["Tensor"](dims=[1], data_type=pb.FLOAT, float_data=[0.75]))
    da = pb.AttributeProto.decode(memoryview(a.SerializeToString()))
    assert (da.i, da.ints, pb.to_array(da.t).tolist()) == (-3, [-1, 0, 5], [0.75])

    d = pb.Dimension.decode(memoryview(cls["Dim"](dim_value=0).SerializeToString()))
    assert d.dim_value == 0  # present, though zero

    back = cls["Attr"]()
    back.ParseFromString(pb.make_attribute("perm", [0, -2, 1]).encode())
    assert list(back.ints) == [0, -2, 1] and back.type == pb.A_INTS
    back_t = cls["Tensor"]()
    back_t.ParseFromString(pb.from_array(np.array([[1.5, 2.0]], np.float32), "w").encode())
    assert list(back_t.dims) == [1, 2] and back_t.name == "w"
    assert struct.unpack("<2f", back_t.raw_data) == (1.5, 2.0)


def test_external_data(tmp_path):
    weights = np.arange(6, dtype=np.float32).reshape(2, 3)
    blob = b"\xff" * 16 + weights.tobytes()
    (tmp_path / "weights.bin").write_bytes(blob)
    ext = pb.TensorProto("w", [2, 3], pb.FLOAT, data_location=pb.EXTERNAL,
                         external_data={"location": "weights.bin", "offset": "16", "length": str(weights.nbytes)})
    model = model_of([node("Add", ["x", "w"], ["y"])], [vi("x", [2, 3])], [vi("y", [2, 3])], inits=[ext])
    path = pb.save_model(model, tmp_path / "m.onnx")
    graph = from_onnx(path)
    assert np.array_equal(graph.nodes[0].input(1).data, weights)
    with pytest.raises(ModelImportError, match="load the model from its path"):
        from_onnx(model.encode())
    ext.external_data["location"] = "../escape.bin"
    with pytest.raises(ModelImportError, match="not a file inside"):
        from_onnx(pb.save_model(model, tmp_path / "bad.onnx"))


def test_malformed_files(tmp_path):
    good = model_of([node("Relu", ["x"], ["y"])], [vi("x", [2])], [vi("y", [2])]).encode()
    for bad in (good[:-3], b"\x0a\xff\xff\xff\xff\x0f", b"not a model at all"):
        p = tmp_path / "bad.onnx"
        p.write_bytes(bad)
        with pytest.raises(ModelImportError):
            from_onnx(p)
    with pytest.raises(ModelImportError, match="cannot read"):
        from_onnx(tmp_path / "missing.onnx")


# -- command line -----------------------------------------------------------------------------


def test_cli_compile_binds_dims_and_shapes(tmp_path, capsys):
    """``mgc compile`` imports the file with its symbolic dimensions bound and reports import
    errors with exit status 2; without a GPU the build stops at loading, loudly."""
    path = str(GOLDEN / "mlp_dynamic_batch.onnx")
    assert cli_main(["compile", path]) == 2
    assert "dynamic dimension 'batch'" in capsys.readouterr().err
    assert cli_main(["compile", path, "--dim", "batch"]) == 2
    assert "--dim expects NAME=INT" in capsys.readouterr().err
    assert cli_main(["compile", path, "--shape", "x=2by16"]) == 2
    assert "--shape expects" in capsys.readouterr().err
    assert cli_main(["compile", "no-such-model"]) == 2
    assert "neither a file nor a bundled sample" in capsys.readouterr().err
    assert cli_main(["compile", path, "--dim", "batch=6", "--backend", "c", "--cache-dir", str(tmp_path)]) == 2
    assert "not part of this build" in capsys.readouterr().err
    assert cli_main(["compile", path, "--shape", "x=2x16", "--check", "--cache-dir", str(tmp_path)]) == 2
    assert "no HIP device" in capsys.readouterr().err
    from ml_graph_compiler.cli import load_model

    assert load_model(path, dims=["batch=6"]).inputs[0].type == TensorType("float32", (6, 16))
    assert load_model(path, shapes=["x=2x16"]).outputs[0].type == TensorType("float32", (2, 4))
    # the bundled samples go to ONNX and back unchanged
    out = tmp_path / "cnn.onnx"
    save_onnx(builders.tiny_cnn(), out)
    back = load_model(str(out))
    from ml_graph_compiler.cli import random_inputs
    from ml_graph_compiler.evaluate import evaluate_graph

    counts = {k: v for k, v in back.op_counts().items() if k != "Identity"}  # output renames
    assert counts == builders.tiny_cnn().op_counts()
    feeds = random_inputs(back, 1)
    for k, v in evaluate_graph(builders.tiny_cnn(), feeds).items():
        np.testing.assert_array_equal(evaluate_graph(back, feeds)[k], v)


def test_interpreter_check_matches_the_oracle():
    """``compile --check``'s CPU baseline (the operator table run node by node) agrees with the
    independent oracle."""
    from ml_graph_compiler.cli import random_inputs
    from ml_graph_compiler.evaluate import evaluate_graph

    for make in (builders.tiny_cnn, builders.tiny_bert, builders.mlp):
        g = make()
        feeds = random_inputs(g, 3)
        got, want = evaluate_graph(g, feeds), oracle.run_graph(make(), feeds)
        for k in want:
            np.testing.assert_allclose(got[k], want[k], rtol=2e-5, atol=2e-5)


def test_cli_random_token_ids_stay_in_range():
    """Integer inputs that index a Gather (directly or through reshapes and casts) are drawn
    below the gathered extent, so `compile --check/--bench` does not trip the index check."""
    from ml_graph_compiler import builders
    from ml_graph_compiler.cli import random_inputs

    g = from_onnx(GOLDEN / "tiny_gpt.onnx")
    vocab = next(n for n in g.nodes if n.op == "Gather").input(0).tensor_type.shape[0]
    assert random_inputs(g, int_high=10**6)["ids"].max() < vocab
    assert random_inputs(builders.bert_base(1), int_high=10**6)["input_ids"].max() < 30522
    assert random_inputs(builders.bert_base(1), int_high=7)["input_ids"].max() < 7
