"""IR graph to an ONNX model file.

The inverse of ``onnx_import.from_onnx`` for graphs made of ONNX operators: graph inputs
become typed ValueInfoProtos, constants become initializers (raw little-endian data), nodes keep
their names, operator types and attributes, and the graph outputs keep their public names. It
lets the bundled model builders be saved as ``.onnx`` files (the reference ships its samples as
onnx.helper models, src/ml_graph_compiler/samples.py) and the importer be tested on files.
"""

from __future__ import annotations

from pathlib import Path

from . import onnx_proto as pb
from .errors import GraphError, ModelImportError
from .ir import Graph, Value
from .onnx_import import ELEM_TYPES

_ELEM_CODE = {name: code for code, name in ELEM_TYPES.items()}


def _value_info(v: Value, name: str | None = None) -> pb.ValueInfoProto:
    t = v.tensor_type
    return pb.make_value_info(name or v.name, _ELEM_CODE[t.dtype], list(t.shape))


def to_onnx(graph: Graph, producer_name: str = "ml-graph-compiler") -> pb.ModelProto:
    """An ONNX ModelProto of ``graph`` at ``graph.opset``; attributes whose names start with
    an underscore are compiler-internal and are left out."""
    initializers: list[pb.TensorProto] = []
    seen: set[int] = set()

    def constant(v: Value) -> None:
        if v.data is not None and id(v) not in seen:
            seen.add(id(v))
            initializers.append(pb.from_array(v.data, v.name))

    nodes: list[pb.NodeProto] = []
    for n in graph.nodes:
        for v in n.inputs:
            if v is not None:
                constant(v)
        try:
            attrs = [pb.make_attribute(k, a) for k, a in sorted(n.attrs.items()) if not k.startswith("_")]
        except ModelImportError as exc:
            raise GraphError(f"{n.op} node {n.name!r} cannot be written as ONNX: {exc}") from exc
        nodes.append(pb.NodeProto(["" if v is None else v.name for v in n.inputs],
                                  [v.name for v in n.outputs], n.name, n.op, "", attrs))
    outputs: list[pb.ValueInfoProto] = []
    for name, v in graph.named_outputs():
        constant(v)
        if name != v.name or any(o.name == name for o in outputs):
            nodes.append(pb.make_node("Identity", [v.name], [name], name=f"{name}_identity"))
        outputs.append(_value_info(v, name))
    proto = pb.make_graph(nodes, graph.name, [_value_info(v) for v in graph.inputs], outputs, initializers)
    return pb.make_model(proto, opset=graph.opset, producer_name=producer_name)


def save_onnx(graph: Graph, path: str | Path) -> Path:
    return pb.save_model(to_onnx(graph), path)
