"""ONNX model import: a model file to the SSA IR with every shape static.

Behaviour follows the reference importer (src/ml_graph_compiler/onnx_import.py:31-186): the
same opset range, element types, symbolic-dimension binding, Constant node forms, legacy
(opset < 13) softmax axis handling and error messages. The difference is the parser: the
reference hands the file to the onnx package, this build decodes the protobuf wire format
itself (``onnx_proto``), so a model compiles with no onnx installation.
"""

from __future__ import annotations

from pathlib import Path
from typing import Any

import numpy as np

from . import onnx_proto as pb
from .errors import ModelImportError, UnsupportedOpError
from .ir import Graph, TensorType, Value
from .shape_inference import infer_shapes

# element types a graph input may have (onnx_import.py:16-25)
ELEM_TYPES: dict[int, str] = {
    pb.FLOAT: "float32",
    pb.DOUBLE: "float64",
    pb.FLOAT16: "float16",
    pb.INT64: "int64",
    pb.INT32: "int32",
    pb.INT8: "int8",
    pb.UINT8: "uint8",
    pb.BOOL: "bool",
}

MIN_OPSET = 7
MAX_OPSET = 21

_CONTROL_FLOW = "graph-valued attributes (control flow) are not supported"


def _attribute(attr: pb.AttributeProto, base_dir: Path | None) -> Any:
    """Attribute value as the IR keeps it (onnx_import.py:31-47): str for strings, numpy arrays
    for tensors, lists for repeated values; graph attributes are refused."""
    value = pb.attribute_value(attr)
    if isinstance(value, bytes):
        return value.decode("utf-8")
    if isinstance(value, pb.TensorProto):
        return pb.to_array(value, base_dir)
    if isinstance(value, pb.GraphProto):
        raise ModelImportError(_CONTROL_FLOW)
    if isinstance(value, list):
        if value and isinstance(value[0], bytes):
            return [v.decode("utf-8") for v in value]
        if value and isinstance(value[0], pb.TensorProto):
            return [pb.to_array(v, base_dir) for v in value]
        if value and isinstance(value[0], pb.GraphProto):
            raise ModelImportError(_CONTROL_FLOW)
        return list(value)
    return value


def _constant_value(attrs: dict[str, Any]) -> np.ndarray:
    """The value of a Constant node from whichever attribute form it uses (onnx_import.py:50-61)."""
    forms = (("value", None), ("value_float", np.float32), ("value_floats", np.float32),
             ("value_int", np.int64), ("value_ints", np.int64))
    for key, dtype in forms:
        if key in attrs:
            return np.asarray(attrs[key], dtype=dtype)
    raise ModelImportError(f"unsupported Constant attributes {sorted(attrs)}")


def _input_type(info: pb.ValueInfoProto, input_shapes: dict[str, tuple[int, ...]],
                dims: dict[str, int]) -> TensorType:
    """Static type of a graph input (onnx_import.py:64-89): a whole shape from ``input_shapes``
    wins; otherwise each dimension is its dim_value or the ``dims`` binding of its dim_param."""
    if info.elem_type not in ELEM_TYPES:
        raise ModelImportError(f"input {info.name!r} has unsupported element type {info.elem_type}")
    dtype = ELEM_TYPES[info.elem_type]
    if info.name in input_shapes:
        return TensorType(dtype, tuple(int(d) for d in input_shapes[info.name]))
    shape: list[int] = []
    for d in info.shape or []:
        if d.dim_value is not None:
            shape.append(int(d.dim_value))
        elif d.dim_param and d.dim_param in dims:
            shape.append(int(dims[d.dim_param]))
        else:
            sym = d.dim_param or "?"
            raise ModelImportError(
                f"input {info.name!r} has a dynamic dimension {sym!r}; pass a value for it "
                f"(dims={{'{sym}': N}} or --dim {sym}=N) or a full input shape"
            )
    return TensorType(dtype, tuple(shape))


def opset_version(model: pb.ModelProto) -> int:
    """Version of the default ("" or "ai.onnx") operator set; 21 when the model names none."""
    for entry in model.opset_import:
        if entry.domain in ("", "ai.onnx"):
            return int(entry.version)
    return MAX_OPSET


def from_onnx(
    model: pb.ModelProto | str | Path | bytes,
    input_shapes: dict[str, tuple[int, ...]] | None = None,
    dims: dict[str, int] | None = None,
) -> Graph:
    """Import an ONNX model (a path, serialized bytes or a decoded ModelProto) into the IR and
    infer every static shape (onnx_import.py:99-170).

    ``input_shapes`` fixes whole input shapes by name; ``dims`` gives values to symbolic
    dimensions (for example ``{"batch": 1, "sequence": 128}``).
    """
    if not isinstance(model, pb.ModelProto):
        model = pb.load_model(model)
    shapes = dict(input_shapes or {})
    bindings = dict(dims or {})
    opset = opset_version(model)
    if not MIN_OPSET <= opset <= MAX_OPSET:
        raise ModelImportError(f"opset {opset} is outside the supported range {MIN_OPSET}..{MAX_OPSET}")
    proto = model.graph
    graph = Graph(proto.name or "model")
    env: dict[str, Value] = {}

    for init in proto.initializer:
        env[init.name] = graph.constant(pb.to_array(init, model.base_dir), init.name)
    for info in proto.input:
        if info.name not in env:  # IR < 4 files list initializers among the inputs
            env[info.name] = graph.add_input(info.name, _input_type(info, shapes, bindings))
    unknown = set(shapes) - {v.name for v in graph.inputs}
    if unknown:
        raise ModelImportError(f"input_shapes names unknown inputs: {sorted(unknown)}")

    for node in proto.node:
        if node.domain not in ("", "ai.onnx"):
            raise ModelImportError(f"operator domain {node.domain!r} ({node.op_type}) is not supported")
        attrs = {a.name: _attribute(a, model.base_dir) for a in node.attribute}
        if node.op_type == "Constant":
            env[node.output[0]] = graph.constant(_constant_value(attrs), node.output[0])
            continue
        if node.op_type in ("Softmax", "LogSoftmax", "Hardmax") and opset < 13:
            # before opset 13 these coerce the input to 2-D at ``axis`` (default 1); checked
            # once shapes are known
            attrs.setdefault("axis", 1)
            attrs["_legacy_coerce_2d"] = 1
        inputs: list[Value | None] = []
        for name in node.input:
            if not name:
                inputs.append(None)  # an omitted optional input
            elif name in env:
                inputs.append(env[name])
            else:
                raise ModelImportError(f"node {node.name!r} uses undefined value {name!r}")
        ir_node = graph.add_node(
            node.op_type, inputs, n_outputs=len(node.output), attrs=attrs, name=node.name,
            output_names=[o or f"{node.op_type.lower()}_unused" for o in node.output],
        )
        for name, value in zip(node.output, ir_node.outputs, strict=True):
            if name:
                env[name] = value

    for info in proto.output:
        if info.name not in env:
            raise ModelImportError(f"graph output {info.name!r} is never defined")
        graph.add_output(env[info.name], info.name)
    graph.opset = opset
    infer_shapes(graph)
    _resolve_legacy_softmax(graph)
    return graph


def _resolve_legacy_softmax(graph: Graph) -> None:
    """Opset < 13 Softmax/LogSoftmax/Hardmax flatten the input to 2-D around ``axis``; that is
    the modern (per-axis) operator only when ``axis`` is the last axis (onnx_import.py:173-186)."""
    for node in graph.nodes:
        if node.attrs.pop("_legacy_coerce_2d", None) is None:
            continue
        rank = node.input(0).tensor_type.rank
        axis = int(node.attrs["axis"])
        if (axis + rank if axis < 0 else axis) != rank - 1:
            raise UnsupportedOpError(
                f"{node.op} with opset < 13 over axis {axis} of a rank {rank} tensor "
                "(2-D coercion) is not supported"
            )
        node.attrs["axis"] = -1
