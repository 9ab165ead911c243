"""Static types for every value, with small shape computations evaluated along the way.

Reference behaviour: src/ml_graph_compiler/shape_inference.py. ONNX exporters compute shapes
at run time (Shape -> Gather -> Concat -> Reshape); here those int64 tensors are small and fully
determined by the static input shapes, so while walking the nodes in order the pass keeps the
value of every output of at most KNOWN_VALUE_LIMIT elements whose inputs are all known, and
hands those values to the shape rules of the operators that need them (Reshape, Expand, Slice,
Range, ...).
"""

from __future__ import annotations

import numpy as np

from . import ops
from .errors import ShapeError
from .ir import Graph, Node, TensorType, Value

KNOWN_VALUE_LIMIT = 1 << 16


class _KnownValues:
    """Values known at compile time: constants, plus small results computed during the walk."""

    def __init__(self, table: dict[int, np.ndarray] | None = None):
        self.table = {} if table is None else table

    def of(self, value: Value | None) -> np.ndarray | None:
        if value is None:
            return None
        return value.data if value.data is not None else self.table.get(id(value))

    def learn(self, node: Node, inputs: list[np.ndarray | None], out_types: list[TensorType]) -> None:
        if any(t.size > KNOWN_VALUE_LIMIT for t in out_types):
            return
        if node.op in ops.SHAPE_ONLY_OPS:  # the value follows from the input's type
            x = node.input(0).tensor_type
            self.table[id(node.output)] = (ops.shape_value(node, x.shape) if node.op == "Shape"
                                           else np.asarray(x.size, np.int64))
            return
        if all(known is not None for known, v in zip(inputs, node.inputs) if v is not None):
            for value, array in zip(node.outputs, ops.run(node, inputs), strict=True):
                self.table[id(value)] = array


def infer_node(node: Node, known: dict[int, np.ndarray] | None = None) -> list[TensorType]:
    """Set the output types of one node (and record its small known outputs in ``known``)."""
    values = _KnownValues(known)
    inputs = [values.of(v) for v in node.inputs]
    try:
        out_types = ops.infer(node, [None if v is None else v.type for v in node.inputs], inputs)
    except ShapeError as exc:
        raise ShapeError(f"{node.op} node {node.name!r}: {exc}") from exc
    for value, t in zip(node.outputs, out_types, strict=True):
        value.type = t
    values.learn(node, inputs, out_types)
    return out_types


def infer_shapes(graph: Graph) -> None:
    """Type every value; the nodes must already be in topological order."""
    known: dict[int, np.ndarray] = {}
    for node in graph.nodes:
        infer_node(node, known)
    untyped = next((v for v in graph.outputs if v.type is None), None)
    if untyped is not None:
        raise ShapeError(f"graph output {untyped.name!r} has no type")
