"""Static shape and type inference (reference: src/ml_graph_compiler/shape_inference.py:1-56).

Shape arithmetic (Shape -> Gather -> Concat -> Reshape) produces tiny int64 tensors; their
values are computed during inference (up to KNOWN_VALUE_LIMIT elements) so that operators whose
output shape depends on a tensor value (Reshape, Expand, Slice, Range, ...) can be typed.
"""

from __future__ import annotations

import numpy as np

from . import ops
from .errors import ShapeError
from .ir import Graph, Node, TensorType, Value

KNOWN_VALUE_LIMIT = 1 << 16


def _value_of(value: Value | None, known: dict[int, np.ndarray]) -> np.ndarray | None:
    if value is None:
        return None
    return value.data if value.data is not None else known.get(id(value))


def infer_node(node: Node, known: dict[int, np.ndarray] | None = None) -> list[TensorType]:
    """Type one node's outputs; remember small output values that can be computed now."""
    if known is None:
        known = {}
    in_types = [None if v is None else v.type for v in node.inputs]
    in_values = [_value_of(v, known) for v in node.inputs]
    try:
        out_types = ops.infer(node, in_types, in_values)
    except ShapeError as exc:
        raise ShapeError(f"{node.op} node {node.name!r}: {exc}") from exc
    for v, t in zip(node.outputs, out_types, strict=True):
        v.type = t
    small = all(t.size <= KNOWN_VALUE_LIMIT for t in out_types)
    if not small:
        return out_types
    if node.op in ops.SHAPE_ONLY_OPS:
        x = node.input(0).tensor_type
        if node.op == "Shape":
            known[id(node.output)] = ops.shape_value(node, x.shape)
        else:
            known[id(node.output)] = np.asarray(x.size, np.int64)
    elif all(c is not None for c, v in zip(in_values, node.inputs) if v is not None):
        for v, array in zip(node.outputs, ops.run(node, in_values), strict=True):
            known[id(v)] = array
    return out_types


def infer_shapes(graph: Graph) -> None:
    """Type every value of a graph whose nodes are in topological order."""
    known: dict[int, np.ndarray] = {}
    for node in graph.nodes:
        infer_node(node, known)
    for v in graph.outputs:
        if v.type is None:
            raise ShapeError(f"graph output {v.name!r} has no type")
