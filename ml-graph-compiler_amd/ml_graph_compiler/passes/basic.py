"""Constant folding, dead code elimination, common subexpression elimination.

Reference: src/ml_graph_compiler/passes/basic.py:1-108.
"""

from __future__ import annotations

import hashlib
from typing import Any

import numpy as np

from .. import ops
from ..ir import Graph, Node

# Folding may not grow the constant data by more than this unless the result is small.
FOLD_GROWTH_LIMIT_BYTES = 16 << 20


def _transpose_kept_for_gemm(node: Node) -> bool:
    """A 2-D Transpose feeding only MatMul right operands stays: fusion turns each pair into a
    FusedGemm with trans_b, so no transposed copy of the weight is stored."""
    if node.op != "Transpose" or node.output.type is None or node.output.type.rank != 2:
        return False
    users = node.output.users
    return bool(users) and all(u.op == "MatMul" and u.inputs[1] is node.output for u in users)


def fold_constants(graph: Graph) -> int:
    """Replace nodes whose inputs are all constants (and Shape/Size of typed values) by their
    values. Returns the number of nodes removed."""
    folded: list[Node] = []
    for node in graph.nodes:
        present = [v for v in node.inputs if v is not None]
        if node.op in ops.SHAPE_ONLY_OPS:
            x = node.input(0).tensor_type
            value = ops.shape_value(node, x.shape) if node.op == "Shape" else np.asarray(x.size)
            results = [value.astype(np.int64)]
        elif present and all(v.is_constant for v in present):
            if _transpose_kept_for_gemm(node):
                continue
            in_bytes = sum(v.data.nbytes for v in present if v.data is not None)
            out_bytes = sum(v.tensor_type.nbytes for v in node.outputs if v.type is not None)
            if out_bytes > max(2 * in_bytes, FOLD_GROWTH_LIMIT_BYTES):
                continue
            results = ops.run(node, [None if v is None else v.data for v in node.inputs])
        else:
            continue
        for out, data in zip(node.outputs, results, strict=True):
            graph.replace_all_uses(out, graph.constant(data, out.name + "_folded"))
        folded.append(node)
    graph.remove_nodes(folded)
    return len(folded)


def eliminate_dead_code(graph: Graph) -> int:
    """Remove every node that does not contribute to a graph output."""
    live = {id(v) for v in graph.outputs}
    kept: set[int] = set()
    for node in reversed(graph.nodes):
        if any(id(o) in live for o in node.outputs):
            kept.add(id(node))
            live.update(id(v) for v in node.inputs if v is not None)
    return graph.remove_nodes([n for n in graph.nodes if id(n) not in kept])


def _key(value: Any) -> Any:
    """Hashable structural key of an attribute value (arrays by dtype, shape and content)."""
    if isinstance(value, np.ndarray):
        return ("nd", value.dtype.str, value.shape, hashlib.sha1(value.tobytes()).hexdigest())
    if isinstance(value, (list, tuple)):
        return tuple(_key(v) for v in value)
    if isinstance(value, dict):
        return tuple(sorted((k, _key(v)) for k, v in value.items()))
    return value


COMMUTATIVE = frozenset({"Add", "Mul", "Max", "Min", "Equal", "And", "Or", "Xor"})


def eliminate_common_subexpressions(graph: Graph) -> int:
    """Merge equal constants, then nodes with equal operator, attributes and inputs."""
    merged = 0
    first_by_content: dict[Any, Any] = {}
    for value in list(graph.constants()):
        assert value.data is not None
        first = first_by_content.setdefault(_key(value.data), value)
        if first is not value:
            graph.replace_all_uses(value, first)
            merged += 1
    seen: dict[Any, Node] = {}
    duplicates: list[Node] = []
    for node in graph.nodes:
        ids = [None if v is None else id(v) for v in node.inputs]
        if node.op in COMMUTATIVE and len(ids) == 2:
            ids = sorted(ids, key=lambda k: -1 if k is None else k)
        key = (node.op, tuple(ids), _key(node.attrs), len(node.outputs))
        original = seen.get(key)
        if original is None:
            seen[key] = node
            continue
        for old, new in zip(node.outputs, original.outputs, strict=True):
            graph.replace_all_uses(old, new)
        duplicates.append(node)
    graph.remove_nodes(duplicates)
    return merged + len(duplicates)
