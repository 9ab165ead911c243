"""Constant folding, dead-node removal and duplicate merging.

Behaviour of the reference's basic passes (src/ml_graph_compiler/passes/basic.py): folding
evaluates, in one forward sweep, every node whose present inputs are all constants (results
feed later nodes in the same sweep) and every Shape/Size of a typed value, except a 2-D
Transpose whose only readers take it as MatMul's right operand (fusion turns that pair into a
``trans_b`` GEMM) and results more than twice their inputs' size beyond 16 MiB; merging
deduplicates constants by content, then nodes by operator, inputs (in either order for
commutative binary operators), attributes and output count, again in one forward sweep.
"""

from __future__ import annotations

import hashlib
from typing import Any

import numpy as np

from .. import ops
from ..ir import Graph, Node, Value

FOLD_GROWTH_LIMIT_BYTES = 16 << 20
COMMUTATIVE = frozenset({"Add", "Mul", "Max", "Min", "Equal", "And", "Or", "Xor"})


def _feeds_gemm_weight(node: Node) -> bool:
    if node.op != "Transpose" or node.output.type is None or node.output.type.rank != 2:
        return False
    readers = node.output.users
    return bool(readers) and all(r.op == "MatMul" and r.inputs[1] is node.output for r in readers)


def _fold_values(node: Node) -> list[np.ndarray] | None:
    """Compile-time results of ``node``, or None when it is not folded."""
    if node.op in ops.SHAPE_ONLY_OPS:
        shape = node.input(0).tensor_type.shape
        folded = ops.shape_value(node, shape) if node.op == "Shape" else np.asarray(int(np.prod(shape, dtype=np.int64)))
        return [folded.astype(np.int64)]
    present = [v for v in node.inputs if v is not None]
    if not present or not all(v.is_constant for v in present) or _feeds_gemm_weight(node):
        return None
    read = sum(v.data.nbytes for v in present)
    written = sum(v.type.nbytes for v in node.outputs if v.type is not None)
    if written > max(2 * read, FOLD_GROWTH_LIMIT_BYTES):
        return None
    return ops.run(node, [None if v is None else v.data for v in node.inputs])


def fold_constants(graph: Graph) -> int:
    """Replace foldable nodes by constants; returns how many nodes were folded."""
    gone: list[Node] = []
    for node in graph.nodes:
        results = _fold_values(node)
        if results is None:
            continue
        for value, data in zip(node.outputs, results, strict=True):
            graph.replace_all_uses(value, graph.constant(data, value.name + "_folded"))
        gone.append(node)
    return graph.remove_nodes(gone)


def eliminate_dead_code(graph: Graph) -> int:
    """Remove the nodes no graph output depends on; returns how many."""
    needed = {id(v) for v in graph.outputs}
    alive: set[int] = set()
    for node in reversed(graph.nodes):
        if any(id(o) in needed for o in node.outputs):
            alive.add(id(node))
            needed.update(id(v) for v in node.inputs if v is not None)
    return graph.remove_nodes(n for n in graph.nodes if id(n) not in alive)


def _hashable(item: Any) -> Any:
    """A hashable, content-based key for attribute values and constant arrays."""
    if isinstance(item, np.ndarray):
        return ("array", item.dtype.str, item.shape, hashlib.sha1(item.tobytes()).hexdigest())
    if isinstance(item, dict):
        return tuple(sorted((k, _hashable(v)) for k, v in item.items()))
    if isinstance(item, (list, tuple)):
        return tuple(_hashable(v) for v in item)
    return item


def _node_key(node: Node) -> tuple:
    operands = [None if v is None else id(v) for v in node.inputs]
    if node.op in COMMUTATIVE and len(operands) == 2:
        operands.sort(key=lambda k: -1 if k is None else k)
    return node.op, tuple(operands), _hashable(node.attrs), len(node.outputs)


def eliminate_common_subexpressions(graph: Graph) -> int:
    """Merge equal constants, then identical nodes; returns the number of merges."""
    merged = 0
    first_with: dict[Any, Value] = {}
    for const in graph.constants():
        kept = first_with.setdefault(_hashable(const.data), const)
        if kept is not const:
            graph.replace_all_uses(const, kept)
            merged += 1
    first_node: dict[tuple, Node] = {}
    repeats: list[Node] = []
    for node in graph.nodes:
        key = _node_key(node)
        kept_node = first_node.setdefault(key, node)
        if kept_node is node:
            continue
        for dup, orig in zip(node.outputs, kept_node.outputs, strict=True):
            graph.replace_all_uses(dup, orig)
        repeats.append(node)
    return merged + graph.remove_nodes(repeats)
