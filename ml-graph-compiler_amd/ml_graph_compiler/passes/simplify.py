"""Algebraic simplification and canonicalization.

Reference: src/ml_graph_compiler/passes/simplify.py:1-190. Rewrites, each value-preserving up
to float32 rounding:

* Identity, Dropout (mask unused), same-type Cast, same-shape Expand/Slice/Tile/Pad (all-zero
  pads), single-input Concat: bypassed.
* x + 0, x - 0, x * 1, x / 1, x ^ 1 (and 0 + x, 1 * x) when broadcasting keeps x's type.
* x ^ 2 -> x * x, x ^ 3 -> x * x * x, x ^ 0.5 -> sqrt(x); x / c -> x * (1 / c) for float c != 0.
* Flatten/Squeeze/Unsqueeze/Reshape -> one Reshape with a static ``shape``; reshape chains
  collapse and reshapes to the same shape vanish.
* Transpose(Transpose(x)) composes; an identity permutation vanishes; a Transpose that only
  moves size-1 dims becomes a Reshape.
"""

from __future__ import annotations

import numpy as np

from .. import ops
from ..ir import Graph, Node, Value
from .basic import eliminate_dead_code
from .util import insert_node, is_scalar

RESHAPE_LIKE = frozenset({"Reshape", "Flatten", "Squeeze", "Unsqueeze"})
_NEUTRAL = {"Add": 0.0, "Sub": 0.0, "Mul": 1.0, "Div": 1.0, "Pow": 1.0}


def _bypass(graph: Graph, node: Node, value: Value) -> bool:
    if value.type != node.outputs[0].type:
        return False
    graph.replace_all_uses(node.outputs[0], value)
    return True


def _identity(graph: Graph, node: Node) -> bool:
    op = node.op
    if op == "Identity" or (op == "Dropout" and not any(o.users for o in node.outputs[1:])):
        return _bypass(graph, node, node.input(0))
    x = node.inputs[0] if node.inputs else None
    if x is None:
        return False
    if op == "Cast" and x.type is not None and x.type == node.output.type:
        return _bypass(graph, node, x)
    if op in ("Expand", "Slice", "Tile", "Pad") and x.type == node.output.type:
        if op == "Pad":
            rank = x.tensor_type.rank
            pads = ops.pad_amounts(node, rank, [None if v is None else v.data for v in node.inputs])
            if pads != [0] * (2 * rank):
                return False
        return _bypass(graph, node, x)
    if op == "Concat" and sum(v is not None for v in node.inputs) == 1:
        return _bypass(graph, node, x)
    if op in _NEUTRAL and len(node.inputs) == 2:
        a, b = node.inputs
        neutral = _NEUTRAL[op]
        if a is not None and b is not None and b.data is not None and np.all(b.data == neutral):
            if _bypass(graph, node, a):
                return True
        if (
            op in ("Add", "Mul")
            and a is not None
            and b is not None
            and a.data is not None
            and np.all(a.data == neutral)
            and _bypass(graph, node, b)
        ):
            return True
    return False


def _strength(graph: Graph, node: Node) -> bool:
    if len(node.inputs) != 2:
        return False
    x, c = node.inputs
    if x is None or c is None or x.is_constant or x.type is None:
        return False
    if not np.issubdtype(np.dtype(x.type.dtype), np.floating):
        return False
    out = node.output
    if out.type != x.type:
        return False
    if node.op == "Pow":
        if is_scalar(c, 2.0):
            new = insert_node(graph, "Mul", [x, x], node).output
        elif is_scalar(c, 3.0):
            square = insert_node(graph, "Mul", [x, x], node).output
            new = insert_node(graph, "Mul", [square, x], node).output
        elif is_scalar(c, 0.5):
            new = insert_node(graph, "Sqrt", [x], node).output
        else:
            return False
        graph.replace_all_uses(out, new)
        return True
    if node.op == "Div" and c.data is not None and np.issubdtype(c.data.dtype, np.floating):
        if np.any(c.data == 0):
            return False
        recip = graph.constant((1.0 / c.data).astype(c.data.dtype), c.name + "_recip")
        graph.replace_all_uses(out, insert_node(graph, "Mul", [x, recip], node).output)
        return True
    return False


def _reshape(graph: Graph, node: Node) -> bool:
    if node.op not in RESHAPE_LIKE:
        return False
    x, out = node.input(0), node.output
    if out.type is None or x.type is None:
        return False
    if x.type.shape == out.type.shape:
        return _bypass(graph, node, x)
    source = x
    while source.producer is not None and source.producer.op == "Reshape" and "shape" in source.producer.attrs:
        source = source.producer.input(0)
    canonical = (
        node.op == "Reshape"
        and "shape" in node.attrs
        and sum(v is not None for v in node.inputs) == 1
    )
    if canonical and source is x:
        return False
    if source.type is not None and source.type.shape == out.type.shape:
        return _bypass(graph, node, source)
    new = insert_node(graph, "Reshape", [source], node, attrs={"shape": list(out.type.shape)})
    graph.replace_all_uses(out, new.output)
    return True


def _transpose(graph: Graph, node: Node) -> bool:
    if node.op != "Transpose":
        return False
    x = node.input(0)
    if x.type is None or node.output.type is None:
        return False
    perm = ops.transpose_perm(node, x.type.rank)
    if perm == list(range(len(perm))):
        return _bypass(graph, node, x)
    inner = x.producer
    if inner is not None and inner.op == "Transpose":
        first = ops.transpose_perm(inner, inner.input(0).tensor_type.rank)
        composed = [first[p] for p in perm]
        src = inner.input(0)
        if composed == list(range(len(composed))):
            return _bypass(graph, node, src)
        new = insert_node(graph, "Transpose", [src], node, attrs={"perm": composed})
        graph.replace_all_uses(node.output, new.output)
        return True
    moving = [p for p in perm if x.type.shape[p] != 1]
    if moving == sorted(moving):
        new = insert_node(graph, "Reshape", [x], node, attrs={"shape": list(node.output.type.shape)})
        graph.replace_all_uses(node.output, new.output)
        return True
    return False


RULES = (_identity, _strength, _reshape, _transpose)


def simplify(graph: Graph, max_rounds: int = 10) -> int:
    """Apply the rewrites to a fixed point (at most max_rounds sweeps)."""
    total = 0
    for _ in range(max_rounds):
        changed = 0
        for node in list(graph.nodes):
            if not any(o.users or o in graph.outputs for o in node.outputs):
                continue
            for rule in RULES:
                if rule(graph, node):
                    changed += 1
                    break
        if changed:
            eliminate_dead_code(graph)
        total += changed
        if not changed:
            break
    return total
