"""Algebraic simplification: a table of local rewrite rules applied to a fixed point.

The rules and their precedence are the reference's (src/ml_graph_compiler/passes/simplify.py);
each keeps the computed values up to float32 rounding:

1. pass-through — Identity, Dropout whose mask is unread, Cast to the same type, Expand /
   Slice / Tile / Pad that do not change the type (Pad with all-zero pads), single-input
   Concat, ``x + 0``, ``x - 0``, ``x * 1``, ``x / 1``, ``x ^ 1`` (and ``0 + x``, ``1 * x``), when
   the result has ``x``'s type;
2. strength reduction on floats — ``x ^ 2`` -> ``x * x``, ``x ^ 3`` -> ``(x * x) * x``,
   ``x ^ 0.5`` -> ``sqrt(x)``, ``x / c`` -> ``x * (1 / c)`` for a float constant without zeros;
3. reshapes — Flatten / Squeeze / Unsqueeze / Reshape become one ``Reshape`` with a static
   ``shape`` attribute reading the first non-Reshape source; same-shape reshapes vanish;
4. transposes — two in a row compose (or cancel); one that moves only size-1 axes becomes a
   Reshape.

One sweep visits the nodes present at its start (skipping dead ones) and applies the first rule
that fires; sweeps repeat (at most ``max_rounds``) until none fires.
"""

from __future__ import annotations

from collections.abc import Callable

import numpy as np

from .. import ops
from ..ir import Graph, Node, Value
from .cleanup import eliminate_dead_code
from .graph_tools import in_use, is_number, place_before, substitute

RESHAPES = frozenset({"Reshape", "Flatten", "Squeeze", "Unsqueeze"})
# operator -> the constant operand value that makes it a no-op
NEUTRAL = {"Add": 0.0, "Sub": 0.0, "Mul": 1.0, "Div": 1.0, "Pow": 1.0}


def _forward(graph: Graph, node: Node, value: Value | None) -> bool:
    """Readers of ``node``'s output read ``value`` instead, when the types agree."""
    if value is None or value.type != node.outputs[0].type:
        return False
    graph.replace_all_uses(node.outputs[0], value)
    return True


def _all_equal(value: Value | None, number: float) -> bool:
    return value is not None and value.data is not None and bool(np.all(value.data == number))


def _pass_through(graph: Graph, node: Node) -> bool:
    op = node.op
    if op == "Identity" or (op == "Dropout" and not any(o.users for o in node.outputs[1:])):
        return _forward(graph, node, node.input(0))
    x = node.inputs[0] if node.inputs else None
    if x is None:
        return False
    same_type = x.type is not None and x.type == node.output.type
    if op == "Cast" and same_type:
        return _forward(graph, node, x)
    if op in ("Expand", "Slice", "Tile", "Pad") and x.type == node.output.type:
        if op == "Pad":
            rank = x.tensor_type.rank
            if any(ops.pad_amounts(node, rank, [None if v is None else v.data for v in node.inputs])):
                return False
        return _forward(graph, node, x)
    if op == "Concat" and sum(v is not None for v in node.inputs) == 1:
        return _forward(graph, node, x)
    if op in NEUTRAL and len(node.inputs) == 2:
        a, b = node.inputs
        if a is not None and b is not None:
            if _all_equal(b, NEUTRAL[op]) and _forward(graph, node, a):
                return True
            if op in ("Add", "Mul") and _all_equal(a, NEUTRAL[op]) and _forward(graph, node, b):
                return True
    return False


def _strength_reduce(graph: Graph, node: Node) -> bool:
    if node.op not in ("Pow", "Div") or len(node.inputs) != 2:
        return False
    x, c = node.inputs
    if x is None or c is None or x.is_constant or x.type is None:
        return False
    if not np.issubdtype(np.dtype(x.type.dtype), np.floating) or node.output.type != x.type:
        return False
    if node.op == "Pow":
        if is_number(c, 2.0):
            substitute(graph, node, "Mul", [x, x])
        elif is_number(c, 3.0):
            square = place_before(graph, node, "Mul", [x, x]).output
            substitute(graph, node, "Mul", [square, x])
        elif is_number(c, 0.5):
            substitute(graph, node, "Sqrt", [x])
        else:
            return False
        return True
    divisor = c.data
    if divisor is None or not np.issubdtype(divisor.dtype, np.floating) or np.any(divisor == 0):
        return False
    inverse = graph.constant((1.0 / divisor).astype(divisor.dtype), c.name + "_recip")
    substitute(graph, node, "Mul", [x, inverse])
    return True


def _canonical_reshape(graph: Graph, node: Node) -> bool:
    if node.op not in RESHAPES:
        return False
    x, out = node.input(0), node.output
    if x.type is None or out.type is None:
        return False
    if x.type.shape == out.type.shape:
        return _forward(graph, node, x)
    origin = x
    while origin.producer is not None and origin.producer.op == "Reshape" and "shape" in origin.producer.attrs:
        origin = origin.producer.input(0)
    already = node.op == "Reshape" and "shape" in node.attrs and sum(v is not None for v in node.inputs) == 1
    if already and origin is x:
        return False
    if origin.type is not None and origin.type.shape == out.type.shape:
        return _forward(graph, node, origin)
    substitute(graph, node, "Reshape", [origin], {"shape": list(out.type.shape)})
    return True


def _transposes(graph: Graph, node: Node) -> bool:
    if node.op != "Transpose":
        return False
    x = node.input(0)
    if x.type is None or node.output.type is None:
        return False
    perm = ops.transpose_perm(node, x.type.rank)
    if perm == sorted(perm):
        return _forward(graph, node, x)
    first = x.producer
    if first is not None and first.op == "Transpose":
        inner = ops.transpose_perm(first, first.input(0).tensor_type.rank)
        both = [inner[p] for p in perm]
        if both == sorted(both):
            return _forward(graph, node, first.input(0))
        substitute(graph, node, "Transpose", [first.input(0)], {"perm": both})
        return True
    moved = [p for p in perm if x.type.shape[p] != 1]
    if moved != sorted(moved):
        return False
    substitute(graph, node, "Reshape", [x], {"shape": list(node.output.type.shape)})
    return True


RULES: tuple[Callable[[Graph, Node], bool], ...] = (_pass_through, _strength_reduce, _canonical_reshape, _transposes)


def simplify(graph: Graph, max_rounds: int = 10) -> int:
    """Apply RULES until nothing changes; returns the number of rewrites."""
    total = 0
    for _ in range(max_rounds):
        fired = sum(1 for node in list(graph.nodes)
                    if in_use(graph, node) and any(rule(graph, node) for rule in RULES))
        if not fired:
            break
        eliminate_dead_code(graph)
        total += fired
    return total
