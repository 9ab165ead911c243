"""Declarative dataflow patterns, and the two subgraph recognizers built on them.

A pattern describes how a value was computed: ``Op("Div", a, b)`` matches a value produced by
a Div node whose inputs match ``a`` and ``b``; ``Any("x")`` matches any value and binds it to
the name ``x`` (a second ``Any("x")`` must then be the very same value); ``Num(2.0)`` matches a
one-element constant close to 2; ``Op(..., commutative=True)`` also tries the two inputs
swapped. A match returns the bindings (values by name, nodes by ``node=`` name) or None.

Recognized here, as the reference's fusion pass does (src/ml_graph_compiler/passes/fusion.py):

* the LayerNorm torch.onnx decomposes below opset 17 — ``(x - mean(x)) / sqrt(mean(d*d) + eps)``
  with ``d`` the centred value, means over the last axis with keepdims, ``d*d`` as Mul or
  ``Pow 2``, followed optionally by ``* gamma`` and ``+ beta`` with per-channel constants — into
  one LayerNormalization (every intermediate read once, ``d`` read only by the square and the
  division);
* the erf GELU (BERT) ``0.5 * x * (1 + erf(x / sqrt 2))`` and the tanh GELU (GPT-2)
  ``0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3)))``, in any of the three
  association orders of the final products, into one Gelu node.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .. import ops
from ..ir import Graph, Node, Value
from .cleanup import eliminate_dead_code
from .graph_tools import is_number, made_by, operand_with, other_operand, per_channel, place_before, sole_reader

Bindings = dict[str, object]


class Pattern:
    def match(self, value: Value | None, env: Bindings) -> Bindings | None:
        raise NotImplementedError


@dataclass
class Any(Pattern):
    """Any value (``constant``: must / must not be constant when set); binds ``name``."""

    name: str | None = None
    constant: bool | None = None

    def match(self, value: Value | None, env: Bindings) -> Bindings | None:
        if value is None or (self.constant is not None and value.is_constant != self.constant):
            return None
        if self.name is None:
            return env
        bound = env.get(self.name)
        if bound is not None:
            return env if bound is value else None
        return {**env, self.name: value}


@dataclass
class Num(Pattern):
    """A one-element constant near ``target`` (any one-element constant when None); binds
    its number to ``name``."""

    target: float | None = None
    name: str | None = None

    def match(self, value: Value | None, env: Bindings) -> Bindings | None:
        if value is None or value.data is None or value.data.size != 1:
            return None
        if self.target is not None and not is_number(value, self.target):
            return None
        return {**env, self.name: float(value.data.reshape(()))} if self.name else env


class Op(Pattern):
    """A value produced by one of ``ops`` whose inputs match ``args`` (leading inputs only
    when not ``exact_arity``)."""

    def __init__(self, ops: str | tuple[str, ...], *args: Pattern, commutative: bool = False, node: str | None = None,
                 exact_arity: bool = True):
        self.ops = (ops,) if isinstance(ops, str) else ops
        self.args, self.commutative, self.node, self.exact_arity = args, commutative, node, exact_arity

    def match(self, value: Value | None, env: Bindings) -> Bindings | None:
        producer = None if value is None else value.producer
        if producer is None or producer.op not in self.ops:
            return None
        if len(producer.inputs) < len(self.args) or (self.exact_arity and len(producer.inputs) != len(self.args)):
            return None
        orders = [self.args]
        if self.commutative and len(self.args) == 2:
            orders.append((self.args[1], self.args[0]))
        for order in orders:
            got: Bindings | None = env if self.node is None else {**env, self.node: producer}
            for pattern, operand in zip(order, producer.inputs):
                got = pattern.match(operand, got) if got is not None else None
            if got is not None:
                return got
        return None


class Either(Pattern):
    """The first of ``options`` that matches."""

    def __init__(self, *options: Pattern):
        self.options = options

    def match(self, value: Value | None, env: Bindings) -> Bindings | None:
        for option in self.options:
            got = option.match(value, env)
            if got is not None:
                return got
        return None


# ---------------------------------------------------------------------------------------------
# LayerNorm
# ---------------------------------------------------------------------------------------------
_CENTRED = Op("Sub", Any("x"), Op("ReduceMean", Any("x"), node="mean", exact_arity=False), node="sub")
_SQUARE = Either(Op("Mul", Any("d"), Any("d"), node="square"), Op("Pow", Any("d"), Num(2.0), node="square"))
_VARIANCE = Op("ReduceMean", _SQUARE, node="var_mean", exact_arity=False)
LAYER_NORM = Op("Div", Any("d"), Op("Sqrt", Op("Add", Any("var", constant=False), Num(name="eps"), commutative=True,
                                                   node="add"), node="sqrt"), node="div")


def _mean_over_last_axis(node: Node) -> bool:
    x = node.inputs[0]
    if x is None or x.type is None:
        return False
    try:
        axes = ops.reduce_axes(node, x.type.rank, [None if v is None else v.data for v in node.inputs])
    except Exception:
        return False
    return axes == (x.type.rank - 1,) and int(node.attrs.get("keepdims", 1)) == 1


def _affine_tail(graph: Graph, div: Node, dim: int) -> tuple[Node, np.ndarray | None, np.ndarray | None]:
    """The last node of ``div * gamma + beta`` (each step optional) and the two vectors."""
    tail, scale, shift = div, None, None
    for op in ("Mul", "Add"):
        reader = sole_reader(graph, tail.output)
        if reader is None or reader.op != op:
            continue
        vector = per_channel(other_operand(reader, tail.output), dim, 1)
        if vector is not None:
            if op == "Mul":
                scale = vector
            else:
                shift = vector
            tail = reader
    return tail, scale, shift


def _layer_norm_at(graph: Graph, div: Node) -> bool:
    m = LAYER_NORM.match(div.output, {})
    if m is None:
        return False
    d = m["d"]
    rest = _CENTRED.match(d, {})
    variance = _VARIANCE.match(m["var"], {"d": d}) if rest is not None else None
    if rest is None or variance is None:
        return False
    x = rest["x"]
    if not (_mean_over_last_axis(rest["mean"]) and _mean_over_last_axis(variance["var_mean"])):
        return False
    square = variance["square"]
    internal = [rest["mean"].output, square.output, m["var"], m["add"].output, m["sqrt"].output]
    if any(sole_reader(graph, v) is None for v in internal):
        return False
    if any(r is not square and r is not div for r in d.users) or any(d is o for o in graph.outputs):
        return False
    dim = x.tensor_type.shape[-1]
    tail, scale, shift = _affine_tail(graph, div, dim)
    if tail.output.type != x.type:
        return False
    gamma = graph.constant(scale if scale is not None else np.ones(dim, np.float32), "ln_gamma")
    beta = graph.constant(shift if shift is not None else np.zeros(dim, np.float32), "ln_beta")
    ln = place_before(graph, tail, "LayerNormalization", [x, gamma, beta], {"axis": -1, "epsilon": m["eps"]})
    graph.replace_all_uses(tail.output, ln.output)
    return True


def fuse_layer_norm(graph: Graph) -> int:
    found = 0
    for node in list(graph.nodes):
        if node.op == "Div" and node in graph.nodes and _layer_norm_at(graph, node):
            found += 1
    if found:
        eliminate_dead_code(graph)
    return found


# ---------------------------------------------------------------------------------------------
# GELU
# ---------------------------------------------------------------------------------------------
_ERF_ARGUMENT = Either(Op("Div", Any("x", constant=False), Num(math.sqrt(2.0))),
                       Op("Mul", Any("x", constant=False), Num(1.0 / math.sqrt(2.0)), commutative=True))
# x^3 as Pow(x, 3) or (x * x) * x in either order; its base must be the x added beside it
_CUBE = Either(Op("Pow", Any("x"), Num(3.0)),
               Op("Mul", Op("Mul", Any("x"), Any("x")), Any("x"), commutative=True))
_TANH_ARGUMENT = Op("Mul", Op("Add", Any("x"), Op("Mul", _CUBE, Num(0.044715), commutative=True), commutative=True),
                    Num(math.sqrt(2.0 / math.pi)), commutative=True)


def _gelu_input(node: Node) -> tuple[Value, str] | None:
    """(x, approximate) when ``node`` (an Erf or a Tanh) is the core of a GELU of x."""
    if node.op == "Erf":
        m = _ERF_ARGUMENT.match(node.input(0), {})
        return (m["x"], "none") if m is not None else None
    m = _TANH_ARGUMENT.match(node.input(0), {})
    return (m["x"], "tanh") if m is not None else None


def _gelu_end(graph: Graph, one_plus: Node, x: Value) -> Node | None:
    """The node computing ``0.5 * x * one_plus`` as (x * s) * 0.5, (0.5 * x) * s or
    (s * 0.5) * x."""
    product = sole_reader(graph, one_plus.output)
    if product is None or product.op != "Mul":
        return None
    partner = other_operand(product, one_plus.output)
    if partner is x:
        last = sole_reader(graph, product.output)
        return last if last is not None and operand_with(last, "Mul", 0.5) is product.output else None
    half = made_by(partner, "Mul")
    if half is not None and operand_with(half, "Mul", 0.5) is x and sole_reader(graph, half.output) is not None:
        return product
    if is_number(partner, 0.5):
        last = sole_reader(graph, product.output)
        if last is not None and last.op == "Mul" and any(v is x for v in last.inputs):
            return last
    return None


def _gelu_at(graph: Graph, core: Node) -> bool:
    found = _gelu_input(core)
    if found is None:
        return False
    x, approximate = found
    one_plus = sole_reader(graph, core.output)
    if one_plus is None or operand_with(one_plus, "Add", 1.0) is not core.output:
        return False
    end = _gelu_end(graph, one_plus, x)
    if end is None or end.output.type != x.type:
        return False
    gelu = place_before(graph, end, "Gelu", [x], {"approximate": approximate})
    graph.replace_all_uses(end.output, gelu.output)
    return True


def fuse_gelu(graph: Graph) -> int:
    found = 0
    for node in list(graph.nodes):
        if node.op in ("Erf", "Tanh") and node.output.users and _gelu_at(graph, node):
            found += 1
    if found:
        eliminate_dead_code(graph)
    return found
