"""Operator table: output types and compile-time evaluation of every operator.

Each operator is one ``OpDef`` record in ``REGISTRY``: a shape rule (input types, plus the
values of constant inputs, to output types) and an evaluator (numpy arrays to numpy arrays).
Shape inference, constant folding and the passes all read this one table. The records are
generated from operator families — elementwise arithmetic, predicates, unary maps, data
movement, reductions, normalization, contractions, windows — rather than written out one by
one.

The semantics are the reference's (src/ml_graph_compiler/ops.py: ONNX opsets 7-21 plus the
compiler's own FusedGemm, FusedConv, FusedElementwise and Gelu): results take the first
operand's dtype, integer Div truncates toward zero, Pow converts the exponent to the base's
dtype, erf is the rational approximation below, LayerNormalization runs in float64, ArgMax
returns the first maximum, Gather wraps negative indices. The error messages are the
reference's, since callers match on them.
"""

from __future__ import annotations

import math
from collections.abc import Callable, Sequence
from dataclasses import dataclass
from typing import Any

import numpy as np

from .errors import ShapeError, UnsupportedOpError
from .ir import Node, TensorType, Value, contiguous, dtype_name

Arrays = list[np.ndarray | None]
Types = list[TensorType | None]
ShapeRule = Callable[["Node", "_Static"], list[TensorType]]
Evaluator = Callable[["Node", "_Dynamic"], list[np.ndarray]]

ACTIVATIONS = ("none", "relu", "clip", "gelu", "gelu_tanh", "tanh", "sigmoid")
# operators whose output value follows from the input types alone
SHAPE_ONLY_OPS = frozenset({"Shape", "Size"})


@dataclass(frozen=True)
class OpDef:
    name: str
    shape_rule: ShapeRule
    evaluate: Evaluator
    elementwise: bool = False

    def infer(self, node: Node, types: Types, consts: Arrays) -> list[TensorType]:
        return self.shape_rule(node, _Static(types, consts))

    def run(self, node: Node, arrays: Arrays) -> list[np.ndarray]:
        return self.evaluate(node, _Dynamic(arrays))


REGISTRY: dict[str, OpDef] = {}


def _define(name: str, shape_rule: ShapeRule, evaluate: Evaluator, elementwise: bool = False) -> None:
    REGISTRY[name] = OpDef(name, shape_rule, evaluate, elementwise)


def spec(op: str) -> OpDef:
    found = REGISTRY.get(op)
    if found is None:
        raise UnsupportedOpError(f"operator {op!r} is not supported")
    return found


def supported_ops() -> list[str]:
    return sorted(REGISTRY)


def is_elementwise(op: str) -> bool:
    found = REGISTRY.get(op)
    return found is not None and found.elementwise


def infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    """Output types of ``node``; trailing outputs the node does not have are dropped."""
    out = spec(node.op).infer(node, types, consts)
    if len(out) < len(node.outputs):
        raise ShapeError(f"{node.op}: inferred {len(out)} outputs, node has {len(node.outputs)}")
    return out[: len(node.outputs)]


def run(node: Node, arrays: Arrays) -> list[np.ndarray]:
    """Evaluate ``node`` on numpy arrays (constant folding, shape arithmetic)."""
    return spec(node.op).run(node, arrays)


# ---------------------------------------------------------------------------------------------
# operand access
# ---------------------------------------------------------------------------------------------
class _Static:
    """Operands seen by a shape rule: input types, and the arrays of constant inputs."""

    __slots__ = ("types", "consts")

    def __init__(self, types: Types, consts: Arrays):
        self.types, self.consts = list(types), list(consts)

    def t(self, i: int) -> TensorType:
        found = self.types[i] if i < len(self.types) else None
        if found is None:
            raise ShapeError(f"missing type for input {i}")
        return found

    def c(self, i: int, what: str) -> np.ndarray:
        found = self.consts[i] if i < len(self.consts) else None
        if found is None:
            raise ShapeError(f"{what} must be a constant (static shapes are required)")
        return found

    def maybe(self, i: int) -> np.ndarray | None:
        return self.consts[i] if i < len(self.consts) else None

    def present(self) -> list[TensorType]:
        return [t for t in self.types if t is not None]


class _Dynamic:
    """Operands seen by an evaluator: input arrays, None for an omitted optional input."""

    __slots__ = ("arrays",)

    def __init__(self, arrays: Arrays):
        self.arrays = list(arrays)

    def a(self, i: int) -> np.ndarray:
        found = self.arrays[i] if i < len(self.arrays) else None
        if found is None:
            raise UnsupportedOpError(f"missing input {i}")
        return found

    def maybe(self, i: int) -> np.ndarray | None:
        return self.arrays[i] if i < len(self.arrays) else None

    # shape helpers evaluate the same arguments as the shape rules
    c = maybe


def _like(x: Any, ref: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=ref.dtype)


def _as_ints(values: Any) -> list[int]:
    return [int(v) for v in np.asarray(values).reshape(-1)]


def _axis(axis: int, rank: int) -> int:
    wrapped = axis + rank if axis < 0 else axis
    if wrapped < 0 or wrapped >= max(rank, 1):
        raise ShapeError(f"axis {axis} out of range for rank {rank}")
    return wrapped


def _prod(dims: Sequence[int]) -> int:
    return int(np.prod(dims, dtype=np.int64))


def _first(node: Node, ins: _Static) -> list[TensorType]:
    return [ins.t(0)]


def _broadcast_shape(node: Node, ins: _Static) -> tuple[int, ...]:
    shapes = [t.shape for t in ins.present()]
    try:
        return tuple(int(d) for d in np.broadcast_shapes(*shapes))
    except ValueError as exc:
        raise ShapeError(f"{node.op}: shapes do not broadcast: {shapes}") from exc


# ---------------------------------------------------------------------------------------------
# elementwise families
# ---------------------------------------------------------------------------------------------
def _divide(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    if np.issubdtype(a.dtype, np.integer):
        return np.trunc(a / b)  # C semantics: toward zero
    return a / b


def _power(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.power(a, b.astype(a.dtype))


# binary, broadcasting, result in the first operand's dtype
_ARITHMETIC: dict[str, Callable[[np.ndarray, np.ndarray], Any]] = {
    "Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": _divide, "Pow": _power,
    "Max": np.maximum, "Min": np.minimum,
}
# binary, broadcasting, bool result
_PREDICATES: dict[str, Callable[[np.ndarray, np.ndarray], Any]] = {
    "Equal": np.equal, "Less": np.less, "Greater": np.greater, "LessOrEqual": np.less_equal,
    "GreaterOrEqual": np.greater_equal, "And": np.logical_and, "Or": np.logical_or, "Xor": np.logical_xor,
}

# erf(x) ~ x P(x^2) / Q(x^2) on [-4, 4] (a public rational approximation, absolute error ~1e-7)
ERF_P = (-2.72614225801306e-10, 2.77068142495902e-08, -2.10102402082508e-06, -5.69250639462346e-05,
         -7.34990630326855e-04, -2.95459980854025e-03, -1.60960333262415e-02)
ERF_Q = (-1.45660718464996e-05, -2.13374055278905e-04, -1.68282697438203e-03, -7.37332916720468e-03,
         -1.42647390514189e-02)


def _horner(coefficients: Sequence[float], z: np.ndarray) -> np.ndarray:
    acc = np.full_like(z, coefficients[0])
    for c in coefficients[1:]:
        acc = acc * z + c
    return acc


def erf(x: np.ndarray) -> np.ndarray:
    t = np.clip(np.asarray(x, dtype=np.float64), -4.0, 4.0)
    z = t * t
    return np.asarray(t * _horner(ERF_P, z) / _horner(ERF_Q, z), dtype=np.asarray(x).dtype)


def gelu(x: np.ndarray, approximate: str = "none") -> np.ndarray:
    if approximate == "tanh":
        inner = math.sqrt(2.0 / math.pi) * (x + 0.044715 * x * x * x)
        return _like(0.5 * x * (1.0 + np.tanh(inner)), x)
    return _like(0.5 * x * (1.0 + erf(x / math.sqrt(2.0))), x)


def sigmoid(x: np.ndarray) -> np.ndarray:
    return _like(0.5 * (1.0 + np.tanh(0.5 * x)), x)


def clip_bounds(node: Node, xs: Sequence[np.ndarray | None]) -> tuple[float, float]:
    """Clip's (lo, hi): optional inputs 1 and 2 (opset >= 11) over the min/max attributes."""
    bounds = [node.attrs.get("min", -np.inf), node.attrs.get("max", np.inf)]
    for k in (0, 1):
        given = xs[k + 1] if len(xs) > k + 1 else None
        if given is not None:
            bounds[k] = float(np.asarray(given).reshape(()))
    return float(bounds[0]), float(bounds[1])


# unary maps: fn(x, node, operands) -> array, result in x's dtype
_UNARY: dict[str, Callable[[np.ndarray, Node, _Dynamic], Any]] = {
    "Relu": lambda x, n, o: np.maximum(x, 0),
    "Sigmoid": lambda x, n, o: sigmoid(x),
    "Tanh": lambda x, n, o: np.tanh(x),
    "Erf": lambda x, n, o: erf(x),
    "Sqrt": lambda x, n, o: np.sqrt(x),
    "Exp": lambda x, n, o: np.exp(x),
    "Log": lambda x, n, o: np.log(x),
    "Neg": lambda x, n, o: np.negative(x),
    "Abs": lambda x, n, o: np.abs(x),
    "Reciprocal": lambda x, n, o: np.reciprocal(x),
    "Floor": lambda x, n, o: np.floor(x),
    "Ceil": lambda x, n, o: np.ceil(x),
    "Sin": lambda x, n, o: np.sin(x),
    "Cos": lambda x, n, o: np.cos(x),
    "Softplus": lambda x, n, o: np.logaddexp(0, x),
    "Identity": lambda x, n, o: x.copy(),
    "Gelu": lambda x, n, o: gelu(x, str(n.attrs.get("approximate", "none"))),
    "LeakyRelu": lambda x, n, o: np.where(x >= 0, x, float(n.attrs.get("alpha", 0.01)) * x),
    "HardSigmoid": lambda x, n, o: np.clip(float(n.attrs.get("alpha", 0.2)) * x + float(n.attrs.get("beta", 0.5)), 0, 1),
    "Clip": lambda x, n, o: np.clip(x, *clip_bounds(n, o.arrays)),
}


def _arith_family(fn: Callable[[np.ndarray, np.ndarray], Any]) -> tuple[ShapeRule, Evaluator]:
    def shape_rule(node: Node, ins: _Static) -> list[TensorType]:
        return [TensorType(ins.present()[0].dtype, _broadcast_shape(node, ins))]

    def evaluate(node: Node, ins: _Dynamic) -> list[np.ndarray]:
        a = ins.a(0)
        return [_like(fn(a, ins.a(1)), a)]

    return shape_rule, evaluate


def _predicate_family(fn: Callable[[np.ndarray, np.ndarray], Any]) -> tuple[ShapeRule, Evaluator]:
    def shape_rule(node: Node, ins: _Static) -> list[TensorType]:
        return [TensorType("bool", _broadcast_shape(node, ins))]

    def evaluate(node: Node, ins: _Dynamic) -> list[np.ndarray]:
        return [np.asarray(fn(ins.a(0), ins.a(1)), dtype=np.bool_)]

    return shape_rule, evaluate


def _unary_family(fn: Callable[[np.ndarray, Node, _Dynamic], Any]) -> Evaluator:
    def evaluate(node: Node, ins: _Dynamic) -> list[np.ndarray]:
        x = ins.a(0)
        return [_like(fn(x, node, ins), x)]

    return evaluate


for _op, _fn in _ARITHMETIC.items():
    _define(_op, *_arith_family(_fn), elementwise=True)
for _op, _fn in _PREDICATES.items():
    _define(_op, *_predicate_family(_fn), elementwise=True)
for _op, _fn in _UNARY.items():
    _define(_op, _first, _unary_family(_fn), elementwise=True)
_define("Not", _first, lambda n, o: [np.logical_not(o.a(0))], elementwise=True)
_define("Where", lambda n, s: [TensorType(s.t(1).dtype, _broadcast_shape(n, s))],
        lambda n, o: [_like(np.where(o.a(0), o.a(1), o.a(2)), o.a(1))], elementwise=True)

# ONNX TensorProto element type codes Cast accepts
ONNX_CAST_TYPES = {1: "float32", 2: "uint8", 3: "int8", 6: "int32", 7: "int64", 9: "bool", 10: "float16",
                   11: "float64"}


def cast_dtype(node: Node) -> str:
    to = node.attrs.get("to", 1)
    if isinstance(to, str):
        return to
    if int(to) not in ONNX_CAST_TYPES:
        raise UnsupportedOpError(f"Cast to ONNX type {to} is not supported")
    return ONNX_CAST_TYPES[int(to)]


_define("Cast", lambda n, s: [TensorType(cast_dtype(n), s.t(0).shape)],
        lambda n, o: [o.a(0).astype(cast_dtype(n))], elementwise=True)


# ---------------------------------------------------------------------------------------------
# FusedElementwise: a straight-line program of elementwise instructions
# ---------------------------------------------------------------------------------------------
# ``program`` is a list of [op, attrs, args]; argument a < len(inputs) names node input a,
# a >= len(inputs) the result of instruction a - len(inputs), -1 an omitted input. The last
# instruction's result is the output.
def _instructions(node: Node) -> list[tuple[Node, list[int]]]:
    program = node.attrs.get("program")
    if not program:
        raise UnsupportedOpError("FusedElementwise without a program")
    steps = []
    for op, attrs, args in program:
        if not is_elementwise(str(op)):
            raise UnsupportedOpError(f"FusedElementwise: {op} is not elementwise")
        steps.append((Node(str(op), [], [Value("_")], dict(attrs)), [int(a) for a in args]))
    return steps


def _pick(items: list, args: list[int]) -> list:
    return [items[a] if a >= 0 else None for a in args]


def _program_shape(node: Node, ins: _Static) -> list[TensorType]:
    types, consts = list(ins.types), list(ins.consts)
    for step, args in _instructions(node):
        types.append(spec(step.op).infer(step, _pick(types, args), _pick(consts, args))[0])
        consts.append(None)
    return [types[-1]]


def _program_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    registers = list(ins.arrays)
    for step, args in _instructions(node):
        registers.append(spec(step.op).run(step, _pick(registers, args))[0])
    return [registers[-1]]


_define("FusedElementwise", _program_shape, _program_run)


# ---------------------------------------------------------------------------------------------
# data movement and shape operators
# ---------------------------------------------------------------------------------------------
def _dropout_shape(node: Node, ins: _Static) -> list[TensorType]:
    x = ins.t(0)
    return [x, TensorType("bool", x.shape)] if len(node.outputs) > 1 else [x]


def _dropout_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    x = ins.a(0)
    if len(node.outputs) > 1:
        return [x.copy(), np.ones(x.shape, dtype=np.bool_)]
    return [x.copy()]


_define("Dropout", _dropout_shape, _dropout_run)


def reshape_target(shape_in: tuple[int, ...], spec_: Sequence[int], allowzero: int = 0) -> tuple[int, ...]:
    """ONNX Reshape: 0 copies the input dimension (unless allowzero), one -1 is inferred."""
    target = [int(d) for d in spec_]
    if not allowzero:
        for i, d in enumerate(target):
            if d == 0:
                if i >= len(shape_in):
                    raise ShapeError("Reshape copies a dimension that does not exist")
                target[i] = shape_in[i]
    total = _prod(shape_in)
    holes = [i for i, d in enumerate(target) if d == -1]
    if len(holes) > 1:
        raise ShapeError("Reshape has more than one -1")
    if holes:
        rest = _prod([d for d in target if d != -1])
        if rest == 0 or total % rest:
            raise ShapeError(f"cannot reshape {shape_in} to {list(spec_)}")
        target[holes[0]] = total // rest
    if _prod(target) != total:
        raise ShapeError(f"cannot reshape {shape_in} to {list(spec_)}")
    return tuple(target)


def _reshape_to(node: Node, ins: _Static | _Dynamic, shape_in: tuple[int, ...], at_run: bool) -> tuple[int, ...]:
    if "shape" in node.attrs:
        wanted = list(node.attrs["shape"])
    else:
        wanted = _as_ints(ins.a(1) if at_run else ins.c(1, "Reshape shape"))
    return reshape_target(shape_in, wanted, int(node.attrs.get("allowzero", 0)))


_define("Reshape",
        lambda n, s: [TensorType(s.t(0).dtype, _reshape_to(n, s, s.t(0).shape, False))],
        lambda n, o: [o.a(0).reshape(_reshape_to(n, o, o.a(0).shape, True)).copy()])


def _flat2(shape: tuple[int, ...], axis: int) -> tuple[int, int]:
    cut = axis + len(shape) if axis < 0 else axis
    return _prod(shape[:cut]), _prod(shape[cut:])


_define("Flatten",
        lambda n, s: [TensorType(s.t(0).dtype, _flat2(s.t(0).shape, int(n.attrs.get("axis", 1))))],
        lambda n, o: [o.a(0).reshape(_flat2(o.a(0).shape, int(n.attrs.get("axis", 1)))).copy()])


def transpose_perm(node: Node, rank: int) -> list[int]:
    """The permutation of a Transpose; without ``perm`` the axes are reversed."""
    perm = node.attrs.get("perm")
    return [int(p) for p in perm] if perm is not None else list(reversed(range(rank)))


_define("Transpose",
        lambda n, s: [TensorType(s.t(0).dtype, tuple(s.t(0).shape[p] for p in transpose_perm(n, s.t(0).rank)))],
        lambda n, o: [contiguous(o.a(0).transpose(transpose_perm(n, o.a(0).ndim)))])


def _axes_of(node: Node, ins: _Static | _Dynamic, index: int) -> list[int] | None:
    """Axes from the attribute (old opsets) or the constant input ``index`` (new opsets)."""
    if "axes" in node.attrs:
        return [int(a) for a in node.attrs["axes"]]
    given = ins.maybe(index)
    if given is not None:
        return _as_ints(given)
    if len(node.inputs) > index and node.inputs[index] is not None:
        raise ShapeError(f"{node.op} axes must be a constant")
    return None


def _squeezed(shape: tuple[int, ...], axes: list[int] | None) -> tuple[int, ...]:
    if axes is None:
        return tuple(d for d in shape if d != 1)
    drop = {_axis(a, len(shape)) for a in axes}
    bad = next((a for a in sorted(drop) if shape[a] != 1), None)
    if bad is not None:
        raise ShapeError(f"cannot squeeze axis {bad} of size {shape[bad]}")
    return tuple(d for i, d in enumerate(shape) if i not in drop)


def _unsqueezed(shape: tuple[int, ...], axes: list[int] | None) -> tuple[int, ...]:
    if axes is None:
        raise ShapeError("Unsqueeze needs axes")
    rank = len(shape) + len(axes)
    ones = {_axis(a, rank) for a in axes}
    dims = iter(shape)
    return tuple(1 if i in ones else next(dims) for i in range(rank))


for _op, _fn in (("Squeeze", _squeezed), ("Unsqueeze", _unsqueezed)):
    def _family(fn: Callable[[tuple[int, ...], list[int] | None], tuple[int, ...]]) -> tuple[ShapeRule, Evaluator]:
        return (lambda n, s: [TensorType(s.t(0).dtype, fn(s.t(0).shape, _axes_of(n, s, 1)))],
                lambda n, o: [o.a(0).reshape(fn(o.a(0).shape, _axes_of(n, o, 1))).copy()])

    _define(_op, *_family(_fn))


def _concat_shape(node: Node, ins: _Static) -> list[TensorType]:
    parts = ins.present()
    head = parts[0]
    axis = _axis(int(node.attrs.get("axis", 0)), head.rank)
    for p in parts:
        if p.rank != head.rank or any(p.shape[i] != head.shape[i] for i in range(head.rank) if i != axis):
            raise ShapeError(f"Concat shapes differ: {[q.shape for q in parts]}")
    shape = list(head.shape)
    shape[axis] = sum(p.shape[axis] for p in parts)
    return [TensorType(head.dtype, tuple(shape))]


_define("Concat", _concat_shape,
        lambda n, o: [np.concatenate([x for x in o.arrays if x is not None], axis=int(n.attrs.get("axis", 0)))])


def _split_lengths(node: Node, shape: tuple[int, ...], given: np.ndarray | None) -> list[int]:
    axis = _axis(int(node.attrs.get("axis", 0)), len(shape))
    if "split" in node.attrs:
        return [int(s) for s in node.attrs["split"]]
    if given is not None:
        return _as_ints(given)
    if "num_outputs" in node.attrs:
        parts = int(node.attrs["num_outputs"])
        chunk = -(-shape[axis] // parts)
        return [chunk] * (parts - 1) + [shape[axis] - chunk * (parts - 1)]
    parts = len(node.outputs)
    if shape[axis] % parts:
        raise ShapeError("Split cannot divide the axis evenly")
    return [shape[axis] // parts] * parts


def _split_shape(node: Node, ins: _Static) -> list[TensorType]:
    x = ins.t(0)
    axis = _axis(int(node.attrs.get("axis", 0)), x.rank)
    return [TensorType(x.dtype, x.shape[:axis] + (n,) + x.shape[axis + 1:])
            for n in _split_lengths(node, x.shape, ins.maybe(1))]


def _split_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    x = ins.a(0)
    axis = _axis(int(node.attrs.get("axis", 0)), x.ndim)
    cuts = np.cumsum(_split_lengths(node, x.shape, ins.maybe(1)))[:-1]
    return [piece.copy() for piece in np.split(x, cuts, axis=axis)]


_define("Split", _split_shape, _split_run)


def slice_params(node: Node, shape: tuple[int, ...], consts: Sequence[np.ndarray | None]) -> list[slice]:
    """One normalized python slice per axis (ONNX Slice, attribute form and input form)."""
    if "starts" in node.attrs:
        starts, ends = [int(v) for v in node.attrs["starts"]], [int(v) for v in node.attrs["ends"]]
        axes = [int(v) for v in node.attrs.get("axes", range(len(starts)))]
        steps = [1] * len(starts)
    else:
        operands = _Static([], list(consts))
        starts = _as_ints(operands.c(1, "Slice starts"))
        ends = _as_ints(operands.c(2, "Slice ends"))
        axes = _as_ints(operands.maybe(3)) if operands.maybe(3) is not None else list(range(len(starts)))
        steps = _as_ints(operands.maybe(4)) if operands.maybe(4) is not None else [1] * len(starts)
    if not len(starts) == len(ends) == len(axes) == len(steps):
        raise ValueError("Slice starts, ends, axes and steps differ in length")
    out = [slice(None)] * len(shape)
    for first, last, ax, step in zip(starts, ends, axes, steps):
        a = _axis(ax, len(shape))
        if step == 0:
            raise ShapeError("Slice step cannot be 0")
        dim = shape[a]
        lo, hi, st = slice(min(max(first, -dim - 1), dim), min(max(last, -dim - 1), dim), step).indices(dim)
        out[a] = slice(lo, hi if hi >= 0 else None, st)
    return out


def _sliced_shape(shape: tuple[int, ...], cuts: list[slice]) -> tuple[int, ...]:
    return tuple(len(range(*s.indices(d))) for s, d in zip(cuts, shape))


_define("Slice",
        lambda n, s: [TensorType(s.t(0).dtype, _sliced_shape(s.t(0).shape, slice_params(n, s.t(0).shape, s.consts)))],
        lambda n, o: [contiguous(o.a(0)[tuple(slice_params(n, o.a(0).shape, o.arrays))])])


def _gather_shape(node: Node, ins: _Static) -> list[TensorType]:
    x, idx = ins.t(0), ins.t(1)
    axis = _axis(int(node.attrs.get("axis", 0)), x.rank)
    return [TensorType(x.dtype, x.shape[:axis] + idx.shape + x.shape[axis + 1:])]


def _gather_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    x = ins.a(0)
    axis = _axis(int(node.attrs.get("axis", 0)), x.ndim)
    dim = x.shape[axis]
    idx = ins.a(1)
    idx = np.where(idx < 0, idx + dim, idx)
    if idx.size and (idx.min() < 0 or idx.max() >= dim):
        raise ShapeError(f"Gather index out of range for axis {axis} of size {dim}")
    return [np.take(x, idx, axis=axis)]


_define("Gather", _gather_shape, _gather_run)


def shape_value(node: Node, shape: tuple[int, ...]) -> np.ndarray:
    """The int64 vector a Shape node produces (with its optional start/end attributes)."""
    end = node.attrs.get("end")
    window = slice(int(node.attrs.get("start", 0)), None if end is None else int(end))
    return np.asarray(shape[window], dtype=np.int64)


_define("Shape", lambda n, s: [TensorType("int64", (len(shape_value(n, s.t(0).shape)),))],
        lambda n, o: [shape_value(n, o.a(0).shape)])
_define("Size", lambda n, s: [TensorType("int64", ())], lambda n, o: [np.asarray(o.a(0).size, dtype=np.int64)])


def _fill_of(node: Node) -> tuple[Any, np.dtype]:
    value = node.attrs.get("value")
    if isinstance(value, np.ndarray):
        return np.asarray(value).reshape(-1)[0], value.dtype
    if value is not None:
        return np.asarray(value).reshape(-1)[0], np.dtype(np.float32)
    return np.float32(0), np.dtype(np.float32)


_define("ConstantOfShape",
        lambda n, s: [TensorType(dtype_name(_fill_of(n)[1]), tuple(_as_ints(s.c(0, "ConstantOfShape shape"))))],
        lambda n, o: [np.full(tuple(_as_ints(o.a(0))), _fill_of(n)[0], dtype=_fill_of(n)[1])])


def _expanded(x_shape: tuple[int, ...], target: np.ndarray) -> tuple[int, ...]:
    return tuple(int(d) for d in np.broadcast_shapes(x_shape, tuple(_as_ints(target))))


_define("Expand",
        lambda n, s: [TensorType(s.t(0).dtype, _expanded(s.t(0).shape, s.c(1, "Expand shape")))],
        lambda n, o: [contiguous(np.broadcast_to(o.a(0), _expanded(o.a(0).shape, o.a(1))))])
_define("Tile",
        lambda n, s: [TensorType(s.t(0).dtype, tuple(d * r for d, r in
                                                      zip(s.t(0).shape, _as_ints(s.c(1, "Tile repeats")), strict=True)))],
        lambda n, o: [np.tile(o.a(0), _as_ints(o.a(1)))])


def _range_values(start: np.ndarray, limit: np.ndarray, delta: np.ndarray) -> np.ndarray:
    s, lim, d = (np.asarray(v).reshape(()) for v in (start, limit, delta))
    count = max(math.ceil((float(lim) - float(s)) / float(d)), 0)
    return np.asarray(s + np.arange(count, dtype=s.dtype) * d, dtype=s.dtype)


_define("Range",
        lambda n, s: [TensorType(s.t(0).dtype, _range_values(s.c(0, "Range"), s.c(1, "Range"), s.c(2, "Range")).shape)],
        lambda n, o: [_range_values(o.a(0), o.a(1), o.a(2))])


def _trilu_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    k = ins.maybe(1)
    diagonal = int(np.asarray(k).reshape(())) if k is not None else 0
    keep = np.triu if int(node.attrs.get("upper", 1)) else np.tril
    return [keep(ins.a(0), diagonal)]


_define("Trilu", _first, _trilu_run)


def pad_amounts(node: Node, rank: int, consts: Sequence[np.ndarray | None]) -> list[int]:
    """[begin_0 .. begin_{r-1}, end_0 .. end_{r-1}] of a Pad (attribute or input form, optional
    axes input)."""
    if "pads" in node.attrs:
        pads = [int(p) for p in node.attrs["pads"]]
    else:
        pads = _as_ints(_Static([], list(consts)).c(1, "Pad pads"))
    axes_given = consts[3] if len(consts) > 3 else None
    if axes_given is None:
        return pads
    axes = [_axis(a, rank) for a in _as_ints(axes_given)]
    full = [0] * (2 * rank)
    for i, a in enumerate(axes):
        full[a] = pads[i]
        full[a + rank] = pads[i + len(axes)]
    return full


def _pad_shape(node: Node, ins: _Static) -> list[TensorType]:
    x = ins.t(0)
    p = pad_amounts(node, x.rank, ins.consts)
    return [TensorType(x.dtype, tuple(d + p[i] + p[i + x.rank] for i, d in enumerate(x.shape)))]


def _pad_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    x = ins.a(0)
    mode = node.attrs.get("mode", "constant")
    if mode != "constant":
        raise UnsupportedOpError(f"Pad mode {mode!r} is not supported")
    p = pad_amounts(node, x.ndim, ins.arrays)
    fill = ins.maybe(2)
    value = float(np.asarray(fill).reshape(())) if fill is not None else 0.0
    return [np.pad(x, [(p[i], p[i + x.ndim]) for i in range(x.ndim)], constant_values=value)]


_define("Pad", _pad_shape, _pad_run)


# ---------------------------------------------------------------------------------------------
# reductions and normalization
# ---------------------------------------------------------------------------------------------
def reduce_axes(node: Node, rank: int, consts: Sequence[np.ndarray | None]) -> tuple[int, ...]:
    """Sorted reduced axes; all axes when none are given unless noop_with_empty_axes."""
    axes = _axes_of(node, _Static([], list(consts)), 1)
    if axes:
        return tuple(sorted(_axis(a, rank) for a in axes))
    return () if int(node.attrs.get("noop_with_empty_axes", 0)) else tuple(range(rank))


def _reduce_shape(node: Node, ins: _Static) -> list[TensorType]:
    x = ins.t(0)
    axes = set(reduce_axes(node, x.rank, ins.consts))
    keep = int(node.attrs.get("keepdims", 1))
    dims = [1 if i in axes else d for i, d in enumerate(x.shape) if keep or i not in axes]
    return [TensorType(x.dtype, tuple(dims))]


def _reducer(fn: Callable[..., np.ndarray]) -> Evaluator:
    def evaluate(node: Node, ins: _Dynamic) -> list[np.ndarray]:
        x = ins.a(0)
        axes = reduce_axes(node, x.ndim, ins.arrays)
        if not axes:
            return [x.copy()]
        return [_like(fn(x, axis=axes, keepdims=bool(int(node.attrs.get("keepdims", 1)))), x)]

    return evaluate


for _op, _fn in (("ReduceMean", np.mean), ("ReduceSum", np.sum), ("ReduceMax", np.max), ("ReduceMin", np.min),
                 ("ReduceProd", np.prod)):
    _define(_op, _reduce_shape, _reducer(_fn))


def _argmax_shape(node: Node, ins: _Static) -> list[TensorType]:
    x = ins.t(0)
    axis = _axis(int(node.attrs.get("axis", 0)), x.rank)
    keep = int(node.attrs.get("keepdims", 1))
    return [TensorType("int64", tuple(1 if i == axis else d for i, d in enumerate(x.shape) if keep or i != axis))]


def _argmax_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    x = ins.a(0)
    axis = _axis(int(node.attrs.get("axis", 0)), x.ndim)
    winners = np.argmax(x, axis=axis)  # the first of equal maxima
    if int(node.attrs.get("keepdims", 1)):
        winners = np.expand_dims(winners, axis)
    return [winners.astype(np.int64)]


_define("ArgMax", _argmax_shape, _argmax_run)


def softmax(x: np.ndarray, axis: int) -> np.ndarray:
    shifted = np.exp(x - np.max(x, axis=axis, keepdims=True))
    return _like(shifted / np.sum(shifted, axis=axis, keepdims=True), x)


def _log_softmax(x: np.ndarray, axis: int) -> np.ndarray:
    centered = x - np.max(x, axis=axis, keepdims=True)
    return _like(centered - np.log(np.sum(np.exp(centered), axis=axis, keepdims=True)), x)


for _op, _fn in (("Softmax", softmax), ("LogSoftmax", _log_softmax)):
    def _softmax_family(fn: Callable[[np.ndarray, int], np.ndarray]) -> Evaluator:
        return lambda n, o: [fn(o.a(0), _axis(int(n.attrs.get("axis", -1)), o.a(0).ndim))]

    _define(_op, _first, _softmax_family(_fn))


def layer_norm(x: np.ndarray, scale: np.ndarray | None, bias: np.ndarray | None, axis: int, eps: float) -> np.ndarray:
    """(x - mean) / sqrt(var + eps) * scale + bias over axes [axis, rank), in float64."""
    over = tuple(range(axis, x.ndim))
    wide = x.astype(np.float64)
    centered = wide - wide.mean(axis=over, keepdims=True)
    y = centered / np.sqrt((centered * centered).mean(axis=over, keepdims=True) + eps)
    y = y if scale is None else y * scale
    y = y if bias is None else y + bias
    return _like(y, x)


def _ln_shape(node: Node, ins: _Static) -> list[TensorType]:
    if len(node.outputs) > 1:
        raise UnsupportedOpError("LayerNormalization mean and inverse std outputs")
    return [ins.t(0)]


_define("LayerNormalization", _ln_shape,
        lambda n, o: [layer_norm(o.a(0), o.maybe(1), o.maybe(2), _axis(int(n.attrs.get("axis", -1)), o.a(0).ndim),
                                 float(n.attrs.get("epsilon", 1e-5)))])


def _batch_norm_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    x, scale, bias, mean, var = (ins.a(i) for i in range(5))
    per_channel = [1] * x.ndim
    per_channel[x.ndim - 1 if node.attrs.get("layout") == "NHWC" else 1] = -1
    factor = (scale / np.sqrt(var + float(node.attrs.get("epsilon", 1e-5)))).reshape(per_channel)
    return [_like((x - mean.reshape(per_channel)) * factor + bias.reshape(per_channel), x)]


_define("BatchNormalization", _first, _batch_norm_run)


# ---------------------------------------------------------------------------------------------
# contractions
# ---------------------------------------------------------------------------------------------
def _matmul_shape(a: tuple[int, ...], b: tuple[int, ...]) -> tuple[int, ...]:
    if not a or not b:
        raise ShapeError("MatMul operands must have rank >= 1")
    lhs = a if len(a) > 1 else (1, *a)
    rhs = b if len(b) > 1 else (*b, 1)
    if lhs[-1] != rhs[-2]:
        raise ShapeError(f"MatMul inner dimensions differ: {a} x {b}")
    rows = (lhs[-2],) if len(a) > 1 else ()
    cols = (rhs[-1],) if len(b) > 1 else ()
    return tuple(int(d) for d in np.broadcast_shapes(lhs[:-2], rhs[:-2])) + rows + cols


_define("MatMul", lambda n, s: [TensorType(s.t(0).dtype, _matmul_shape(s.t(0).shape, s.t(1).shape))],
        lambda n, o: [_like(np.matmul(o.a(0), o.a(1)), o.a(0))])


def _gemm_dims(node: Node, a: tuple[int, ...], b: tuple[int, ...]) -> tuple[int, int, int, int]:
    """(m, k of A, k of B, n) of a Gemm after its transposes."""
    m, ka = (a[1], a[0]) if int(node.attrs.get("transA", 0)) else (a[0], a[1])
    kb, n = (b[1], b[0]) if int(node.attrs.get("transB", 0)) else (b[0], b[1])
    return m, ka, kb, n


def _gemm_shape(node: Node, ins: _Static) -> list[TensorType]:
    a, b = ins.t(0), ins.t(1)
    m, ka, kb, n = _gemm_dims(node, a.shape, b.shape)
    if ka != kb:
        raise ShapeError(f"Gemm inner dimensions differ: {a.shape} x {b.shape}")
    return [TensorType(a.dtype, (m, n))]


def _gemm_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    a, b, c = ins.a(0), ins.a(1), ins.maybe(2)
    lhs = a.T if int(node.attrs.get("transA", 0)) else a
    rhs = b.T if int(node.attrs.get("transB", 0)) else b
    y = float(node.attrs.get("alpha", 1.0)) * (lhs @ rhs)
    if c is not None:
        y = y + float(node.attrs.get("beta", 1.0)) * c
    return [_like(y, lhs)]


_define("Gemm", _gemm_shape, _gemm_run)


def apply_activation(y: np.ndarray, node: Node) -> np.ndarray:
    """The ``activation`` attribute of a fused GEMM / convolution applied to ``y``."""
    act = str(node.attrs.get("activation", "none"))
    table: dict[str, Callable[[np.ndarray], np.ndarray]] = {
        "none": lambda v: v,
        "relu": lambda v: np.asarray(np.maximum(v, 0), dtype=v.dtype),
        "clip": lambda v: np.asarray(np.clip(v, float(node.attrs.get("clip_min", 0.0)),
                                             float(node.attrs.get("clip_max", 6.0))), dtype=v.dtype),
        "gelu": lambda v: gelu(v, "none"),
        "gelu_tanh": lambda v: gelu(v, "tanh"),
        "tanh": np.tanh,
        "sigmoid": sigmoid,
    }
    if act not in table:
        raise UnsupportedOpError(f"activation {act!r}")
    return table[act](y)


def _fused_gemm_shape(node: Node, ins: _Static) -> list[TensorType]:
    a, b = ins.t(0), ins.t(1)
    k, n = (b.shape[1], b.shape[0]) if int(node.attrs.get("trans_b", 0)) else b.shape
    if b.rank != 2 or a.shape[-1] != k:
        raise ShapeError(f"FusedGemm shapes: {a.shape} x {b.shape}")
    return [TensorType(a.dtype, a.shape[:-1] + (n,))]


def _fused_gemm_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    """act(A B + bias + residual), A of any rank, B two-dimensional."""
    a, b = ins.a(0), ins.a(1)
    y = a @ (b.T if int(node.attrs.get("trans_b", 0)) else b)
    for extra in (ins.maybe(2), ins.maybe(3)):
        if extra is not None:
            y = y + extra
    return [_like(apply_activation(y, node), a)]


_define("FusedGemm", _fused_gemm_shape, _fused_gemm_run)


@dataclass(frozen=True)
class Conv2dGeometry:
    """A 2-D window after auto_pad: pads are (top, left, bottom, right)."""

    kernel: tuple[int, int]
    strides: tuple[int, int]
    dilations: tuple[int, int]
    pads: tuple[int, int, int, int]
    out_hw: tuple[int, int]


def _same_pads(in_hw: tuple[int, int], strides: Sequence[int], span: Sequence[int], upper: bool) -> list[int]:
    begin, end = [], []
    for i in range(2):
        out = -(-in_hw[i] // strides[i])
        total = max((out - 1) * strides[i] + span[i] - in_hw[i], 0)
        low, high = total // 2, total - total // 2
        begin.append(low if upper else high)
        end.append(high if upper else low)
    return begin + end


def window_geometry(node: Node, in_hw: tuple[int, int], kernel: tuple[int, int], ceil_mode: bool = False) -> Conv2dGeometry:
    """Pads and output size of a 2-D convolution or pooling window (ONNX rules: auto_pad SAME_*
    and VALID, dilation, ceil_mode where the last window must start inside the padded input)."""
    strides = [int(s) for s in node.attrs.get("strides", (1, 1))]
    dilations = [int(d) for d in node.attrs.get("dilations", (1, 1))]
    pads = [int(p) for p in node.attrs.get("pads", (0, 0, 0, 0))]
    if (len(strides), len(dilations), len(pads)) != (2, 2, 4):
        raise UnsupportedOpError(f"{node.op}: only 2-D windows are supported")
    span = [(kernel[i] - 1) * dilations[i] + 1 for i in range(2)]
    auto_pad = node.attrs.get("auto_pad", "NOTSET")
    if auto_pad in ("SAME_UPPER", "SAME_LOWER"):
        pads = _same_pads(in_hw, strides, span, auto_pad == "SAME_UPPER")
    elif auto_pad == "VALID":
        pads = [0, 0, 0, 0]
    out_hw = []
    for i in range(2):
        room = in_hw[i] + pads[i] + pads[i + 2] - span[i]
        if room < 0:
            raise ShapeError(f"{node.op}: window larger than the padded input")
        if ceil_mode:
            count = -(-room // strides[i]) + 1
            if (count - 1) * strides[i] >= in_hw[i] + pads[i]:
                count -= 1
        else:
            count = room // strides[i] + 1
        out_hw.append(count)
    return Conv2dGeometry((kernel[0], kernel[1]), (strides[0], strides[1]), (dilations[0], dilations[1]),
                          (pads[0], pads[1], pads[2], pads[3]), (out_hw[0], out_hw[1]))


def conv_layout(node: Node) -> str:
    layout = str(node.attrs.get("layout", "NCHW"))
    if layout not in ("NCHW", "NHWC"):
        raise UnsupportedOpError(f"layout {layout!r}")
    return layout


def _conv_shape(node: Node, ins: _Static) -> list[TensorType]:
    x, w = ins.t(0), ins.t(1)
    if x.rank != 4 or w.rank != 4:
        raise UnsupportedOpError(f"{node.op}: only 2-D convolution (rank 4) is supported")
    nhwc = conv_layout(node) == "NHWC"
    n, h, wd, c = x.shape if nhwc else (x.shape[0], x.shape[2], x.shape[3], x.shape[1])
    kh, kw, cg, k = w.shape if nhwc else (w.shape[2], w.shape[3], w.shape[1], w.shape[0])
    group = int(node.attrs.get("group", 1))
    if cg * group != c or k % group:
        raise ShapeError(f"{node.op}: channels {c} do not match weights {w.shape} with group {group}")
    oh, ow = window_geometry(node, (h, wd), (kh, kw)).out_hw
    return [TensorType(x.dtype, (n, oh, ow, k) if nhwc else (n, k, oh, ow))]


def _im2col_conv(x: np.ndarray, w: np.ndarray, g: Conv2dGeometry, group: int) -> np.ndarray:
    """NCHW input, OIHW weights: one matrix product per group over gathered window columns."""
    n, c, h, wd = x.shape
    k, cg, kh, kw = w.shape
    pt, pl, pb, pr = g.pads
    padded = np.pad(x, ((0, 0), (0, 0), (pt, pb), (pl, pr)))
    oh, ow = g.out_hw
    taps = []
    for i in range(kh):
        for j in range(kw):
            r0, c0 = i * g.dilations[0], j * g.dilations[1]
            taps.append(padded[:, :, r0: r0 + (oh - 1) * g.strides[0] + 1: g.strides[0],
                               c0: c0 + (ow - 1) * g.strides[1] + 1: g.strides[1]])
    cols = np.stack(taps, axis=2)  # [n, c, kh*kw, oh, ow]
    kg = k // group
    out = np.empty((n, k, oh, ow), dtype=np.result_type(x, w))
    for gi in range(group):
        block = cols[:, gi * cg:(gi + 1) * cg].reshape(n, cg * kh * kw, oh * ow)
        weights = w[gi * kg:(gi + 1) * kg].reshape(kg, cg * kh * kw)
        out[:, gi * kg:(gi + 1) * kg] = np.matmul(weights, block).reshape(n, kg, oh, ow)
    return out


def _conv_value(node: Node, x: np.ndarray, w: np.ndarray, b: np.ndarray | None) -> np.ndarray:
    nhwc = conv_layout(node) == "NHWC"
    xc = x.transpose(0, 3, 1, 2) if nhwc else x
    wc = w.transpose(3, 2, 0, 1) if nhwc else w
    g = window_geometry(node, (xc.shape[2], xc.shape[3]), (wc.shape[2], wc.shape[3]))
    y = _im2col_conv(xc, wc, g, int(node.attrs.get("group", 1)))
    if b is not None:
        y = y + b.reshape(1, -1, 1, 1)
    return y.transpose(0, 2, 3, 1) if nhwc else y


def _conv_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    x = ins.a(0)
    y = _conv_value(node, x, ins.a(1), ins.maybe(2))
    if node.op == "FusedConv":  # act(conv + bias + residual)
        residual = ins.maybe(3)
        y = apply_activation(y if residual is None else y + residual, node)
    return [_like(contiguous(y), x)]


_define("Conv", _conv_shape, _conv_run)
_define("FusedConv", _conv_shape, _conv_run)


# ---------------------------------------------------------------------------------------------
# pooling
# ---------------------------------------------------------------------------------------------
def _pool_geometry(node: Node, x: TensorType) -> tuple[Conv2dGeometry, tuple[int, ...]]:
    if x.rank != 4:
        raise UnsupportedOpError(f"{node.op}: only 2-D pooling is supported")
    kernel = [int(k) for k in node.attrs["kernel_shape"]]
    nhwc = conv_layout(node) == "NHWC"
    hw = x.shape[1:3] if nhwc else x.shape[2:4]
    g = window_geometry(node, (hw[0], hw[1]), (kernel[0], kernel[1]), bool(node.attrs.get("ceil_mode", 0)))
    oh, ow = g.out_hw
    return g, ((x.shape[0], oh, ow, x.shape[3]) if nhwc else (x.shape[0], x.shape[1], oh, ow))


def _pool_shape(node: Node, ins: _Static) -> list[TensorType]:
    if len(node.outputs) > 1:
        raise UnsupportedOpError("MaxPool indices output is not supported")
    x = ins.t(0)
    return [TensorType(x.dtype, _pool_geometry(node, x)[1])]


def _pool_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    """Window max / mean: each kernel tap is one strided view of the padded input; the mean
    divides the float32 window sum by the number of counted positions (padding counts only
    with count_include_pad; positions of ceil-mode windows past the padding never count)."""
    x = ins.a(0)
    nhwc = conv_layout(node) == "NHWC"
    xc = x.transpose(0, 3, 1, 2) if nhwc else x
    g, _ = _pool_geometry(node, TensorType.of(x))
    oh, ow = g.out_hw
    (sh, sw), (dh, dw), (kh, kw) = g.strides, g.dilations, g.kernel
    pt, pl, pb, pr = g.pads
    h, wd = xc.shape[2], xc.shape[3]
    extra_h = max((oh - 1) * sh + (kh - 1) * dh + 1 - (h + pt + pb), 0)
    extra_w = max((ow - 1) * sw + (kw - 1) * dw + 1 - (wd + pl + pr), 0)
    biggest = node.op == "MaxPool"
    grid = ((0, 0), (0, 0), (pt, pb + extra_h), (pl, pr + extra_w))
    padded = np.pad(xc, grid, constant_values=-np.inf if biggest else 0.0)
    counted = np.zeros((h, wd))
    counted = np.pad(counted + 1.0, ((pt, pb), (pl, pr)),
                     constant_values=1.0 if int(node.attrs.get("count_include_pad", 0)) else 0.0)
    counted = np.pad(counted, ((0, extra_h), (0, extra_w)))
    acc = None
    count = np.zeros((oh, ow))
    for i in range(kh):
        for j in range(kw):
            rows = slice(i * dh, i * dh + (oh - 1) * sh + 1, sh)
            cols = slice(j * dw, j * dw + (ow - 1) * sw + 1, sw)
            tap = padded[:, :, rows, cols]
            count += counted[rows, cols]
            acc = tap.copy() if acc is None else (np.maximum(acc, tap) if biggest else acc + tap)
    y = acc if biggest else acc / count
    y = contiguous(np.asarray(y, dtype=x.dtype))
    return [contiguous(y.transpose(0, 2, 3, 1)) if nhwc else y]


_define("MaxPool", _pool_shape, _pool_run)
_define("AveragePool", _pool_shape, _pool_run)


def _global_shape(node: Node, ins: _Static) -> list[TensorType]:
    x = ins.t(0)
    if x.rank < 3:
        raise ShapeError(f"{node.op} needs rank >= 3")
    ones = (1,) * (x.rank - 2)
    if conv_layout(node) == "NHWC":
        return [TensorType(x.dtype, (x.shape[0], *ones, x.shape[-1]))]
    return [TensorType(x.dtype, (*x.shape[:2], *ones))]


def _global_run(node: Node, ins: _Dynamic) -> list[np.ndarray]:
    x = ins.a(0)
    spatial = tuple(range(1, x.ndim - 1)) if conv_layout(node) == "NHWC" else tuple(range(2, x.ndim))
    if node.op == "GlobalMaxPool":
        return [x.max(axis=spatial, keepdims=True)]
    return [_like(x.mean(axis=spatial, keepdims=True), x)]


_define("GlobalAveragePool", _global_shape, _global_run)
_define("GlobalMaxPool", _global_shape, _global_run)


# ---------------------------------------------------------------------------------------------
# cost model
# ---------------------------------------------------------------------------------------------
def flops(node: Node) -> int:
    """Floating-point operations of one node, a multiply-add counting as 2 (the reference's
    cost model: contractions 2 per MAC, a FusedElementwise program one per instruction and
    element, anything else one per output element)."""
    out = node.outputs[0].type
    if out is None:
        return 0
    if node.op in ("Conv", "FusedConv"):
        w = node.input(1).tensor_type
        out_channels = w.shape[3] if conv_layout(node) == "NHWC" else w.shape[0]
        return 2 * out.size * (w.size // out_channels)
    if node.op in ("MatMul", "FusedGemm", "Gemm"):
        a = node.input(0).tensor_type
        transposed = node.op == "Gemm" and int(node.attrs.get("transA", 0))
        return 2 * out.size * (a.shape[0] if transposed else a.shape[-1])
    if node.op == "FusedElementwise":
        return out.size * len(node.attrs.get("program", ()))
    return out.size
