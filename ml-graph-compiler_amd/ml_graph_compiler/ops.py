"""Operator table: static shape/type inference and compile-time evaluation.

Reference: src/ml_graph_compiler/ops.py:1-1239. Each operator has an ``infer`` rule (input types
plus any known constant inputs -> output types) and an ``evaluate`` rule (numpy arrays in, numpy
arrays out). The compiler uses ``evaluate`` only at compile time: constant folding, partial
evaluation of shape arithmetic during inference, and the Batch-Norm fold. Compiled models never
call it; the run-time path is the HIP kernels of libmgc_hip.so. The dtype rules follow the
reference exactly (results keep the first operand's dtype, integer Div truncates, LayerNorm runs
in float64, erf is the shared rational approximation, argmax takes the first maximum).
"""

from __future__ import annotations

import math
from collections.abc import Callable, Sequence
from dataclasses import dataclass
from typing import Any

import numpy as np

from .errors import ShapeError, UnsupportedOpError
from .ir import Node, TensorType, Value, contiguous, dtype_name

Arrays = list  # list[np.ndarray | None]
Types = list  # list[TensorType | None]
InferFn = Callable[[Node, Types, Arrays], list[TensorType]]
EvalFn = Callable[[Node, Arrays], list[np.ndarray]]


@dataclass(frozen=True)
class OpSpec:
    infer: InferFn
    run: EvalFn
    elementwise: bool = False


REGISTRY: dict[str, OpSpec] = {}
SHAPE_ONLY_OPS = frozenset({"Shape", "Size"})
ACTIVATIONS = ("none", "relu", "clip", "gelu", "gelu_tanh", "tanh", "sigmoid")
_PLACEHOLDER = Value("_")


def _register(name: str, infer: InferFn, run: EvalFn, elementwise: bool = False) -> None:
    REGISTRY[name] = OpSpec(infer, run, elementwise)


def spec(op: str) -> OpSpec:
    if op not in REGISTRY:
        raise UnsupportedOpError(f"operator {op!r} is not supported")
    return REGISTRY[op]


def supported_ops() -> list[str]:
    return sorted(REGISTRY)


# ---------------------------------------------------------------------------------------------
# small helpers
# ---------------------------------------------------------------------------------------------
def _type(types: Types, i: int) -> TensorType:
    t = types[i] if i < len(types) else None
    if t is None:
        raise ShapeError(f"missing type for input {i}")
    return t


def _known(consts: Arrays, i: int, what: str) -> np.ndarray:
    c = consts[i] if i < len(consts) else None
    if c is None:
        raise ShapeError(f"{what} must be a constant (static shapes are required)")
    return c


def _need(arrays: Arrays, i: int) -> np.ndarray:
    a = arrays[i] if i < len(arrays) else None
    if a is None:
        raise UnsupportedOpError(f"missing input {i}")
    return a


def _maybe(arrays: Arrays, i: int) -> np.ndarray | None:
    return arrays[i] if i < len(arrays) else None


def norm_axis(axis: int, rank: int) -> int:
    a = axis + rank if axis < 0 else axis
    if a < 0 or a >= max(rank, 1):
        raise ShapeError(f"axis {axis} out of range for rank {rank}")
    return a


def int_list(values: Any) -> list[int]:
    return [int(v) for v in np.asarray(values).reshape(-1)]


def keep_dtype(x: Any, like: np.ndarray) -> np.ndarray:
    """numpy result cast back to the dtype of the first operand."""
    return np.asarray(x, dtype=like.dtype)


def _same_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    return [_type(types, 0)]


def _broadcast_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    present = [t for t in types if t is not None]
    try:
        shape = np.broadcast_shapes(*(t.shape for t in present))
    except ValueError as exc:
        raise ShapeError(
            f"{node.op}: shapes do not broadcast: {[t.shape for t in present]}"
        ) from exc
    return [TensorType(present[0].dtype, tuple(int(d) for d in shape))]


def _bool_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    return [TensorType("bool", _broadcast_infer(node, types, consts)[0].shape)]


# ---------------------------------------------------------------------------------------------
# elementwise operators
# ---------------------------------------------------------------------------------------------
def _binary(fn: Callable[[np.ndarray, np.ndarray], np.ndarray]) -> EvalFn:
    def run(node: Node, xs: Arrays) -> list[np.ndarray]:
        a = _need(xs, 0)
        return [keep_dtype(fn(a, _need(xs, 1)), a)]

    return run


for _op, _fn in (
    ("Add", np.add),
    ("Sub", np.subtract),
    ("Mul", np.multiply),
    ("Max", np.maximum),
    ("Min", np.minimum),
):
    _register(_op, _broadcast_infer, _binary(_fn), elementwise=True)


def _div_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    a, b = _need(xs, 0), _need(xs, 1)
    if np.issubdtype(a.dtype, np.integer):
        return [np.asarray(np.trunc(a / b), dtype=a.dtype)]
    return [keep_dtype(a / b, a)]


def _pow_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    a, b = _need(xs, 0), _need(xs, 1)
    return [keep_dtype(np.power(a, b.astype(a.dtype)), a)]


_register("Div", _broadcast_infer, _div_run, elementwise=True)
_register("Pow", _broadcast_infer, _pow_run, elementwise=True)


def _logical(fn: Callable[[np.ndarray, np.ndarray], np.ndarray]) -> EvalFn:
    def run(node: Node, xs: Arrays) -> list[np.ndarray]:
        return [np.asarray(fn(_need(xs, 0), _need(xs, 1)), dtype=np.bool_)]

    return run


for _op, _fn in (
    ("Equal", np.equal),
    ("Less", np.less),
    ("Greater", np.greater),
    ("LessOrEqual", np.less_equal),
    ("GreaterOrEqual", np.greater_equal),
    ("And", np.logical_and),
    ("Or", np.logical_or),
    ("Xor", np.logical_xor),
):
    _register(_op, _bool_infer, _logical(_fn), elementwise=True)


def _where_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    return [TensorType(_type(types, 1).dtype, _broadcast_infer(node, types, consts)[0].shape)]


def _where_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 1)
    return [keep_dtype(np.where(_need(xs, 0), x, _need(xs, 2)), x)]


_register("Where", _where_infer, _where_run, elementwise=True)

# Rational approximation of erf on [-4, 4] (about 1e-7 absolute error), evaluated in float64.
# The same coefficients are used by the reference's interpreter and C runtime and by the HIP
# kernels, so GELU agrees between all of them to float rounding.
ERF_NUMERATOR = (
    -2.72614225801306e-10,
    2.77068142495902e-08,
    -2.10102402082508e-06,
    -5.69250639462346e-05,
    -7.34990630326855e-04,
    -2.95459980854025e-03,
    -1.60960333262415e-02,
)
ERF_DENOMINATOR = (
    -1.45660718464996e-05,
    -2.13374055278905e-04,
    -1.68282697438203e-03,
    -7.37332916720468e-03,
    -1.42647390514189e-02,
)


def erf(x: np.ndarray) -> np.ndarray:
    x64 = np.clip(np.asarray(x, dtype=np.float64), -4.0, 4.0)
    z = x64 * x64
    num = np.full_like(x64, ERF_NUMERATOR[0])
    for c in ERF_NUMERATOR[1:]:
        num = num * z + c
    den = np.full_like(x64, ERF_DENOMINATOR[0])
    for c in ERF_DENOMINATOR[1:]:
        den = den * z + c
    return np.asarray(num * x64 / den, dtype=np.asarray(x).dtype)


def gelu(x: np.ndarray, approximate: str = "none") -> np.ndarray:
    if approximate == "tanh":
        k = math.sqrt(2.0 / math.pi)
        return keep_dtype(0.5 * x * (1.0 + np.tanh(k * (x + 0.044715 * x * x * x))), x)
    return keep_dtype(0.5 * x * (1.0 + erf(x / math.sqrt(2.0))), x)


def sigmoid(x: np.ndarray) -> np.ndarray:
    return keep_dtype(0.5 * (1.0 + np.tanh(0.5 * x)), x)


def _unary(fn: Callable[[np.ndarray], np.ndarray]) -> EvalFn:
    def run(node: Node, xs: Arrays) -> list[np.ndarray]:
        x = _need(xs, 0)
        return [keep_dtype(fn(x), x)]

    return run


for _op, _ufn in (
    ("Relu", lambda x: np.maximum(x, 0)),
    ("Sigmoid", sigmoid),
    ("Tanh", np.tanh),
    ("Erf", erf),
    ("Sqrt", np.sqrt),
    ("Exp", np.exp),
    ("Log", np.log),
    ("Neg", np.negative),
    ("Abs", np.abs),
    ("Reciprocal", np.reciprocal),
    ("Floor", np.floor),
    ("Ceil", np.ceil),
    ("Sin", np.sin),
    ("Cos", np.cos),
    ("Softplus", lambda x: np.logaddexp(0, x)),
    ("Identity", lambda x: x.copy()),
):
    _register(_op, _same_infer, _unary(_ufn), elementwise=True)

_register("Not", _same_infer, lambda n, xs: [np.logical_not(_need(xs, 0))], elementwise=True)
_register(
    "Gelu",
    _same_infer,
    lambda n, xs: [gelu(_need(xs, 0), str(n.attrs.get("approximate", "none")))],
    elementwise=True,
)


def _leaky_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    alpha = float(node.attrs.get("alpha", 0.01))
    return [keep_dtype(np.where(x >= 0, x, alpha * x), x)]


def _hard_sigmoid_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    alpha = float(node.attrs.get("alpha", 0.2))
    beta = float(node.attrs.get("beta", 0.5))
    return [keep_dtype(np.clip(alpha * x + beta, 0, 1), x)]


_register("LeakyRelu", _same_infer, _leaky_run, elementwise=True)
_register("HardSigmoid", _same_infer, _hard_sigmoid_run, elementwise=True)


def clip_bounds(node: Node, xs: Sequence[np.ndarray | None]) -> tuple[float, float]:
    """Clip bounds: attributes (opset < 11) overridden by the optional inputs (opset >= 11)."""
    lo = node.attrs.get("min", -np.inf)
    hi = node.attrs.get("max", np.inf)
    if len(xs) > 1 and xs[1] is not None:
        lo = float(np.asarray(xs[1]).reshape(()))
    if len(xs) > 2 and xs[2] is not None:
        hi = float(np.asarray(xs[2]).reshape(()))
    return float(lo), float(hi)


def _clip_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    lo, hi = clip_bounds(node, xs)
    return [keep_dtype(np.clip(x, lo, hi), x)]


_register("Clip", _same_infer, _clip_run, elementwise=True)

ONNX_CAST_TYPES = {
    1: "float32",
    2: "uint8",
    3: "int8",
    6: "int32",
    7: "int64",
    9: "bool",
    10: "float16",
    11: "float64",
}


def cast_dtype(node: Node) -> str:
    to = node.attrs.get("to", 1)
    if isinstance(to, str):
        return to
    if int(to) not in ONNX_CAST_TYPES:
        raise UnsupportedOpError(f"Cast to ONNX type {to} is not supported")
    return ONNX_CAST_TYPES[int(to)]


_register(
    "Cast",
    lambda n, t, c: [TensorType(cast_dtype(n), _type(t, 0).shape)],
    lambda n, xs: [_need(xs, 0).astype(cast_dtype(n))],
    elementwise=True,
)


def _dropout_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x = _type(types, 0)
    return [x, TensorType("bool", x.shape)] if len(node.outputs) > 1 else [x]


def _dropout_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    result = [x.copy()]
    if len(node.outputs) > 1:
        result.append(np.ones(x.shape, dtype=np.bool_))
    return result


_register("Dropout", _dropout_infer, _dropout_run)


# ---------------------------------------------------------------------------------------------
# shape manipulation
# ---------------------------------------------------------------------------------------------
def reshape_target(
    shape_in: tuple[int, ...], target: Sequence[int], allowzero: int = 0
) -> tuple[int, ...]:
    out = [int(d) for d in target]
    for i, d in enumerate(out):
        if d == 0 and not allowzero:
            if i >= len(shape_in):
                raise ShapeError("Reshape copies a dimension that does not exist")
            out[i] = shape_in[i]
    total = int(np.prod(shape_in, dtype=np.int64))
    if out.count(-1) > 1:
        raise ShapeError("Reshape has more than one -1")
    if -1 in out:
        rest = int(np.prod([d for d in out if d != -1], dtype=np.int64))
        if rest == 0 or total % rest:
            raise ShapeError(f"cannot reshape {shape_in} to {list(target)}")
        out[out.index(-1)] = total // rest
    if int(np.prod(out, dtype=np.int64)) != total:
        raise ShapeError(f"cannot reshape {shape_in} to {list(target)}")
    return tuple(out)


def _reshape_spec(node: Node, consts: Arrays) -> list[int]:
    if "shape" in node.attrs:
        return list(node.attrs["shape"])
    return int_list(_known(consts, 1, "Reshape shape"))


def _reshape_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x = _type(types, 0)
    allow = int(node.attrs.get("allowzero", 0))
    return [TensorType(x.dtype, reshape_target(x.shape, _reshape_spec(node, consts), allow))]


def _reshape_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    target = list(node.attrs["shape"]) if "shape" in node.attrs else int_list(_need(xs, 1))
    allow = int(node.attrs.get("allowzero", 0))
    return [x.reshape(reshape_target(x.shape, target, allow)).copy()]


_register("Reshape", _reshape_infer, _reshape_run)


def flatten_shape(shape: tuple[int, ...], axis: int) -> tuple[int, int]:
    a = axis + len(shape) if axis < 0 else axis
    return int(np.prod(shape[:a], dtype=np.int64)), int(np.prod(shape[a:], dtype=np.int64))


_register(
    "Flatten",
    lambda n, t, c: [
        TensorType(_type(t, 0).dtype, flatten_shape(_type(t, 0).shape, int(n.attrs.get("axis", 1))))
    ],
    lambda n, xs: [
        _need(xs, 0).reshape(flatten_shape(_need(xs, 0).shape, int(n.attrs.get("axis", 1)))).copy()
    ],
)


def transpose_perm(node: Node, rank: int) -> list[int]:
    perm = node.attrs.get("perm")
    if perm is None:
        return list(reversed(range(rank)))
    return [int(p) for p in perm]


_register(
    "Transpose",
    lambda n, t, c: [
        TensorType(
            _type(t, 0).dtype,
            tuple(_type(t, 0).shape[p] for p in transpose_perm(n, _type(t, 0).rank)),
        )
    ],
    lambda n, xs: [contiguous(_need(xs, 0).transpose(transpose_perm(n, _need(xs, 0).ndim)))],
)


def axes_argument(node: Node, consts: Sequence[np.ndarray | None], index: int) -> list[int] | None:
    if "axes" in node.attrs:
        return [int(a) for a in node.attrs["axes"]]
    if len(consts) > index and consts[index] is not None:
        return int_list(consts[index])
    if len(node.inputs) > index and node.inputs[index] is not None:
        raise ShapeError(f"{node.op} axes must be a constant")
    return None


def squeeze_shape(shape: tuple[int, ...], axes: list[int] | None) -> tuple[int, ...]:
    if axes is None:
        return tuple(d for d in shape if d != 1)
    drop = {norm_axis(a, len(shape)) for a in axes}
    for a in drop:
        if shape[a] != 1:
            raise ShapeError(f"cannot squeeze axis {a} of size {shape[a]}")
    return tuple(d for i, d in enumerate(shape) if i not in drop)


def unsqueeze_shape(shape: tuple[int, ...], axes: list[int]) -> tuple[int, ...]:
    rank = len(shape) + len(axes)
    out = list(shape)
    for a in sorted(norm_axis(a, rank) for a in axes):
        out.insert(a, 1)
    return tuple(out)


_register(
    "Squeeze",
    lambda n, t, c: [
        TensorType(_type(t, 0).dtype, squeeze_shape(_type(t, 0).shape, axes_argument(n, c, 1)))
    ],
    lambda n, xs: [
        _need(xs, 0).reshape(squeeze_shape(_need(xs, 0).shape, axes_argument(n, xs, 1))).copy()
    ],
)


def _unsqueeze_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    axes = axes_argument(node, consts, 1)
    if axes is None:
        raise ShapeError("Unsqueeze needs axes")
    return [TensorType(_type(types, 0).dtype, unsqueeze_shape(_type(types, 0).shape, axes))]


def _unsqueeze_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    axes = axes_argument(node, xs, 1)
    assert axes is not None
    return [x.reshape(unsqueeze_shape(x.shape, axes)).copy()]


_register("Unsqueeze", _unsqueeze_infer, _unsqueeze_run)


def _concat_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    parts = [t for t in types if t is not None]
    first = parts[0]
    axis = norm_axis(int(node.attrs.get("axis", 0)), first.rank)
    for t in parts:
        if t.rank != first.rank or any(
            t.shape[i] != first.shape[i] for i in range(first.rank) if i != axis
        ):
            raise ShapeError(f"Concat shapes differ: {[p.shape for p in parts]}")
    shape = list(first.shape)
    shape[axis] = sum(t.shape[axis] for t in parts)
    return [TensorType(first.dtype, tuple(shape))]


_register(
    "Concat",
    _concat_infer,
    lambda n, xs: [np.concatenate([x for x in xs if x is not None], axis=int(n.attrs.get("axis", 0)))],
)


def split_sizes(node: Node, shape: tuple[int, ...], consts: Sequence[np.ndarray | None]) -> list[int]:
    axis = norm_axis(int(node.attrs.get("axis", 0)), len(shape))
    if "split" in node.attrs:
        return [int(s) for s in node.attrs["split"]]
    if len(consts) > 1 and consts[1] is not None:
        return int_list(consts[1])
    parts = len(node.outputs)
    if "num_outputs" in node.attrs:
        parts = int(node.attrs["num_outputs"])
        chunk = -(-shape[axis] // parts)
        return [chunk] * (parts - 1) + [shape[axis] - chunk * (parts - 1)]
    if shape[axis] % parts:
        raise ShapeError("Split cannot divide the axis evenly")
    return [shape[axis] // parts] * parts


def _split_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x = _type(types, 0)
    axis = norm_axis(int(node.attrs.get("axis", 0)), x.rank)
    result = []
    for size in split_sizes(node, x.shape, consts):
        shape = list(x.shape)
        shape[axis] = size
        result.append(TensorType(x.dtype, tuple(shape)))
    return result


def _split_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    axis = norm_axis(int(node.attrs.get("axis", 0)), x.ndim)
    cuts = np.cumsum(split_sizes(node, x.shape, xs))[:-1]
    return [part.copy() for part in np.split(x, cuts, axis=axis)]


_register("Split", _split_infer, _split_run)


def slice_params(
    node: Node, shape: tuple[int, ...], consts: Sequence[np.ndarray | None]
) -> list[slice]:
    """Normalized python slices per axis (ONNX Slice, attribute form and input form)."""
    consts = list(consts)
    if "starts" in node.attrs:
        starts = [int(v) for v in node.attrs["starts"]]
        ends = [int(v) for v in node.attrs["ends"]]
        axes = [int(v) for v in node.attrs.get("axes", range(len(starts)))]
        steps = [1] * len(starts)
    else:
        starts = int_list(_known(consts, 1, "Slice starts"))
        ends = int_list(_known(consts, 2, "Slice ends"))
        axes = int_list(consts[3]) if len(consts) > 3 and consts[3] is not None else list(range(len(starts)))
        steps = int_list(consts[4]) if len(consts) > 4 and consts[4] is not None else [1] * len(starts)
    result = [slice(None)] * len(shape)
    for s, e, a, st in zip(starts, ends, axes, steps, strict=True):
        ax = norm_axis(a, len(shape))
        if st == 0:
            raise ShapeError("Slice step cannot be 0")
        dim = shape[ax]
        s = max(-dim - 1, min(dim, s))
        e = max(-dim - 1, min(dim, e))
        start, stop, step = slice(s, e, st).indices(dim)
        result[ax] = slice(start, stop if stop >= 0 else None, step)
    return result


def _slice_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x = _type(types, 0)
    sl = slice_params(node, x.shape, consts)
    return [TensorType(x.dtype, tuple(len(range(*s.indices(d))) for s, d in zip(sl, x.shape)))]


_register(
    "Slice",
    _slice_infer,
    lambda n, xs: [contiguous(_need(xs, 0)[tuple(slice_params(n, _need(xs, 0).shape, xs))])],
)


def _gather_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x, idx = _type(types, 0), _type(types, 1)
    axis = norm_axis(int(node.attrs.get("axis", 0)), x.rank)
    return [TensorType(x.dtype, x.shape[:axis] + idx.shape + x.shape[axis + 1 :])]


def _gather_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x, idx = _need(xs, 0), _need(xs, 1)
    axis = norm_axis(int(node.attrs.get("axis", 0)), x.ndim)
    idx = np.where(idx < 0, idx + x.shape[axis], idx)
    if idx.size and (int(idx.min()) < 0 or int(idx.max()) >= x.shape[axis]):
        raise ShapeError(f"Gather index out of range for axis {axis} of size {x.shape[axis]}")
    return [np.take(x, idx, axis=axis)]


_register("Gather", _gather_infer, _gather_run)


def shape_value(node: Node, shape: tuple[int, ...]) -> np.ndarray:
    start = int(node.attrs.get("start", 0))
    end = node.attrs.get("end")
    dims = shape[start:] if end is None else shape[start : int(end)]
    return np.asarray(dims, dtype=np.int64)


_register(
    "Shape",
    lambda n, t, c: [TensorType("int64", (len(shape_value(n, _type(t, 0).shape)),))],
    lambda n, xs: [shape_value(n, _need(xs, 0).shape)],
)
_register(
    "Size",
    lambda n, t, c: [TensorType("int64", ())],
    lambda n, xs: [np.asarray(_need(xs, 0).size, dtype=np.int64)],
)


def _cos_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    shape = tuple(int_list(_known(consts, 0, "ConstantOfShape shape")))
    value = node.attrs.get("value")
    dtype = dtype_name(value.dtype) if isinstance(value, np.ndarray) else "float32"
    return [TensorType(dtype, shape)]


def _cos_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    value = node.attrs.get("value")
    fill = np.asarray(value).reshape(-1)[0] if value is not None else np.float32(0)
    dtype = value.dtype if isinstance(value, np.ndarray) else np.float32
    return [np.full(tuple(int_list(_need(xs, 0))), fill, dtype=dtype)]


_register("ConstantOfShape", _cos_infer, _cos_run)


def _expand_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x = _type(types, 0)
    target = tuple(int_list(_known(consts, 1, "Expand shape")))
    return [TensorType(x.dtype, tuple(int(d) for d in np.broadcast_shapes(x.shape, target)))]


def _expand_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    shape = np.broadcast_shapes(x.shape, tuple(int_list(_need(xs, 1))))
    return [contiguous(np.broadcast_to(x, shape))]


_register("Expand", _expand_infer, _expand_run)


def _tile_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x = _type(types, 0)
    reps = int_list(_known(consts, 1, "Tile repeats"))
    return [TensorType(x.dtype, tuple(d * r for d, r in zip(x.shape, reps, strict=True)))]


_register("Tile", _tile_infer, lambda n, xs: [np.tile(_need(xs, 0), int_list(_need(xs, 1)))])


def range_values(start: np.ndarray, limit: np.ndarray, delta: np.ndarray) -> np.ndarray:
    s, lim, d = (np.asarray(v).reshape(()) for v in (start, limit, delta))
    count = max(math.ceil((float(lim) - float(s)) / float(d)), 0)
    return np.asarray(s + np.arange(count, dtype=s.dtype) * d, dtype=s.dtype)


_register(
    "Range",
    lambda n, t, c: [
        TensorType(
            _type(t, 0).dtype,
            range_values(_known(c, 0, "Range"), _known(c, 1, "Range"), _known(c, 2, "Range")).shape,
        )
    ],
    lambda n, xs: [range_values(_need(xs, 0), _need(xs, 1), _need(xs, 2))],
)


def _trilu_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    k = int(np.asarray(xs[1]).reshape(())) if len(xs) > 1 and xs[1] is not None else 0
    return [np.triu(x, k) if int(node.attrs.get("upper", 1)) else np.tril(x, k)]


_register("Trilu", _same_infer, _trilu_run)


def pad_amounts(node: Node, rank: int, consts: Sequence[np.ndarray | None]) -> list[int]:
    consts = list(consts)
    if "pads" in node.attrs:
        pads = [int(p) for p in node.attrs["pads"]]
    else:
        pads = int_list(_known(consts, 1, "Pad pads"))
    if len(consts) > 3 and consts[3] is not None:
        axes = [norm_axis(a, rank) for a in int_list(consts[3])]
        full = [0] * (2 * rank)
        for i, a in enumerate(axes):
            full[a] = pads[i]
            full[a + rank] = pads[i + len(axes)]
        pads = full
    return pads


def _pad_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x = _type(types, 0)
    p = pad_amounts(node, x.rank, consts)
    return [TensorType(x.dtype, tuple(d + p[i] + p[i + x.rank] for i, d in enumerate(x.shape)))]


def _pad_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    mode = node.attrs.get("mode", "constant")
    if mode != "constant":
        raise UnsupportedOpError(f"Pad mode {mode!r} is not supported")
    p = pad_amounts(node, x.ndim, xs)
    fill = float(np.asarray(xs[2]).reshape(())) if len(xs) > 2 and xs[2] is not None else 0.0
    return [np.pad(x, [(p[i], p[i + x.ndim]) for i in range(x.ndim)], constant_values=fill)]


_register("Pad", _pad_infer, _pad_run)


# ---------------------------------------------------------------------------------------------
# reductions and normalization
# ---------------------------------------------------------------------------------------------
def reduce_axes(node: Node, rank: int, consts: Sequence[np.ndarray | None]) -> tuple[int, ...]:
    axes = axes_argument(node, consts, 1)
    if not axes:
        if int(node.attrs.get("noop_with_empty_axes", 0)):
            return ()
        return tuple(range(rank))
    return tuple(sorted(norm_axis(a, rank) for a in axes))


def _reduce_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x = _type(types, 0)
    axes = reduce_axes(node, x.rank, consts)
    keep = int(node.attrs.get("keepdims", 1))
    shape = tuple(1 if i in axes else d for i, d in enumerate(x.shape) if keep or i not in axes)
    return [TensorType(x.dtype, shape)]


def _reducer(fn: Callable[..., np.ndarray]) -> EvalFn:
    def run(node: Node, xs: Arrays) -> list[np.ndarray]:
        x = _need(xs, 0)
        axes = reduce_axes(node, x.ndim, xs)
        if not axes:
            return [x.copy()]
        keep = bool(int(node.attrs.get("keepdims", 1)))
        return [keep_dtype(fn(x, axis=axes, keepdims=keep), x)]

    return run


for _op, _rfn in (
    ("ReduceMean", np.mean),
    ("ReduceSum", np.sum),
    ("ReduceMax", np.max),
    ("ReduceMin", np.min),
    ("ReduceProd", np.prod),
):
    _register(_op, _reduce_infer, _reducer(_rfn))


def _argmax_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x = _type(types, 0)
    axis = norm_axis(int(node.attrs.get("axis", 0)), x.rank)
    keep = int(node.attrs.get("keepdims", 1))
    shape = tuple(1 if i == axis else d for i, d in enumerate(x.shape) if keep or i != axis)
    return [TensorType("int64", shape)]


def _argmax_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    axis = norm_axis(int(node.attrs.get("axis", 0)), x.ndim)
    result = np.argmax(x, axis=axis)
    if int(node.attrs.get("keepdims", 1)):
        result = np.expand_dims(result, axis)
    return [result.astype(np.int64)]


_register("ArgMax", _argmax_infer, _argmax_run)


def softmax(x: np.ndarray, axis: int) -> np.ndarray:
    shifted = np.exp(x - np.max(x, axis=axis, keepdims=True))
    return keep_dtype(shifted / np.sum(shifted, axis=axis, keepdims=True), x)


def _softmax_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    return [softmax(x, norm_axis(int(node.attrs.get("axis", -1)), x.ndim))]


def _log_softmax_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    axis = norm_axis(int(node.attrs.get("axis", -1)), x.ndim)
    m = np.max(x, axis=axis, keepdims=True)
    return [keep_dtype(x - m - np.log(np.sum(np.exp(x - m), axis=axis, keepdims=True)), x)]


_register("Softmax", _same_infer, _softmax_run)
_register("LogSoftmax", _same_infer, _log_softmax_run)


def layer_norm(
    x: np.ndarray, scale: np.ndarray | None, bias: np.ndarray | None, axis: int, eps: float
) -> np.ndarray:
    axes = tuple(range(axis, x.ndim))
    x64 = x.astype(np.float64)
    mean = x64.mean(axis=axes, keepdims=True)
    var = ((x64 - mean) ** 2).mean(axis=axes, keepdims=True)
    y = (x64 - mean) / np.sqrt(var + eps)
    if scale is not None:
        y = y * scale
    if bias is not None:
        y = y + bias
    return keep_dtype(y, x)


def _ln_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    if len(node.outputs) > 1:
        raise UnsupportedOpError("LayerNormalization mean and inverse std outputs")
    return [_type(types, 0)]


def _ln_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    axis = norm_axis(int(node.attrs.get("axis", -1)), x.ndim)
    eps = float(node.attrs.get("epsilon", 1e-5))
    return [layer_norm(x, _maybe(xs, 1), _maybe(xs, 2), axis, eps)]


_register("LayerNormalization", _ln_infer, _ln_run)


def _bn_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x, scale, bias, mean, var = (_need(xs, i) for i in range(5))
    eps = float(node.attrs.get("epsilon", 1e-5))
    channel = x.ndim - 1 if node.attrs.get("layout") == "NHWC" else 1
    shape = [1] * x.ndim
    shape[channel] = -1
    inv = (scale / np.sqrt(var + eps)).reshape(shape)
    return [keep_dtype((x - mean.reshape(shape)) * inv + bias.reshape(shape), x)]


_register("BatchNormalization", lambda n, t, c: [_type(t, 0)], _bn_run)


# ---------------------------------------------------------------------------------------------
# matrix products
# ---------------------------------------------------------------------------------------------
def matmul_shape(a: tuple[int, ...], b: tuple[int, ...]) -> tuple[int, ...]:
    if not a or not b:
        raise ShapeError("MatMul operands must have rank >= 1")
    a2 = (1, *a) if len(a) == 1 else a
    b2 = (*b, 1) if len(b) == 1 else b
    if a2[-1] != b2[-2]:
        raise ShapeError(f"MatMul inner dimensions differ: {a} x {b}")
    out = [*np.broadcast_shapes(a2[:-2], b2[:-2]), a2[-2], b2[-1]]
    if len(a) == 1:
        out.pop(-2)
    if len(b) == 1:
        out.pop(-1)
    return tuple(int(d) for d in out)


_register(
    "MatMul",
    lambda n, t, c: [TensorType(_type(t, 0).dtype, matmul_shape(_type(t, 0).shape, _type(t, 1).shape))],
    lambda n, xs: [keep_dtype(np.matmul(_need(xs, 0), _need(xs, 1)), _need(xs, 0))],
)


def _gemm_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    a, b = _type(types, 0), _type(types, 1)
    ta = int(node.attrs.get("transA", 0))
    m, k = (a.shape[1], a.shape[0]) if ta else (a.shape[0], a.shape[1])
    kb, n = (b.shape[1], b.shape[0]) if int(node.attrs.get("transB", 0)) else b.shape
    if k != kb:
        raise ShapeError(f"Gemm inner dimensions differ: {a.shape} x {b.shape}")
    return [TensorType(a.dtype, (m, n))]


def _gemm_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    a, b, c = _need(xs, 0), _need(xs, 1), _maybe(xs, 2)
    if int(node.attrs.get("transA", 0)):
        a = a.T
    if int(node.attrs.get("transB", 0)):
        b = b.T
    y = float(node.attrs.get("alpha", 1.0)) * (a @ b)
    if c is not None:
        y = y + float(node.attrs.get("beta", 1.0)) * c
    return [keep_dtype(y, a)]


_register("Gemm", _gemm_infer, _gemm_run)


def apply_activation(y: np.ndarray, node: Node) -> np.ndarray:
    act = str(node.attrs.get("activation", "none"))
    if act == "none":
        return y
    if act == "relu":
        return np.asarray(np.maximum(y, 0), dtype=y.dtype)
    if act == "clip":
        lo = float(node.attrs.get("clip_min", 0.0))
        hi = float(node.attrs.get("clip_max", 6.0))
        return np.asarray(np.clip(y, lo, hi), dtype=y.dtype)
    if act == "gelu":
        return gelu(y, "none")
    if act == "gelu_tanh":
        return gelu(y, "tanh")
    if act == "tanh":
        return np.tanh(y)
    if act == "sigmoid":
        return sigmoid(y)
    raise UnsupportedOpError(f"activation {act!r}")


def _fused_gemm_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    a, b = _type(types, 0), _type(types, 1)
    k, n = (b.shape[1], b.shape[0]) if int(node.attrs.get("trans_b", 0)) else b.shape
    if b.rank != 2 or a.shape[-1] != k:
        raise ShapeError(f"FusedGemm shapes: {a.shape} x {b.shape}")
    return [TensorType(a.dtype, (*a.shape[:-1], n))]


def _fused_gemm_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    a, b, bias, residual = _need(xs, 0), _need(xs, 1), _maybe(xs, 2), _maybe(xs, 3)
    if int(node.attrs.get("trans_b", 0)):
        b = b.T
    y = a @ b
    if bias is not None:
        y = y + bias
    if residual is not None:
        y = y + residual
    return [keep_dtype(apply_activation(y, node), a)]


_register("FusedGemm", _fused_gemm_infer, _fused_gemm_run)


# ---------------------------------------------------------------------------------------------
# convolution and pooling
# ---------------------------------------------------------------------------------------------
@dataclass(frozen=True)
class Conv2dGeometry:
    """2-D window geometry; pads are (top, left, bottom, right)."""

    kernel: tuple[int, int]
    strides: tuple[int, int]
    dilations: tuple[int, int]
    pads: tuple[int, int, int, int]
    out_hw: tuple[int, int]


def window_geometry(
    node: Node, in_hw: tuple[int, int], kernel: tuple[int, int], ceil_mode: bool = False
) -> Conv2dGeometry:
    strides = [int(s) for s in node.attrs.get("strides", (1, 1))]
    dil = [int(d) for d in node.attrs.get("dilations", (1, 1))]
    pads = [int(p) for p in node.attrs.get("pads", (0, 0, 0, 0))]
    if len(strides) != 2 or len(dil) != 2 or len(pads) != 4:
        raise UnsupportedOpError(f"{node.op}: only 2-D windows are supported")
    span = [(kernel[i] - 1) * dil[i] + 1 for i in range(2)]
    auto_pad = node.attrs.get("auto_pad", "NOTSET")
    if auto_pad in ("SAME_UPPER", "SAME_LOWER"):
        total = []
        for i in range(2):
            out = -(-in_hw[i] // strides[i])
            total.append(max((out - 1) * strides[i] + span[i] - in_hw[i], 0))
        small = [t // 2 for t in total]
        large = [t - t // 2 for t in total]
        pads = small + large if auto_pad == "SAME_UPPER" else large + small
    elif auto_pad == "VALID":
        pads = [0, 0, 0, 0]
    out_hw = []
    for i in range(2):
        room = in_hw[i] + pads[i] + pads[i + 2] - span[i]
        if room < 0:
            raise ShapeError(f"{node.op}: window larger than the padded input")
        o = (-(-room // strides[i]) if ceil_mode else room // strides[i]) + 1
        if ceil_mode and (o - 1) * strides[i] >= in_hw[i] + pads[i]:
            o -= 1
        out_hw.append(o)
    return Conv2dGeometry(
        (kernel[0], kernel[1]),
        (strides[0], strides[1]),
        (dil[0], dil[1]),
        (pads[0], pads[1], pads[2], pads[3]),
        (out_hw[0], out_hw[1]),
    )


def conv_layout(node: Node) -> str:
    layout = str(node.attrs.get("layout", "NCHW"))
    if layout not in ("NCHW", "NHWC"):
        raise UnsupportedOpError(f"layout {layout!r}")
    return layout


def conv_dims(node: Node, x: TensorType, w: TensorType) -> tuple[int, int, int, Conv2dGeometry]:
    """(batch, out channels, in channels, geometry) of a Conv / FusedConv."""
    if x.rank != 4 or w.rank != 4:
        raise UnsupportedOpError(f"{node.op}: only 2-D convolution (rank 4) is supported")
    group = int(node.attrs.get("group", 1))
    if conv_layout(node) == "NHWC":
        n, h, wd, c = x.shape
        kh, kw, cg, k = w.shape
    else:
        n, c, h, wd = x.shape
        k, cg, kh, kw = w.shape
    if cg * group != c or k % group:
        raise ShapeError(f"{node.op}: channels {c} do not match weights {w.shape} with group {group}")
    return n, k, c, window_geometry(node, (h, wd), (kh, kw))


def _conv_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x, w = _type(types, 0), _type(types, 1)
    n, k, _, g = conv_dims(node, x, w)
    oh, ow = g.out_hw
    shape = (n, oh, ow, k) if conv_layout(node) == "NHWC" else (n, k, oh, ow)
    return [TensorType(x.dtype, shape)]


def conv2d_nchw(x: np.ndarray, w: np.ndarray, g: Conv2dGeometry, group: int) -> np.ndarray:
    """Grouped NCHW x OIHW convolution through a strided window view and one einsum."""
    n = x.shape[0]
    k, cg, kh, kw = w.shape
    pt, pl, pb, pr = g.pads
    padded = np.pad(x, ((0, 0), (0, 0), (pt, pb), (pl, pr)))
    (dh, dw), (sh, sw), (oh, ow) = g.dilations, g.strides, g.out_hw
    windows = np.lib.stride_tricks.sliding_window_view(
        padded, ((kh - 1) * dh + 1, (kw - 1) * dw + 1), axis=(2, 3)
    )[:, :, : (oh - 1) * sh + 1 : sh, : (ow - 1) * sw + 1 : sw, ::dh, ::dw]
    windows = windows.reshape(n, group, cg, oh, ow, kh, kw)
    out = np.einsum("ngchwij,gkcij->ngkhw", windows, w.reshape(group, k // group, cg, kh, kw), optimize=True)
    return contiguous(out.reshape(n, k, oh, ow), dtype=x.dtype)


def _conv_core(node: Node, x: np.ndarray, w: np.ndarray, b: np.ndarray | None) -> np.ndarray:
    nhwc = conv_layout(node) == "NHWC"
    xn = x.transpose(0, 3, 1, 2) if nhwc else x
    wn = w.transpose(3, 2, 0, 1) if nhwc else w
    g = window_geometry(node, (xn.shape[2], xn.shape[3]), (wn.shape[2], wn.shape[3]))
    y = conv2d_nchw(xn, wn, g, int(node.attrs.get("group", 1)))
    if b is not None:
        y = y + b.reshape(1, -1, 1, 1)
    return y.transpose(0, 2, 3, 1) if nhwc else y


def _conv_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    return [keep_dtype(contiguous(_conv_core(node, x, _need(xs, 1), _maybe(xs, 2))), x)]


def _fused_conv_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    x = _need(xs, 0)
    y = _conv_core(node, x, _need(xs, 1), _maybe(xs, 2))
    residual = _maybe(xs, 3)
    if residual is not None:
        y = y + residual
    return [keep_dtype(contiguous(apply_activation(y, node)), x)]


_register("Conv", _conv_infer, _conv_run)
_register("FusedConv", _conv_infer, _fused_conv_run)


def pool_dims(node: Node, x: TensorType) -> tuple[Conv2dGeometry, tuple[int, ...]]:
    if x.rank != 4:
        raise UnsupportedOpError(f"{node.op}: only 2-D pooling is supported")
    kernel = [int(k) for k in node.attrs["kernel_shape"]]
    nhwc = conv_layout(node) == "NHWC"
    hw = (x.shape[1], x.shape[2]) if nhwc else (x.shape[2], x.shape[3])
    g = window_geometry(node, hw, (kernel[0], kernel[1]), bool(node.attrs.get("ceil_mode", 0)))
    oh, ow = g.out_hw
    shape = (x.shape[0], oh, ow, x.shape[3]) if nhwc else (x.shape[0], x.shape[1], oh, ow)
    return g, shape


def _pool_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    if len(node.outputs) > 1:
        raise UnsupportedOpError("MaxPool indices output is not supported")
    x = _type(types, 0)
    return [TensorType(x.dtype, pool_dims(node, x)[1])]


def _pool(node: Node, x: np.ndarray, kind: str) -> np.ndarray:
    nhwc = conv_layout(node) == "NHWC"
    xn = x.transpose(0, 3, 1, 2) if nhwc else x
    g, _ = pool_dims(node, TensorType.of(x))
    pt, pl, pb, pr = g.pads
    (kh, kw), (sh, sw), (dh, dw), (oh, ow) = g.kernel, g.strides, g.dilations, g.out_hw
    extra_b = max((oh - 1) * sh + (kh - 1) * dh + 1 - (xn.shape[2] + pt + pb), 0)
    extra_r = max((ow - 1) * sw + (kw - 1) * dw + 1 - (xn.shape[3] + pl + pr), 0)
    fill = -np.inf if kind == "max" else 0.0
    padded = np.pad(
        xn, ((0, 0), (0, 0), (pt, pb + extra_b), (pl, pr + extra_r)), constant_values=fill
    )
    win = np.lib.stride_tricks.sliding_window_view(
        padded, ((kh - 1) * dh + 1, (kw - 1) * dw + 1), axis=(2, 3)
    )[:, :, : (oh - 1) * sh + 1 : sh, : (ow - 1) * sw + 1 : sw, ::dh, ::dw]
    if kind == "max":
        y = win.max(axis=(4, 5))
    else:
        ones = np.ones(xn.shape[2:], dtype=np.float64)
        if int(node.attrs.get("count_include_pad", 0)):
            ones = np.pad(ones, ((pt, pb), (pl, pr)), constant_values=1)
            ones = np.pad(ones, ((0, extra_b), (0, extra_r)))
        else:
            ones = np.pad(ones, ((pt, pb + extra_b), (pl, pr + extra_r)))
        counts = np.lib.stride_tricks.sliding_window_view(
            ones, ((kh - 1) * dh + 1, (kw - 1) * dw + 1)
        )[: (oh - 1) * sh + 1 : sh, : (ow - 1) * sw + 1 : sw, ::dh, ::dw].sum(axis=(2, 3))
        y = win.sum(axis=(4, 5)) / counts
    y = contiguous(y.astype(x.dtype))
    return contiguous(y.transpose(0, 2, 3, 1)) if nhwc else y


_register("MaxPool", _pool_infer, lambda n, xs: [_pool(n, _need(xs, 0), "max")])
_register("AveragePool", _pool_infer, lambda n, xs: [_pool(n, _need(xs, 0), "avg")])


def _global_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    x = _type(types, 0)
    if x.rank < 3:
        raise ShapeError(f"{node.op} needs rank >= 3")
    if conv_layout(node) == "NHWC":
        return [TensorType(x.dtype, (x.shape[0], *([1] * (x.rank - 2)), x.shape[-1]))]
    return [TensorType(x.dtype, (*x.shape[:2], *([1] * (x.rank - 2))))]


def spatial_axes(node: Node, rank: int) -> tuple[int, ...]:
    return tuple(range(1, rank - 1)) if conv_layout(node) == "NHWC" else tuple(range(2, rank))


_register(
    "GlobalAveragePool",
    _global_infer,
    lambda n, xs: [
        keep_dtype(_need(xs, 0).mean(axis=spatial_axes(n, _need(xs, 0).ndim), keepdims=True), _need(xs, 0))
    ],
)
_register(
    "GlobalMaxPool",
    _global_infer,
    lambda n, xs: [_need(xs, 0).max(axis=spatial_axes(n, _need(xs, 0).ndim), keepdims=True)],
)


# ---------------------------------------------------------------------------------------------
# fused elementwise programs (loop fusion output)
# ---------------------------------------------------------------------------------------------
# ``program`` is a list of [op, attrs, args]; arg a < len(inputs) is node input a, a larger arg
# is the result of instruction a - len(inputs), and -1 is an omitted optional input. The last
# instruction's result is the node's output.
def program_nodes(node: Node) -> list[tuple[Node, list[int]]]:
    program = node.attrs.get("program")
    if not program:
        raise UnsupportedOpError("FusedElementwise without a program")
    result = []
    for op, attrs, args in program:
        if not is_elementwise(str(op)):
            raise UnsupportedOpError(f"FusedElementwise: {op} is not elementwise")
        result.append((Node(str(op), [], [_PLACEHOLDER], dict(attrs)), [int(a) for a in args]))
    return result


def _fused_ew_infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    ts = list(types)
    cs = list(consts)
    for sub, args in program_nodes(node):
        ts.append(
            spec(sub.op).infer(
                sub, [ts[a] if a >= 0 else None for a in args], [cs[a] if a >= 0 else None for a in args]
            )[0]
        )
        cs.append(None)
    return [ts[-1]]


def _fused_ew_run(node: Node, xs: Arrays) -> list[np.ndarray]:
    vals = list(xs)
    for sub, args in program_nodes(node):
        vals.append(spec(sub.op).run(sub, [vals[a] if a >= 0 else None for a in args])[0])
    return [vals[-1]]


_register("FusedElementwise", _fused_ew_infer, _fused_ew_run)


# ---------------------------------------------------------------------------------------------
# public entry points
# ---------------------------------------------------------------------------------------------
def infer(node: Node, types: Types, consts: Arrays) -> list[TensorType]:
    out = spec(node.op).infer(node, types, consts)
    if len(out) < len(node.outputs):
        raise ShapeError(f"{node.op}: inferred {len(out)} outputs, node has {len(node.outputs)}")
    return out[: len(node.outputs)]


def run(node: Node, arrays: Arrays) -> list[np.ndarray]:
    """Compile-time evaluation of one node (constant folding and shape arithmetic)."""
    return spec(node.op).run(node, arrays)


def is_elementwise(op: str) -> bool:
    s = REGISTRY.get(op)
    return bool(s is not None and s.elementwise)


def flops(node: Node) -> int:
    """Floating point operations of one node, a multiply-add counting as 2."""
    out = node.outputs[0].type
    if out is None:
        return 0
    if node.op in ("Conv", "FusedConv"):
        w = node.input(1).tensor_type
        per_output = w.size // (w.shape[3] if conv_layout(node) == "NHWC" else w.shape[0])
        return 2 * out.size * per_output
    if node.op == "FusedElementwise":
        return out.size * len(node.attrs.get("program", ()))
    if node.op in ("MatMul", "FusedGemm", "Gemm"):
        a = node.input(0).tensor_type
        k = a.shape[0] if node.op == "Gemm" and int(node.attrs.get("transA", 0)) else a.shape[-1]
        return 2 * out.size * k
    return out.size
