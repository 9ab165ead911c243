"""CPU oracle: a numpy restatement of the reference interpreter's operator semantics.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
may import this module, and only as the checker. The compiler never calls it.

Follows src/ml_graph_compiler/interpreter.py:1-141 (node-by-node execution, feed checks,
random_feeds) and the ``run`` functions of src/ml_graph_compiler/ops.py:122-1202, restated
independently of the product's compile-time evaluator:

* contractions (MatMul, Gemm, FusedGemm, Conv, FusedConv) accumulate in float64 through an
  explicit im2col matrix and cast to the first operand's dtype, so the oracle is closer to the
  exact result than any fp32 summation order (the reference's own np.matmul/einsum order is
  BLAS-dependent, so it is pinned only to tolerance);
* pooling walks the kernel window position by position with validity masks (ONNX rules,
  count_include_pad, ceil mode) instead of padded window views;
* every other operator keeps the reference's dtype rules: results take the first operand's
  dtype (``_keep``), integer Div truncates, LayerNorm runs in float64, erf is the rational
  approximation with the coefficients of ops.py:201-216, ArgMax takes the first maximum,
  Gather wraps negative indices and raises on out-of-range ones.
"""

from __future__ import annotations

import math
from collections.abc import Mapping

import numpy as np

ERF_P = (-2.72614225801306e-10, 2.77068142495902e-08, -2.10102402082508e-06, -5.69250639462346e-05,
         -7.34990630326855e-04, -2.95459980854025e-03, -1.60960333262415e-02)
ERF_Q = (-1.45660718464996e-05, -2.13374055278905e-04, -1.68282697438203e-03, -7.37332916720468e-03,
         -1.42647390514189e-02)

CAST = {1: "float32", 2: "uint8", 3: "int8", 6: "int32", 7: "int64", 9: "bool", 10: "float16", 11: "float64"}


class OracleError(Exception):
    """Raised for invalid feeds or an out-of-range Gather index (the reference's GraphError)."""


def _keep(x, like):
    return np.asarray(x, dtype=like.dtype)


def erf(x):
    """erf(x) = x P(x^2) / Q(x^2) on [-4, 4], clamped outside (ops.py:201-229)."""
    t = np.clip(np.asarray(x, np.float64), -4.0, 4.0)
    z = t * t
    p = np.zeros_like(t) + ERF_P[0]
    for c in ERF_P[1:]:
        p = p * z + c
    q = np.zeros_like(t) + ERF_Q[0]
    for c in ERF_Q[1:]:
        q = q * z + c
    return np.asarray(t * p / q, dtype=np.asarray(x).dtype)


def gelu(x, approximate="none"):
    if approximate == "tanh":
        c = math.sqrt(2.0 / math.pi)
        return _keep(0.5 * x * (1.0 + np.tanh(c * (x + 0.044715 * x * x * x))), x)
    return _keep(0.5 * x * (1.0 + erf(x / math.sqrt(2.0))), x)


def sigmoid(x):
    return _keep(0.5 * (1.0 + np.tanh(0.5 * x)), x)


def activation(y, attrs):
    act = str(attrs.get("activation", "none"))
    if act == "none":
        return y
    if act == "relu":
        return np.asarray(np.maximum(y, 0), dtype=y.dtype)
    if act == "clip":
        return np.asarray(np.clip(y, float(attrs.get("clip_min", 0.0)), float(attrs.get("clip_max", 6.0))), dtype=y.dtype)
    if act == "gelu":
        return gelu(y)
    if act == "gelu_tanh":
        return gelu(y, "tanh")
    if act == "tanh":
        return np.tanh(y)
    if act == "sigmoid":
        return sigmoid(y)
    raise OracleError(f"activation {act!r}")


def _axis(a, rank):
    return a + rank if a < 0 else a


def _ints(v):
    return [int(t) for t in np.asarray(v).reshape(-1)]


# ---------------------------------------------------------------------------------------------
# windows (ONNX Conv/Pool geometry: ops.py:951-987)
# ---------------------------------------------------------------------------------------------
def geometry(attrs, in_hw, kernel, ceil_mode=False):
    strides = [int(s) for s in attrs.get("strides", (1, 1))]
    dil = [int(d) for d in attrs.get("dilations", (1, 1))]
    pads = [int(p) for p in attrs.get("pads", (0, 0, 0, 0))]
    span = [(kernel[i] - 1) * dil[i] + 1 for i in range(2)]
    mode = attrs.get("auto_pad", "NOTSET")
    if mode in ("SAME_UPPER", "SAME_LOWER"):
        tot = [max((-(-in_hw[i] // strides[i]) - 1) * strides[i] + span[i] - in_hw[i], 0) for i in range(2)]
        lo = [t // 2 for t in tot]
        hi = [t - t // 2 for t in tot]
        pads = lo + hi if mode == "SAME_UPPER" else hi + lo
    elif mode == "VALID":
        pads = [0, 0, 0, 0]
    out = []
    for i in range(2):
        room = in_hw[i] + pads[i] + pads[i + 2] - span[i]
        o = (-(-room // strides[i]) if ceil_mode else room // strides[i]) + 1
        if ceil_mode and (o - 1) * strides[i] >= in_hw[i] + pads[i]:
            o -= 1
        out.append(o)
    return strides, dil, pads, out


def conv_nchw(x, w, b, attrs):
    """Grouped NCHW convolution as float64 im2col @ weights (OIHW)."""
    n, c, h, wd = x.shape
    k, cg, kh, kw = w.shape
    group = int(attrs.get("group", 1))
    (sh, sw), (dh, dw), pads, (oh, ow) = geometry(attrs, (h, wd), (kh, kw))
    xp = np.zeros((n, c, h + pads[0] + pads[2], wd + pads[1] + pads[3]), np.float64)
    xp[:, :, pads[0] : pads[0] + h, pads[1] : pads[1] + wd] = x
    cols = np.empty((n, c, kh, kw, oh, ow), np.float64)
    for i in range(kh):
        for j in range(kw):
            r0, c0 = i * dh, j * dw
            cols[:, :, i, j] = xp[:, :, r0 : r0 + (oh - 1) * sh + 1 : sh, c0 : c0 + (ow - 1) * sw + 1 : sw]
    kg = k // group
    out = np.empty((n, k, oh, ow), np.float64)
    for g in range(group):
        a = cols[:, g * cg : (g + 1) * cg].transpose(0, 4, 5, 1, 2, 3).reshape(n * oh * ow, cg * kh * kw)
        wm = w[g * kg : (g + 1) * kg].reshape(kg, cg * kh * kw).astype(np.float64)
        out[:, g * kg : (g + 1) * kg] = (a @ wm.T).reshape(n, oh, ow, kg).transpose(0, 3, 1, 2)
    if b is not None:
        out += np.asarray(b, np.float64).reshape(1, -1, 1, 1)
    return out


def conv(x, w, b, attrs):
    """Conv in float64 for NCHW/OIHW or NHWC/HWIO layouts; returns float64 in x's layout."""
    if attrs.get("layout") == "NHWC":
        y = conv_nchw(x.transpose(0, 3, 1, 2), w.transpose(3, 2, 0, 1), b, attrs)
        return y.transpose(0, 2, 3, 1)
    return conv_nchw(x, w, b, attrs)


def pool(x, attrs, kind):
    nhwc = attrs.get("layout") == "NHWC"
    xn = x.transpose(0, 3, 1, 2) if nhwc else x
    n, c, h, wd = xn.shape
    kh, kw = (int(v) for v in attrs["kernel_shape"])
    (sh, sw), (dh, dw), pads, (oh, ow) = geometry(attrs, (h, wd), (kh, kw), bool(attrs.get("ceil_mode", 0)))
    include = int(attrs.get("count_include_pad", 0))
    acc = np.full((n, c, oh, ow), -np.inf if kind == "max" else 0.0, np.float64)
    count = np.zeros((oh, ow), np.float64)
    rows = np.arange(oh) * sh - pads[0]
    cols = np.arange(ow) * sw - pads[1]
    for i in range(kh):
        ih = rows + i * dh
        in_h = (ih >= 0) & (ih < h)
        pad_h = (ih >= -pads[0]) & (ih < h + pads[2])
        for j in range(kw):
            iw = cols + j * dw
            in_w = (iw >= 0) & (iw < wd)
            pad_w = (iw >= -pads[1]) & (iw < wd + pads[3])
            valid = in_h[:, None] & in_w[None, :]
            count += (pad_h[:, None] & pad_w[None, :]) if include else valid
            vals = xn[:, :, np.clip(ih, 0, h - 1)][:, :, :, np.clip(iw, 0, wd - 1)].astype(np.float64)
            if kind == "max":
                acc = np.where(valid, np.maximum(acc, vals), acc)
            else:
                acc = acc + np.where(valid, vals, 0.0)
    y = acc if kind == "max" else acc / count
    y = y.astype(x.dtype)
    return np.ascontiguousarray(y.transpose(0, 2, 3, 1)) if nhwc else y


# ---------------------------------------------------------------------------------------------
# shape helpers
# ---------------------------------------------------------------------------------------------
def reshape_to(shape_in, spec, allowzero=0):
    out = [int(d) for d in spec]
    for i, d in enumerate(out):
        if d == 0 and not allowzero:
            out[i] = shape_in[i]
    if -1 in out:
        rest = int(np.prod([d for d in out if d != -1]))
        out[out.index(-1)] = int(np.prod(shape_in)) // rest
    return tuple(out)


def slices(attrs, shape, xs):
    if "starts" in attrs:
        starts, ends = list(attrs["starts"]), list(attrs["ends"])
        axes = list(attrs.get("axes", range(len(starts))))
        steps = [1] * len(starts)
    else:
        starts, ends = _ints(xs[1]), _ints(xs[2])
        axes = _ints(xs[3]) if len(xs) > 3 and xs[3] is not None else list(range(len(starts)))
        steps = _ints(xs[4]) if len(xs) > 4 and xs[4] is not None else [1] * len(starts)
    sl = [slice(None)] * len(shape)
    for s, e, a, st in zip(starts, ends, axes, steps):
        a = _axis(int(a), len(shape))
        d = shape[a]
        s = max(-d - 1, min(d, int(s)))
        e = max(-d - 1, min(d, int(e)))
        b0, b1, b2 = slice(s, e, int(st)).indices(d)
        sl[a] = slice(b0, b1 if b1 >= 0 else None, b2)
    return tuple(sl)


def axes_of(attrs, xs, index):
    if "axes" in attrs:
        return [int(a) for a in attrs["axes"]]
    if len(xs) > index and xs[index] is not None:
        return _ints(xs[index])
    return None


def clip_bounds(attrs, xs):
    lo, hi = attrs.get("min", -np.inf), attrs.get("max", np.inf)
    if len(xs) > 1 and xs[1] is not None:
        lo = float(np.asarray(xs[1]).reshape(()))
    if len(xs) > 2 and xs[2] is not None:
        hi = float(np.asarray(xs[2]).reshape(()))
    return float(lo), float(hi)


# ---------------------------------------------------------------------------------------------
# operators: (node-like op, attrs, inputs, n_outputs) -> list of arrays
# ---------------------------------------------------------------------------------------------
def _binary(fn):
    return lambda at, xs, no: [_keep(fn(xs[0], xs[1]), xs[0])]


def _unary(fn):
    return lambda at, xs, no: [_keep(fn(xs[0]), xs[0])]


def _bool(fn):
    return lambda at, xs, no: [np.asarray(fn(xs[0], xs[1]), dtype=np.bool_)]


def _div(at, xs, no):
    a, b = xs[0], xs[1]
    if np.issubdtype(a.dtype, np.integer):
        return [np.asarray(np.trunc(a / b), dtype=a.dtype)]
    return [_keep(a / b, a)]


def _gather(at, xs, no):
    x, idx = xs[0], xs[1]
    axis = _axis(int(at.get("axis", 0)), x.ndim)
    idx = np.where(idx < 0, idx + x.shape[axis], idx)
    if idx.size and (idx.min() < 0 or idx.max() >= x.shape[axis]):
        raise OracleError(f"Gather index out of range for axis {axis} of size {x.shape[axis]}")
    return [np.take(x, idx, axis=axis)]


def _split(at, xs, no):
    x = xs[0]
    axis = _axis(int(at.get("axis", 0)), x.ndim)
    if "split" in at:
        sizes = [int(s) for s in at["split"]]
    elif len(xs) > 1 and xs[1] is not None:
        sizes = _ints(xs[1])
    elif "num_outputs" in at:
        k = int(at["num_outputs"])
        ch = -(-x.shape[axis] // k)
        sizes = [ch] * (k - 1) + [x.shape[axis] - ch * (k - 1)]
    else:
        sizes = [x.shape[axis] // no] * no
    return [p.copy() for p in np.split(x, np.cumsum(sizes)[:-1], axis=axis)]


def _reduce(fn):
    def run(at, xs, no):
        x = xs[0]
        axes = axes_of(at, xs, 1)
        if not axes:
            if int(at.get("noop_with_empty_axes", 0)):
                return [x.copy()]
            axes = list(range(x.ndim))
        axes = tuple(sorted(_axis(a, x.ndim) for a in axes))
        return [_keep(fn(x, axis=axes, keepdims=bool(int(at.get("keepdims", 1)))), x)]

    return run


def _argmax(at, xs, no):
    x = xs[0]
    axis = _axis(int(at.get("axis", 0)), x.ndim)
    out = np.argmax(x, axis=axis)
    if int(at.get("keepdims", 1)):
        out = np.expand_dims(out, axis)
    return [out.astype(np.int64)]


def _softmax(at, xs, no, log=False):
    x = xs[0]
    axis = _axis(int(at.get("axis", -1)), x.ndim)
    m = np.max(x, axis=axis, keepdims=True)
    if log:
        return [_keep(x - m - np.log(np.sum(np.exp(x - m), axis=axis, keepdims=True)), x)]
    e = np.exp(x - m)
    return [_keep(e / np.sum(e, axis=axis, keepdims=True), x)]


def _layer_norm(at, xs, no):
    x = xs[0]
    axis = _axis(int(at.get("axis", -1)), x.ndim)
    axes = tuple(range(axis, x.ndim))
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=axes, keepdims=True)
    var = ((x64 - mu) ** 2).mean(axis=axes, keepdims=True)
    y = (x64 - mu) / np.sqrt(var + float(at.get("epsilon", 1e-5)))
    if len(xs) > 1 and xs[1] is not None:
        y = y * xs[1]
    if len(xs) > 2 and xs[2] is not None:
        y = y + xs[2]
    return [_keep(y, x)]


def _batch_norm(at, xs, no):
    x, s, b, m, v = xs[:5]
    ch = x.ndim - 1 if at.get("layout") == "NHWC" else 1
    shape = [1] * x.ndim
    shape[ch] = -1
    inv = (s / np.sqrt(v + float(at.get("epsilon", 1e-5)))).reshape(shape)
    return [_keep((x - m.reshape(shape)) * inv + b.reshape(shape), x)]


def _matmul(at, xs, no):
    a, b = xs[0], xs[1]
    return [_keep(np.matmul(a.astype(np.float64), b.astype(np.float64)), a)]


def _gemm(at, xs, no):
    a, b = xs[0], xs[1]
    c = xs[2] if len(xs) > 2 else None
    a64 = (a.T if int(at.get("transA", 0)) else a).astype(np.float64)
    b64 = (b.T if int(at.get("transB", 0)) else b).astype(np.float64)
    y = float(at.get("alpha", 1.0)) * (a64 @ b64)
    if c is not None:
        y = y + float(at.get("beta", 1.0)) * c
    return [_keep(y, a)]


def _fused_gemm(at, xs, no):
    a, b = xs[0], xs[1]
    bias = xs[2] if len(xs) > 2 else None
    res = xs[3] if len(xs) > 3 else None
    b64 = (b.T if int(at.get("trans_b", 0)) else b).astype(np.float64)
    y = a.astype(np.float64) @ b64
    if bias is not None:
        y = y + bias
    if res is not None:
        y = y + res
    return [_keep(activation(_keep(y, a), at), a)]


def _conv(at, xs, no, fused=False):
    x = xs[0]
    b = xs[2] if len(xs) > 2 else None
    y = conv(x, xs[1], b, at)
    if fused and len(xs) > 3 and xs[3] is not None:
        y = y + xs[3]
    y = _keep(y, x)
    return [np.ascontiguousarray(activation(y, at) if fused else y)]


def _global(at, xs, no, kind):
    x = xs[0]
    axes = tuple(range(1, x.ndim - 1)) if at.get("layout") == "NHWC" else tuple(range(2, x.ndim))
    if kind == "max":
        return [x.max(axis=axes, keepdims=True)]
    return [_keep(x.mean(axis=axes, keepdims=True), x)]


def _pad(at, xs, no):
    x = xs[0]
    pads = [int(p) for p in at["pads"]] if "pads" in at else _ints(xs[1])
    if len(xs) > 3 and xs[3] is not None:
        full = [0] * (2 * x.ndim)
        axes = [_axis(a, x.ndim) for a in _ints(xs[3])]
        for i, a in enumerate(axes):
            full[a], full[a + x.ndim] = pads[i], pads[i + len(axes)]
        pads = full
    if at.get("mode", "constant") != "constant":
        raise OracleError("Pad mode")
    fill = float(np.asarray(xs[2]).reshape(())) if len(xs) > 2 and xs[2] is not None else 0.0
    return [np.pad(x, [(pads[i], pads[i + x.ndim]) for i in range(x.ndim)], constant_values=fill)]


def _shape(at, xs, no):
    dims = xs[0].shape
    start = int(at.get("start", 0))
    end = at.get("end")
    return [np.asarray(dims[start:] if end is None else dims[start : int(end)], dtype=np.int64)]


def _range(at, xs, no):
    s, lim, d = (np.asarray(v).reshape(()) for v in xs[:3])
    count = max(math.ceil((float(lim) - float(s)) / float(d)), 0)
    return [np.asarray(s + np.arange(count, dtype=s.dtype) * d, dtype=s.dtype)]


def _constant_of_shape(at, xs, no):
    value = at.get("value")
    fill = np.asarray(value).reshape(-1)[0] if value is not None else np.float32(0)
    dtype = value.dtype if isinstance(value, np.ndarray) else np.float32
    return [np.full(tuple(_ints(xs[0])), fill, dtype=dtype)]


def _cast(at, xs, no):
    to = at.get("to", 1)
    return [xs[0].astype(to if isinstance(to, str) else CAST[int(to)])]


def _squeeze(at, xs, no):
    x = xs[0]
    axes = axes_of(at, xs, 1)
    if axes is None:
        return [x.reshape(tuple(d for d in x.shape if d != 1)).copy()]
    drop = {_axis(a, x.ndim) for a in axes}
    return [x.reshape(tuple(d for i, d in enumerate(x.shape) if i not in drop)).copy()]


def _unsqueeze(at, xs, no):
    x = xs[0]
    axes = axes_of(at, xs, 1)
    rank = x.ndim + len(axes)
    shape = list(x.shape)
    for a in sorted(_axis(a, rank) for a in axes):
        shape.insert(a, 1)
    return [x.reshape(shape).copy()]


def _flatten(at, xs, no):
    x = xs[0]
    a = _axis(int(at.get("axis", 1)), x.ndim) if x.ndim else 0
    return [x.reshape(int(np.prod(x.shape[:a])), int(np.prod(x.shape[a:]))).copy()]


def _reshape(at, xs, no):
    x = xs[0]
    spec = list(at["shape"]) if "shape" in at else _ints(xs[1])
    return [x.reshape(reshape_to(x.shape, spec, int(at.get("allowzero", 0)))).copy()]


def _transpose(at, xs, no):
    x = xs[0]
    perm = at.get("perm")
    return [np.ascontiguousarray(x.transpose(list(reversed(range(x.ndim))) if perm is None else [int(p) for p in perm]))]


def _dropout(at, xs, no):
    out = [xs[0].copy()]
    if no > 1:
        out.append(np.ones(xs[0].shape, np.bool_))
    return out


def _fused_elementwise(at, xs, no):
    vals = list(xs)
    for op, sub_attrs, args in at["program"]:
        vals.append(OPS[str(op)](dict(sub_attrs), [vals[a] if a >= 0 else None for a in args], 1)[0])
    return [vals[-1]]


OPS = {
    "Add": _binary(np.add),
    "Sub": _binary(np.subtract),
    "Mul": _binary(np.multiply),
    "Max": _binary(np.maximum),
    "Min": _binary(np.minimum),
    "Div": _div,
    "Pow": lambda at, xs, no: [_keep(np.power(xs[0], xs[1].astype(xs[0].dtype)), xs[0])],
    "Equal": _bool(np.equal),
    "Less": _bool(np.less),
    "Greater": _bool(np.greater),
    "LessOrEqual": _bool(np.less_equal),
    "GreaterOrEqual": _bool(np.greater_equal),
    "And": _bool(np.logical_and),
    "Or": _bool(np.logical_or),
    "Xor": _bool(np.logical_xor),
    "Where": lambda at, xs, no: [_keep(np.where(xs[0], xs[1], xs[2]), xs[1])],
    "Relu": _unary(lambda x: np.maximum(x, 0)),
    "Sigmoid": _unary(sigmoid),
    "Tanh": _unary(np.tanh),
    "Erf": _unary(erf),
    "Sqrt": _unary(np.sqrt),
    "Exp": _unary(np.exp),
    "Log": _unary(np.log),
    "Neg": _unary(np.negative),
    "Abs": _unary(np.abs),
    "Reciprocal": _unary(np.reciprocal),
    "Floor": _unary(np.floor),
    "Ceil": _unary(np.ceil),
    "Sin": _unary(np.sin),
    "Cos": _unary(np.cos),
    "Softplus": _unary(lambda x: np.logaddexp(0, x)),
    "Identity": _unary(lambda x: x.copy()),
    "Not": lambda at, xs, no: [np.logical_not(xs[0])],
    "Gelu": lambda at, xs, no: [gelu(xs[0], str(at.get("approximate", "none")))],
    "LeakyRelu": lambda at, xs, no: [_keep(np.where(xs[0] >= 0, xs[0], float(at.get("alpha", 0.01)) * xs[0]), xs[0])],
    "HardSigmoid": lambda at, xs, no: [
        _keep(np.clip(float(at.get("alpha", 0.2)) * xs[0] + float(at.get("beta", 0.5)), 0, 1), xs[0])
    ],
    "Clip": lambda at, xs, no: [_keep(np.clip(xs[0], *clip_bounds(at, xs)), xs[0])],
    "Cast": _cast,
    "Dropout": _dropout,
    "Reshape": _reshape,
    "Flatten": _flatten,
    "Transpose": _transpose,
    "Squeeze": _squeeze,
    "Unsqueeze": _unsqueeze,
    "Concat": lambda at, xs, no: [np.concatenate([x for x in xs if x is not None], axis=int(at.get("axis", 0)))],
    "Split": _split,
    "Slice": lambda at, xs, no: [np.ascontiguousarray(xs[0][slices(at, xs[0].shape, xs)])],
    "Gather": _gather,
    "Shape": _shape,
    "Size": lambda at, xs, no: [np.asarray(xs[0].size, np.int64)],
    "ConstantOfShape": _constant_of_shape,
    "Expand": lambda at, xs, no: [
        np.ascontiguousarray(np.broadcast_to(xs[0], np.broadcast_shapes(xs[0].shape, tuple(_ints(xs[1])))))
    ],
    "Tile": lambda at, xs, no: [np.tile(xs[0], _ints(xs[1]))],
    "Range": _range,
    "Trilu": lambda at, xs, no: [
        (np.triu if int(at.get("upper", 1)) else np.tril)(
            xs[0], int(np.asarray(xs[1]).reshape(())) if len(xs) > 1 and xs[1] is not None else 0
        )
    ],
    "Pad": _pad,
    "ReduceMean": _reduce(np.mean),
    "ReduceSum": _reduce(np.sum),
    "ReduceMax": _reduce(np.max),
    "ReduceMin": _reduce(np.min),
    "ReduceProd": _reduce(np.prod),
    "ArgMax": _argmax,
    "Softmax": _softmax,
    "LogSoftmax": lambda at, xs, no: _softmax(at, xs, no, log=True),
    "LayerNormalization": _layer_norm,
    "BatchNormalization": _batch_norm,
    "MatMul": _matmul,
    "Gemm": _gemm,
    "FusedGemm": _fused_gemm,
    "Conv": lambda at, xs, no: _conv(at, xs, no),
    "FusedConv": lambda at, xs, no: _conv(at, xs, no, fused=True),
    "MaxPool": lambda at, xs, no: [pool(xs[0], at, "max")],
    "AveragePool": lambda at, xs, no: [pool(xs[0], at, "avg")],
    "GlobalAveragePool": lambda at, xs, no: _global(at, xs, no, "avg"),
    "GlobalMaxPool": lambda at, xs, no: _global(at, xs, no, "max"),
    "FusedElementwise": _fused_elementwise,
}


def run_node(node, arrays):
    if node.op not in OPS:
        raise OracleError(f"oracle has no operator {node.op!r}")
    return OPS[node.op](node.attrs, arrays, len(node.outputs))


def check_feeds(graph, feeds: Mapping[str, np.ndarray]) -> dict[str, np.ndarray]:
    names = {v.name for v in graph.inputs}
    if names != set(feeds):
        raise OracleError(f"inputs: missing {sorted(names - set(feeds))}, unexpected {sorted(set(feeds) - names)}")
    out = {}
    for v in graph.inputs:
        a = np.asarray(feeds[v.name])
        if tuple(a.shape) != v.type.shape or a.dtype != np.dtype(v.type.dtype):
            raise OracleError(f"input {v.name!r}: expected {v.type}, got {a.dtype}{list(a.shape)}")
        out[v.name] = np.asarray(a, order="C")
    return out


def run_graph(graph, feeds: Mapping[str, np.ndarray]) -> dict[str, np.ndarray]:
    """Execute ``graph`` node by node (interpreter.py:71-93), freeing values after last use."""
    env: dict[int, np.ndarray] = {}
    checked = check_feeds(graph, feeds)
    for v in graph.inputs:
        env[id(v)] = checked[v.name]
    last: dict[int, int] = {}
    for i, node in enumerate(graph.nodes):
        for v in node.inputs:
            if v is not None:
                last[id(v)] = i
    keep = {id(v) for v in graph.outputs}

    def get(v):
        if v is None:
            return None
        if v.data is not None:
            return v.data
        return env[id(v)]

    for i, node in enumerate(graph.nodes):
        results = run_node(node, [get(v) for v in node.inputs])
        for v, a in zip(node.outputs, results):
            if v.type is not None and tuple(a.shape) != v.type.shape:
                raise OracleError(f"{node.op} {node.name!r}: produced {a.shape}, inferred {v.type.shape}")
            env[id(v)] = a
        for v in node.inputs:
            if v is not None and v.data is None and id(v) not in keep and last.get(id(v)) == i:
                env.pop(id(v), None)
    return {name: get(v) for name, v in graph.named_outputs()}


def random_feeds(graph, seed: int = 0, int_high: int = 100) -> dict[str, np.ndarray]:
    """interpreter.random_feeds: standard normal floats, {0,1} bools, integers in [0, int_high)."""
    rng = np.random.default_rng(seed)
    feeds = {}
    for v in graph.inputs:
        dt = np.dtype(v.type.dtype)
        if np.issubdtype(dt, np.floating):
            feeds[v.name] = rng.standard_normal(v.type.shape).astype(dt)
        elif dt == np.bool_:
            feeds[v.name] = rng.integers(0, 2, v.type.shape).astype(np.bool_)
        else:
            feeds[v.name] = rng.integers(0, int_high, v.type.shape).astype(dt)
    return feeds
