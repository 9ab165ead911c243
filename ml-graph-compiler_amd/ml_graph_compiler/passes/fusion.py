"""Operator fusion (reference: src/ml_graph_compiler/passes/fusion.py:1-426).

* Conv + BatchNormalization: the normalization is folded into the convolution weights and bias
  (float64 factor scale / sqrt(var + eps), cast to float32).
* Conv, and Gemm/MatMul with a constant 2-D right operand, become FusedConv / FusedGemm, which
  then absorb a constant per-channel bias add, a residual add of a same-typed tensor, and one
  activation: ``act(op(x) + bias + residual)``. Bias and residual are absorbed before the
  activation, never after it.
* MatMul(x, Transpose(W)) with constant 2-D W becomes FusedGemm with ``trans_b``.
* FusedGemm between a flatten-to-2-D Reshape and a reshape back (GPT-2's Conv1D export) takes
  the un-flattened operand directly.
* The decomposed LayerNorm (ReduceMean, Sub, Pow/Mul, ReduceMean, Add, Sqrt, Div, Mul, Add)
  becomes LayerNormalization; the erf GELU and tanh GELU subgraphs become one Gelu node.
"""

from __future__ import annotations

import math

import numpy as np

from .. import ops
from ..ir import Graph, Node, Value
from .basic import eliminate_dead_code
from .util import binary_with_const, insert_node, is_scalar, only_user, producer, scalar


def _mean_over_last_axis(node: Node | None, x: Value) -> bool:
    if node is None or node.op != "ReduceMean" or node.inputs[0] is not x or x.type is None:
        return False
    try:
        axes = ops.reduce_axes(node, x.type.rank, [None if v is None else v.data for v in node.inputs])
    except Exception:
        return False
    return axes == (x.type.rank - 1,) and int(node.attrs.get("keepdims", 1)) == 1


def _single_use(value: Value, graph: Graph) -> bool:
    return only_user(value, graph) is not None


def channel_vector(value: Value | None, n: int, axis_from_end: int) -> np.ndarray | None:
    """A constant broadcasting like a length-n vector along axis -axis_from_end, flattened."""
    if value is None or value.data is None:
        return None
    data = value.data
    if data.size == 1:
        return np.full(n, float(data.reshape(())), dtype=np.float32)
    if data.size != n or data.ndim < axis_from_end or data.shape[data.ndim - axis_from_end] != n:
        return None
    return data.reshape(n).astype(np.float32)


# ---------------------------------------------------------------------------------------------
# LayerNorm and GELU patterns
# ---------------------------------------------------------------------------------------------
def _ln_match(graph: Graph, div: Node) -> tuple[Value, float, Node, np.ndarray | None, np.ndarray | None] | None:
    d, s = div.inputs[0], div.inputs[1]
    sub, sqrt = producer(d, "Sub"), producer(s, "Sqrt")
    if sub is None or sqrt is None or d is None:
        return None
    x, mean = sub.inputs[0], sub.inputs[1]
    if x is None or mean is None or not _mean_over_last_axis(mean.producer, x):
        return None
    add = producer(sqrt.input(0), "Add")
    if add is None:
        return None
    left, right = add.inputs[0], add.inputs[1]
    if scalar(right) is not None and left is not None and not left.is_constant:
        var, eps = left, scalar(right)
    elif scalar(left) is not None and right is not None and not right.is_constant:
        var, eps = right, scalar(left)
    else:
        return None
    if eps is None:
        return None
    second = var.producer
    if second is None or second.op != "ReduceMean":
        return None
    sq = second.input(0)
    sq_node = sq.producer
    if not _mean_over_last_axis(second, sq) or sq_node is None:
        return None
    squares = (sq_node.op == "Mul" and sq_node.inputs[0] is d and sq_node.inputs[1] is d) or (
        sq_node.op == "Pow" and sq_node.inputs[0] is d and is_scalar(sq_node.inputs[1], 2.0)
    )
    if not squares:
        return None
    if not all(_single_use(v, graph) for v in (mean, sq, var, add.output, sqrt.output)):
        return None
    if any(u not in (sq_node, div) for u in d.users) or d in graph.outputs:
        return None
    dim = x.tensor_type.shape[-1]
    tail, gamma, beta = div, None, None
    user = only_user(div.output, graph)
    if user is not None and user.op == "Mul":
        other = user.inputs[1] if user.inputs[0] is div.output else user.inputs[0]
        gamma = channel_vector(other, dim, 1)
        if gamma is not None:
            tail = user
    user = only_user(tail.output, graph)
    if user is not None and user.op == "Add":
        other = user.inputs[1] if user.inputs[0] is tail.output else user.inputs[0]
        beta = channel_vector(other, dim, 1)
        if beta is not None:
            tail = user
    if tail.output.type != x.type:
        return None
    return x, float(eps), tail, gamma, beta


def fuse_layer_norm(graph: Graph) -> int:
    count = 0
    for div in list(graph.nodes):
        if div.op != "Div" or div not in graph.nodes:
            continue
        match = _ln_match(graph, div)
        if match is None:
            continue
        x, eps, tail, gamma, beta = match
        dim = x.tensor_type.shape[-1]
        g = graph.constant(gamma if gamma is not None else np.ones(dim, np.float32), "ln_gamma")
        b = graph.constant(beta if beta is not None else np.zeros(dim, np.float32), "ln_beta")
        ln = insert_node(graph, "LayerNormalization", [x, g, b], tail, attrs={"axis": -1, "epsilon": eps})
        graph.replace_all_uses(tail.output, ln.output)
        count += 1
    if count:
        eliminate_dead_code(graph)
    return count


def _gelu_tail(graph: Graph, s: Node, x: Value) -> Node | None:
    """Given s = 1 + f(x), the node computing 0.5 * x * s in any association."""
    user = only_user(s.output, graph)
    if user is None or user.op != "Mul":
        return None
    other = user.inputs[1] if user.inputs[0] is s.output else user.inputs[0]
    if other is x:  # (x * s) * 0.5
        last = only_user(user.output, graph)
        if last is not None and binary_with_const(last, "Mul", 0.5) is user.output:
            return last
        return None
    half = producer(other, "Mul")
    if half is not None and binary_with_const(half, "Mul", 0.5) is x and _single_use(half.output, graph):
        return user  # (0.5 * x) * s
    if is_scalar(other, 0.5):  # (s * 0.5) * x
        last = only_user(user.output, graph)
        if last is not None and last.op == "Mul" and x in last.inputs:
            return last
    return None


def _cube_of(value: Value | None) -> Value | None:
    node = producer(value, ("Pow", "Mul"))
    if node is None:
        return None
    if node.op == "Pow" and is_scalar(node.inputs[1], 3.0):
        return node.inputs[0]
    a, b = node.inputs[0], node.inputs[1]
    for sq, x in ((a, b), (b, a)):
        sq_node = producer(sq, "Mul")
        if sq_node is not None and sq_node.inputs[0] is x and sq_node.inputs[1] is x:
            return x
    return None


def fuse_gelu(graph: Graph) -> int:
    count = 0
    for node in list(graph.nodes):
        if node.op not in ("Erf", "Tanh") or not node.output.users:
            continue
        x: Value | None = None
        approximate = "none"
        arg = node.input(0)
        if node.op == "Erf":
            scaled = producer(arg, ("Div", "Mul"))
            if scaled is not None and scaled.op == "Div":
                x = binary_with_const(scaled, "Div", math.sqrt(2.0))
            elif scaled is not None:
                x = binary_with_const(scaled, "Mul", 1.0 / math.sqrt(2.0))
        else:
            approximate = "tanh"
            inner = binary_with_const(producer(arg, "Mul"), "Mul", math.sqrt(2.0 / math.pi))
            add = producer(inner, "Add")
            if add is not None:
                for xa, rest in ((add.inputs[0], add.inputs[1]), (add.inputs[1], add.inputs[0])):
                    cube = binary_with_const(producer(rest, "Mul"), "Mul", 0.044715)
                    if xa is not None and _cube_of(cube) is xa:
                        x = xa
                        break
        if x is None:
            continue
        s = only_user(node.output, graph)
        if s is None or binary_with_const(s, "Add", 1.0) is not node.output:
            continue
        tail = _gelu_tail(graph, s, x)
        if tail is None or tail.output.type != x.type:
            continue
        gelu = insert_node(graph, "Gelu", [x], tail, attrs={"approximate": approximate})
        graph.replace_all_uses(tail.output, gelu.output)
        count += 1
    if count:
        eliminate_dead_code(graph)
    return count


# ---------------------------------------------------------------------------------------------
# Conv and Gemm with epilogues
# ---------------------------------------------------------------------------------------------
def _fold_batch_norm(graph: Graph, conv: Node) -> bool:
    bn = only_user(conv.output, graph)
    if bn is None or bn.op != "BatchNormalization" or bn.inputs[0] is not conv.output:
        return False
    if len(bn.outputs) > 1 and any(o.users for o in bn.outputs[1:]):
        return False
    params = [None if v is None else v.data for v in bn.inputs[1:5]]
    w, b = conv.input(1).data, conv.optional_input(2)
    if w is None or any(p is None for p in params) or (b is not None and b.data is None):
        return False
    scale, beta, mean, var = (np.asarray(p, dtype=np.float64) for p in params)
    factor = scale / np.sqrt(var + float(bn.attrs.get("epsilon", 1e-5)))
    k = w.shape[0]
    new_w = (w.astype(np.float64) * factor.reshape(k, 1, 1, 1)).astype(np.float32)
    old_b = b.data.astype(np.float64) if b is not None and b.data is not None else np.zeros(k)
    new_b = ((old_b - mean) * factor + beta).astype(np.float32)
    inputs: list[Value | None] = [
        conv.input(0),
        graph.constant(new_w, "conv_w_bn"),
        graph.constant(new_b, "conv_b_bn"),
    ]
    folded = insert_node(graph, "Conv", inputs, bn, attrs=dict(conv.attrs))
    graph.replace_all_uses(bn.outputs[0], folded.output)
    return True


def activation_attrs(node: Node) -> dict[str, object] | None:
    """Epilogue attributes for an activation node, or None when it is not one."""
    if node.op == "Relu":
        return {"activation": "relu"}
    if node.op == "Tanh":
        return {"activation": "tanh"}
    if node.op == "Sigmoid":
        return {"activation": "sigmoid"}
    if node.op == "Gelu":
        tanh = node.attrs.get("approximate", "none") == "tanh"
        return {"activation": "gelu_tanh" if tanh else "gelu"}
    if node.op == "Clip":
        if any(v is not None and not v.is_constant for v in node.inputs[1:]):
            return None
        lo, hi = ops.clip_bounds(node, [None if v is None else v.data for v in node.inputs])
        if lo == 0.0 and math.isinf(hi) and hi > 0:
            return {"activation": "relu"}
        return {"activation": "clip", "clip_min": lo, "clip_max": hi}
    return None


def _absorb_epilogue(graph: Graph, node: Node, channel_from_end: int) -> bool:
    """Absorb one bias add, residual add or activation consuming ``node``'s output."""
    user = only_user(node.output, graph)
    if user is None:
        return False
    act = str(node.attrs.get("activation", "none"))
    inputs = list(node.inputs) + [None] * (4 - len(node.inputs))
    out_type = node.output.tensor_type
    if user.op == "Add" and act == "none":
        other = user.inputs[1] if user.inputs[0] is node.output else user.inputs[0]
        if other is None or user.output.type != out_type:
            return False
        n = out_type.shape[-channel_from_end]
        vector = channel_vector(other, n, channel_from_end) if other.is_constant else None
        if vector is not None:
            old = inputs[2].data if inputs[2] is not None else None
            inputs[2] = graph.constant(vector if old is None else (old + vector).astype(np.float32), "bias")
        elif not other.is_constant and other.type == out_type and inputs[3] is None:
            inputs[3] = other
        else:
            return False
        attrs = dict(node.attrs)
    elif act == "none" and (extra := activation_attrs(user)) is not None:
        if user.output.type != out_type:
            return False
        attrs = {**node.attrs, **extra}
    else:
        return False
    while inputs and inputs[-1] is None:
        inputs.pop()
    fused = insert_node(graph, node.op, inputs, user, attrs=attrs)
    graph.replace_all_uses(user.output, fused.output)
    return True


def _to_fused_gemm(graph: Graph, node: Node) -> bool:
    if node.op == "Gemm":
        a, b, c = node.input(0), node.input(1), node.optional_input(2)
        if (
            int(node.attrs.get("transA", 0))
            or b.data is None
            or float(node.attrs.get("alpha", 1.0)) != 1.0
            or (c is not None and (c.data is None or float(node.attrs.get("beta", 1.0)) != 1.0))
        ):
            return False
        n = node.output.tensor_type.shape[1]
        bias = channel_vector(c, n, 1) if c is not None else None
        if c is not None and bias is None:
            return False
        inputs: list[Value | None] = [a, b]
        if bias is not None:
            inputs.append(graph.constant(bias, "gemm_bias"))
        attrs = {"trans_b": int(node.attrs.get("transB", 0))}
    elif node.op == "MatMul":
        a, b = node.input(0), node.input(1)
        if a.tensor_type.rank < 1:
            return False
        transposed = producer(b, "Transpose")
        if b.data is not None and b.tensor_type.rank == 2:
            inputs, attrs = [a, b], {"trans_b": 0}
        elif (
            transposed is not None
            and transposed.input(0).data is not None
            and transposed.input(0).tensor_type.rank == 2
        ):
            inputs, attrs = [a, transposed.input(0)], {"trans_b": 1}
        else:
            return False
    else:
        return False
    fused = insert_node(graph, "FusedGemm", inputs, node, attrs={**attrs, "activation": "none"})
    graph.replace_all_uses(node.output, fused.output)
    return True


def _used(graph: Graph, node: Node) -> bool:
    return any(o.users or o in graph.outputs for o in node.outputs)


def fuse_conv(graph: Graph) -> int:
    count = 0
    for node in list(graph.nodes):
        if node.op == "Conv" and node.output.users and _fold_batch_norm(graph, node):
            count += 1
    eliminate_dead_code(graph)
    for node in list(graph.nodes):
        if node.op == "Conv" and node.input(1).is_constant and _used(graph, node):
            fused = insert_node(
                graph, "FusedConv", list(node.inputs), node, attrs={**node.attrs, "activation": "none"}
            )
            graph.replace_all_uses(node.output, fused.output)
            count += 1
    eliminate_dead_code(graph)
    return count + _absorb_all(graph, "FusedConv", 3)


def _lift_reshapes(graph: Graph, node: Node) -> bool:
    """Reshape(FusedGemm(Reshape(x, [M, K])), lead + [N]) -> FusedGemm(x') with x' shaped
    lead + [K]: the operand may have any rank, so both reshapes disappear."""
    reshape = producer(node.input(0), "Reshape")
    if reshape is None or "shape" not in reshape.attrs or len(node.inputs) > 3:
        return False
    out = node.output.tensor_type
    after = only_user(node.output, graph)
    if out.rank != 2 or after is None or after.op != "Reshape" or "shape" not in after.attrs:
        return False
    target = after.output.tensor_type.shape
    if not target or target[-1] != out.shape[1] or int(np.prod(target[:-1])) != out.shape[0]:
        return False
    x = reshape.input(0)
    a_shape = (*target[:-1], node.input(0).tensor_type.shape[1])
    if x.tensor_type.shape != a_shape:
        x = insert_node(graph, "Reshape", [x], after, attrs={"shape": list(a_shape)}).output
    lifted = insert_node(graph, "FusedGemm", [x, *node.inputs[1:]], after, attrs=dict(node.attrs))
    graph.replace_all_uses(after.output, lifted.output)
    return True


def fuse_gemm(graph: Graph) -> int:
    count = 0
    for node in list(graph.nodes):
        if node.op in ("Gemm", "MatMul") and _used(graph, node) and _to_fused_gemm(graph, node):
            count += 1
    eliminate_dead_code(graph)
    for node in list(graph.nodes):
        if node.op == "FusedGemm" and node.output.users and _lift_reshapes(graph, node):
            count += 1
    eliminate_dead_code(graph)
    return count + _absorb_all(graph, "FusedGemm", 1)


def _absorb_all(graph: Graph, op: str, channel_from_end: int) -> int:
    count = 0
    changed = True
    while changed:
        changed = False
        for node in list(graph.nodes):
            if node.op == op and node.output.users and _absorb_epilogue(graph, node, channel_from_end):
                count += 1
                changed = True
        eliminate_dead_code(graph)
    return count


def fuse(graph: Graph) -> int:
    """All fusions; returns the number of rewrites."""
    return fuse_layer_norm(graph) + fuse_gelu(graph) + fuse_conv(graph) + fuse_gemm(graph)
