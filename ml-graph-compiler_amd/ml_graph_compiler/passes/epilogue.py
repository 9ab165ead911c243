"""Convolution and GEMM fusion with their epilogues.

What the reference's fusion pass does to contractions (src/ml_graph_compiler/passes/fusion.py),
in the same order, since the resulting graph (and with it the planner's offsets) must match:

1. A BatchNormalization that is a Conv's only reader folds into the Conv's weights and bias
   (in float64: factor = scale / sqrt(var + eps), W' = W * factor, b' = (b - mean) * factor +
   beta, both cast to float32).
2. Every Conv with constant weights becomes FusedConv (activation "none"). Every Gemm with
   alpha 1, no transA, constant B and either no C or a per-column constant C with beta 1, and
   every MatMul whose right operand is a constant 2-D matrix or the Transpose of one, becomes
   FusedGemm (``trans_b`` marks a transposed B; no transposed copy is made).
3. A FusedGemm between two static Reshapes that merely flatten and restore its leading
   dimensions (GPT-2's Conv1D export) takes the unflattened operand directly.
4. Epilogues are absorbed into a fused node from the reader of its output, one at a time until
   none is left: an Add of a constant per-channel vector (or scalar) becomes (or adds into) the
   bias, an Add of a same-typed tensor becomes the residual (once), and — while no activation is
   set — an Add or one activation (ReLU, Clip with constant bounds, GELU erf/tanh, Tanh,
   Sigmoid) is taken over; after an activation nothing more is absorbed.
"""

from __future__ import annotations

import math
from typing import Any

import numpy as np

from .. import ops
from ..ir import Graph, Node, Value
from .cleanup import eliminate_dead_code
from .graph_tools import in_use, made_by, other_operand, per_channel, place_before, sole_reader, substitute


def _fold_batch_norm(graph: Graph, conv: Node) -> bool:
    bn = sole_reader(graph, conv.output)
    if bn is None or bn.op != "BatchNormalization" or bn.inputs[0] is not conv.output:
        return False
    if any(o.users for o in bn.outputs[1:]):
        return False
    stats = [None if v is None else v.data for v in bn.inputs[1:5]]
    weights, bias = conv.input(1).data, conv.optional_input(2)
    if weights is None or any(s is None for s in stats) or (bias is not None and bias.data is None):
        return False
    scale, shift, mean, var = (np.asarray(s, dtype=np.float64) for s in stats)
    factor = scale / np.sqrt(var + float(bn.attrs.get("epsilon", 1e-5)))
    k = weights.shape[0]
    folded_w = (weights.astype(np.float64) * factor[:, None, None, None]).astype(np.float32)
    base = bias.data.astype(np.float64) if bias is not None else np.zeros(k)
    folded_b = ((base - mean) * factor + shift).astype(np.float32)
    new_inputs: list[Value | None] = [conv.input(0), graph.constant(folded_w, "conv_w_bn"),
                                      graph.constant(folded_b, "conv_b_bn")]
    conv_bn = place_before(graph, bn, "Conv", new_inputs, dict(conv.attrs))
    graph.replace_all_uses(bn.outputs[0], conv_bn.output)
    return True


def activation_attrs(node: Node) -> dict[str, Any] | None:
    """The epilogue attributes equivalent to an activation node, or None."""
    simple = {"Relu": "relu", "Tanh": "tanh", "Sigmoid": "sigmoid"}
    if node.op in simple:
        return {"activation": simple[node.op]}
    if node.op == "Gelu":
        return {"activation": "gelu_tanh" if node.attrs.get("approximate", "none") == "tanh" else "gelu"}
    if node.op != "Clip" or any(v is not None and not v.is_constant for v in node.inputs[1:]):
        return None
    lo, hi = ops.clip_bounds(node, [None if v is None else v.data for v in node.inputs])
    if lo == 0.0 and hi == math.inf:
        return {"activation": "relu"}
    return {"activation": "clip", "clip_min": lo, "clip_max": hi}


def _take_epilogue(graph: Graph, fused: Node, channel_axis_from_end: int) -> bool:
    """Absorb the reader of ``fused``'s output if it is a bias, a residual or an activation."""
    reader = sole_reader(graph, fused.output)
    if reader is None:
        return False
    result_t = fused.output.tensor_type
    slots: list[Value | None] = (list(fused.inputs) + [None] * 4)[:max(4, len(fused.inputs))]
    no_activation = str(fused.attrs.get("activation", "none")) == "none"
    if reader.op == "Add" and no_activation:
        addend = other_operand(reader, fused.output)
        if addend is None or reader.output.type != result_t:
            return False
        channels = result_t.shape[-channel_axis_from_end]
        vector = per_channel(addend, channels, channel_axis_from_end) if addend.is_constant else None
        if vector is not None:
            previous = slots[2].data if slots[2] is not None else None
            slots[2] = graph.constant(vector if previous is None else (previous + vector).astype(np.float32), "bias")
        elif not addend.is_constant and addend.type == result_t and slots[3] is None:
            slots[3] = addend
        else:
            return False
        attrs = dict(fused.attrs)
    else:
        taken = activation_attrs(reader) if no_activation else None
        if taken is None or reader.output.type != result_t:
            return False
        attrs = {**fused.attrs, **taken}
    while slots and slots[-1] is None:
        slots.pop()
    substitute(graph, reader, fused.op, slots, attrs)
    return True


def _absorb_epilogues(graph: Graph, op: str, channel_axis_from_end: int) -> int:
    taken = 0
    while True:
        round_taken = sum(1 for node in list(graph.nodes)
                          if node.op == op and node.output.users and _take_epilogue(graph, node, channel_axis_from_end))
        eliminate_dead_code(graph)
        taken += round_taken
        if not round_taken:
            return taken


def _gemm_operands(graph: Graph, node: Node) -> tuple[list[Value | None], dict[str, Any]] | None:
    """Operands and attributes of the FusedGemm that replaces a Gemm or MatMul, if it can."""
    if node.op == "Gemm":
        a, b, c = node.input(0), node.input(1), node.optional_input(2)
        plain = (not int(node.attrs.get("transA", 0)) and b.data is not None
                 and float(node.attrs.get("alpha", 1.0)) == 1.0)
        if not plain or (c is not None and (c.data is None or float(node.attrs.get("beta", 1.0)) != 1.0)):
            return None
        operands: list[Value | None] = [a, b]
        if c is not None:
            bias = per_channel(c, node.output.tensor_type.shape[1], 1)
            if bias is None:
                return None
            operands.append(graph.constant(bias, "gemm_bias"))
        return operands, {"trans_b": int(node.attrs.get("transB", 0))}
    a, b = node.input(0), node.input(1)
    if a.tensor_type.rank < 1:
        return None
    if b.data is not None and b.tensor_type.rank == 2:
        return [a, b], {"trans_b": 0}
    flipped = made_by(b, "Transpose")
    if flipped is not None and flipped.input(0).data is not None and flipped.input(0).tensor_type.rank == 2:
        return [a, flipped.input(0)], {"trans_b": 1}
    return None


def _unflatten_operand(graph: Graph, gemm: Node) -> bool:
    """FusedGemm(Reshape(x, [M, K])) read only by Reshape(.., lead + [N]) -> FusedGemm(x')
    with x' of shape lead + [K]; the two reshapes drop out."""
    flatten = made_by(gemm.input(0), "Reshape")
    if flatten is None or "shape" not in flatten.attrs or len(gemm.inputs) > 3:
        return False
    flat = gemm.output.tensor_type
    restore = sole_reader(graph, gemm.output)
    if flat.rank != 2 or restore is None or restore.op != "Reshape" or "shape" not in restore.attrs:
        return False
    lead = restore.output.tensor_type.shape
    if not lead or lead[-1] != flat.shape[1] or int(np.prod(lead[:-1])) != flat.shape[0]:
        return False
    x = flatten.input(0)
    wanted = (*lead[:-1], gemm.input(0).tensor_type.shape[1])
    if x.tensor_type.shape != wanted:
        x = place_before(graph, restore, "Reshape", [x], {"shape": list(wanted)}).output
    substitute(graph, restore, "FusedGemm", [x, *gemm.inputs[1:]], dict(gemm.attrs))
    return True


def fuse_conv(graph: Graph) -> int:
    rewrites = sum(1 for node in list(graph.nodes)
                   if node.op == "Conv" and node.output.users and _fold_batch_norm(graph, node))
    eliminate_dead_code(graph)
    for node in list(graph.nodes):
        if node.op == "Conv" and node.input(1).is_constant and in_use(graph, node):
            substitute(graph, node, "FusedConv", list(node.inputs), {**node.attrs, "activation": "none"})
            rewrites += 1
    eliminate_dead_code(graph)
    return rewrites + _absorb_epilogues(graph, "FusedConv", 3)


def fuse_gemm(graph: Graph) -> int:
    rewrites = 0
    for node in list(graph.nodes):
        if node.op not in ("Gemm", "MatMul") or not in_use(graph, node):
            continue
        found = _gemm_operands(graph, node)
        if found is not None:
            operands, attrs = found
            substitute(graph, node, "FusedGemm", operands, {**attrs, "activation": "none"})
            rewrites += 1
    eliminate_dead_code(graph)
    rewrites += sum(1 for node in list(graph.nodes)
                    if node.op == "FusedGemm" and node.output.users and _unflatten_operand(graph, node))
    eliminate_dead_code(graph)
    return rewrites + _absorb_epilogues(graph, "FusedGemm", 1)
