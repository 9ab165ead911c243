"""Layout pass: convolution and pooling regions from NCHW to NHWC.

The reference's layout transformation (src/ml_graph_compiler/passes/layout.py), which fixes the
graphs the planner sees: every NCHW FusedConv (with constant weights), MaxPool, AveragePool,
GlobalAveragePool and GlobalMaxPool of rank 4 that is in use is wrapped as
``Transpose(NHWC->NCHW) . op[NHWC] . Transpose(NCHW->NHWC)`` (the weights get an OIHW->HWIO
Transpose, a residual input its own NCHW->NHWC one). Then, alternately up to eight times, the
simplifier cancels adjacent transposes and transposes are pushed below elementwise readers —
``f(T(a), T(b), s) -> T(f(a, b, s))`` when every non-scalar operand comes out of a Transpose with
one common permutation — after which the weight transposes fold into the constants. A chain of
convolutions ends up in NHWC with one transpose at the graph input, and the HIP kernels read a
pixel's channels contiguously.
"""

from __future__ import annotations

from .. import ops
from ..ir import Graph, Node, Value
from .algebra import simplify
from .cleanup import eliminate_dead_code, fold_constants
from .graph_tools import in_use, place_before, substitute

TO_NHWC = [0, 2, 3, 1]
TO_NCHW = [0, 3, 1, 2]
OIHW_TO_HWIO = [2, 3, 1, 0]
SPATIAL_OPS = frozenset({"FusedConv", "MaxPool", "AveragePool", "GlobalAveragePool", "GlobalMaxPool"})


def _permuted(graph: Graph, value: Value, perm: list[int], anchor: Node) -> Value:
    return place_before(graph, anchor, "Transpose", [value], {"perm": perm}).output


def _wrap_nhwc(graph: Graph, node: Node) -> None:
    operands: list[Value | None] = list(node.inputs)
    operands[0] = _permuted(graph, node.input(0), TO_NHWC, node)
    if node.op == "FusedConv":
        operands[1] = _permuted(graph, node.input(1), OIHW_TO_HWIO, node)
        if len(operands) > 3 and operands[3] is not None:
            operands[3] = _permuted(graph, operands[3], TO_NHWC, node)
    inner = place_before(graph, node, node.op, operands, {**node.attrs, "layout": "NHWC"})
    substitute(graph, node, "Transpose", [inner.output], {"perm": TO_NCHW})


def _wants_nhwc(graph: Graph, node: Node) -> bool:
    return (node.op in SPATIAL_OPS and node.attrs.get("layout", "NCHW") == "NCHW"
            and node.input(0).tensor_type.rank == 4 and in_use(graph, node)
            and (node.op != "FusedConv" or node.input(1).is_constant))


def _lone_number(value: Value) -> bool:
    return value.is_constant and value.data is not None and value.data.size == 1


def _push_transposes_down(graph: Graph) -> int:
    """Move a Transpose below an elementwise reader whose non-scalar operands all come out of
    Transposes with the same permutation; returns how many readers were rewritten."""
    pushed = 0
    for node in list(graph.nodes):
        if not ops.is_elementwise(node.op) or node.op == "Where" or not node.output.users:
            continue
        operands = [v for v in node.inputs if v is not None]
        tensors = [v for v in operands if not _lone_number(v)]
        flips = [v.producer for v in operands if v.producer is not None and v.producer.op == "Transpose"]
        if not flips or len(flips) != len(tensors):
            continue
        perms = {tuple(ops.transpose_perm(t, t.input(0).tensor_type.rank)) for t in flips}
        if len(perms) != 1:
            continue
        unflipped = [v if v is None or _lone_number(v) else v.producer.input(0) for v in node.inputs]
        inner = place_before(graph, node, node.op, unflipped, dict(node.attrs))
        substitute(graph, node, "Transpose", [inner.output], {"perm": list(perms.pop())})
        pushed += 1
    eliminate_dead_code(graph)
    return pushed


def to_nhwc(graph: Graph) -> int:
    """Convert NCHW spatial operators to NHWC; returns how many were converted."""
    converted = 0
    for node in list(graph.nodes):
        if _wants_nhwc(graph, node):
            _wrap_nhwc(graph, node)
            converted += 1
    if converted:
        eliminate_dead_code(graph)
        for _ in range(8):
            simplify(graph)
            if not _push_transposes_down(graph):
                break
        fold_constants(graph)
        simplify(graph)
        eliminate_dead_code(graph)
    return converted
