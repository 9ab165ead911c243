"""NCHW convolution/pooling regions to NHWC (reference: src/ml_graph_compiler/passes/layout.py).

Each NCHW FusedConv, MaxPool, AveragePool, GlobalAveragePool and GlobalMaxPool is rewritten as
its NHWC form between a Transpose to NHWC and one back to NCHW; convolution weights get an
OIHW -> HWIO Transpose that folding turns into a constant. Elementwise operators whose tensor
operands are all transposed the same way then move below the Transpose, and simplification
cancels back-to-back pairs, so a chain of convolutions runs in NHWC with one transpose at the
graph input. NHWC keeps a pixel's channels contiguous: a 1x1 convolution is a plain GEMM and the
implicit-GEMM A operand is read in 16-byte channel quads.
"""

from __future__ import annotations

from .. import ops
from ..ir import Graph, Node, Value
from .basic import eliminate_dead_code, fold_constants
from .simplify import simplify
from .util import insert_node

TO_NHWC = [0, 2, 3, 1]
TO_NCHW = [0, 3, 1, 2]
OIHW_TO_HWIO = [2, 3, 1, 0]
LAYOUT_OPS = frozenset({"FusedConv", "MaxPool", "AveragePool", "GlobalAveragePool", "GlobalMaxPool"})


def _transpose(graph: Graph, value: Value, perm: list[int], before: Node) -> Value:
    return insert_node(graph, "Transpose", [value], before, attrs={"perm": perm}).output


def _convert(graph: Graph, node: Node) -> None:
    inputs: list[Value | None] = list(node.inputs)
    inputs[0] = _transpose(graph, node.input(0), TO_NHWC, node)
    if node.op == "FusedConv":
        inputs[1] = _transpose(graph, node.input(1), OIHW_TO_HWIO, node)
        if len(inputs) > 3 and inputs[3] is not None:
            inputs[3] = _transpose(graph, inputs[3], TO_NHWC, node)
    nhwc = insert_node(graph, node.op, inputs, node, attrs={**node.attrs, "layout": "NHWC"})
    back = insert_node(graph, "Transpose", [nhwc.output], node, attrs={"perm": TO_NCHW})
    graph.replace_all_uses(node.output, back.output)


def _scalar_constant(value: Value) -> bool:
    return value.is_constant and value.data is not None and value.data.size == 1


def _sink_transposes(graph: Graph) -> int:
    """f(T(a)) -> T(f(a)) and g(T(a), T(b)) -> T(g(a, b)) for elementwise f and g."""
    moved = 0
    for node in list(graph.nodes):
        if not ops.is_elementwise(node.op) or not node.output.users or node.op == "Where":
            continue
        present = [v for v in node.inputs if v is not None]
        transposes = [v.producer for v in present if v.producer is not None and v.producer.op == "Transpose"]
        tensors = [v for v in present if not _scalar_constant(v)]
        if not transposes or len(transposes) != len(tensors):
            continue
        perms = {tuple(ops.transpose_perm(t, t.input(0).tensor_type.rank)) for t in transposes}
        if len(perms) != 1:
            continue
        perm = list(perms.pop())
        new_inputs: list[Value | None] = []
        for v in node.inputs:
            if v is None or _scalar_constant(v):
                new_inputs.append(v)
            else:
                assert v.producer is not None
                new_inputs.append(v.producer.input(0))
        inner = insert_node(graph, node.op, new_inputs, node, attrs=dict(node.attrs))
        graph.replace_all_uses(node.output, _transpose(graph, inner.output, perm, node))
        moved += 1
    eliminate_dead_code(graph)
    return moved


def to_nhwc(graph: Graph) -> int:
    """Convert NCHW convolution and pooling to NHWC; returns the number of converted nodes."""
    converted = 0
    for node in list(graph.nodes):
        if node.op not in LAYOUT_OPS or node.attrs.get("layout", "NCHW") != "NCHW":
            continue
        if node.input(0).tensor_type.rank != 4 or not (node.output.users or node.output in graph.outputs):
            continue
        if node.op == "FusedConv" and not node.input(1).is_constant:
            continue
        _convert(graph, node)
        converted += 1
    if not converted:
        return 0
    eliminate_dead_code(graph)
    for _ in range(8):
        simplify(graph)
        if not _sink_transposes(graph):
            break
    fold_constants(graph)
    simplify(graph)
    eliminate_dead_code(graph)
    return converted
