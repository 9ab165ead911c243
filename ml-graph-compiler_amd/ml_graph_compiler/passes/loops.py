"""Loop fusion: chains of elementwise operators become one FusedElementwise node.

Run alone, each elementwise operator reads its operands from memory and writes a whole
tensor; fused, the chain runs as one loop (one kernel on the GPU) that keeps intermediates in
registers. Grouping follows the reference (src/ml_graph_compiler/passes/loopfuse.py), because
the groups decide which tensors the planner sees: walking the nodes from last to first, an
unassigned elementwise node seeds a group, which then grows upwards (depth first, last added
first) through producers that are elementwise, not yet grouped, not graph outputs, produce the
seed's output shape (nothing is recomputed per element of a broadcast) and are read only inside
the group — until the group holds MAX_PROGRAM nodes. Groups of two or more become one node whose
``program`` lists the members in graph order: ``[op, attrs, args]`` with an argument naming a
node input (its first-seen order) or an earlier member's result, and -1 an omitted input.
"""

from __future__ import annotations

from typing import Any

from .. import ops
from ..ir import Graph, Node, Value
from .cleanup import eliminate_dead_code
from .graph_tools import substitute

MAX_PROGRAM = 32


def _plain_elementwise(node: Node) -> bool:
    return len(node.outputs) == 1 and ops.is_elementwise(node.op)


def _grow(graph: Graph, seed: Node, taken: set[int]) -> list[Node]:
    shape = seed.output.tensor_type.shape
    group, in_group = [seed], {id(seed)}
    stack = [seed]
    while stack and len(group) < MAX_PROGRAM:
        for v in stack.pop().inputs:
            p = None if v is None else v.producer
            if (p is None or id(p) in taken or id(p) in in_group or not _plain_elementwise(p)
                    or any(v is o for o in graph.outputs) or v.tensor_type.shape != shape
                    or any(id(r) not in in_group for r in v.users)):
                continue
            group.append(p)
            in_group.add(id(p))
            stack.append(p)
    return group


def _program(members: list[Node]) -> tuple[list[Value | None], list[list[Any]]]:
    result_of = {id(m.output): k for k, m in enumerate(members)}
    leaves: dict[int, int] = {}
    leaf_values: list[Value | None] = []
    for m in members:
        for v in m.inputs:
            if v is not None and id(v) not in result_of and id(v) not in leaves:
                leaves[id(v)] = len(leaf_values)
                leaf_values.append(v)
    base = len(leaf_values)

    def ref(v: Value | None) -> int:
        if v is None:
            return -1
        return base + result_of[id(v)] if id(v) in result_of else leaves[id(v)]

    return leaf_values, [[m.op, dict(m.attrs), [ref(v) for v in m.inputs]] for m in members]


def fuse_elementwise(graph: Graph) -> int:
    """Group elementwise chains into FusedElementwise nodes; returns the number of groups."""
    order = {id(n): i for i, n in enumerate(graph.nodes)}
    taken: set[int] = set()
    groups: list[list[Node]] = []
    for seed in reversed(graph.nodes):
        if id(seed) in taken or not _plain_elementwise(seed):
            continue
        group = _grow(graph, seed, taken)
        if len(group) > 1:
            taken.update(id(m) for m in group)
            groups.append(sorted(group, key=lambda n: order[id(n)]))
    for members in groups:
        leaves, program = _program(members)
        substitute(graph, members[-1], "FusedElementwise", leaves, {"program": program})
    if groups:
        eliminate_dead_code(graph)
    return len(groups)
