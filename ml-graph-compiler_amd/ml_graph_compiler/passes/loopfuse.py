"""Loop fusion: chains of elementwise operators become one FusedElementwise node.

Reference: src/ml_graph_compiler/passes/loopfuse.py:1-94. A group grows backwards from each
elementwise node (latest first), absorbing producers that are elementwise, are not graph
outputs, produce the group's output shape and are used only inside the group, up to
MAX_PROGRAM members. The group's ``program`` lists the original operators; the hip backend
evaluates it in one kernel pass, keeping intermediates in registers.
"""

from __future__ import annotations

from typing import Any

from .. import ops
from ..ir import Graph, Node, Value
from .basic import eliminate_dead_code
from .util import insert_node

MAX_PROGRAM = 32


def _fusible(node: Node) -> bool:
    return len(node.outputs) == 1 and (ops.is_elementwise(node.op) or node.op == "FusedElementwise")


def fuse_elementwise(graph: Graph) -> int:
    """Group elementwise chains into FusedElementwise nodes; returns the number of groups."""
    position = {id(n): i for i, n in enumerate(graph.nodes)}
    taken: set[int] = set()
    groups: list[list[Node]] = []
    for root in reversed(graph.nodes):
        if id(root) in taken or not _fusible(root) or root.op == "FusedElementwise":
            continue
        shape = root.output.tensor_type.shape
        members = [root]
        stack = [root]
        while stack and len(members) < MAX_PROGRAM:
            node = stack.pop()
            for v in node.inputs:
                p = v.producer if v is not None else None
                if (
                    p is None
                    or id(p) in taken
                    or p in members
                    or not _fusible(p)
                    or p.op == "FusedElementwise"
                    or v in graph.outputs
                    or v is None
                    or v.tensor_type.shape != shape
                    or any(u not in members for u in v.users)
                ):
                    continue
                members.append(p)
                stack.append(p)
        if len(members) < 2:
            continue
        taken.update(id(m) for m in members)
        groups.append(sorted(members, key=lambda n: position[id(n)]))
    for members in groups:
        _build(graph, members)
    if groups:
        eliminate_dead_code(graph)
    return len(groups)


def _build(graph: Graph, members: list[Node]) -> None:
    root = members[-1]
    produced = {id(m.output): k for k, m in enumerate(members)}
    leaves: list[Value | None] = []
    leaf_index: dict[int, int] = {}
    for m in members:
        for v in m.inputs:
            if v is not None and id(v) not in produced and id(v) not in leaf_index:
                leaf_index[id(v)] = len(leaves)
                leaves.append(v)
    n_leaves = len(leaves)
    program: list[list[Any]] = []
    for m in members:
        args = []
        for v in m.inputs:
            if v is None:
                args.append(-1)
            elif id(v) in produced:
                args.append(n_leaves + produced[id(v)])
            else:
                args.append(leaf_index[id(v)])
        program.append([m.op, dict(m.attrs), args])
    fused = insert_node(graph, "FusedElementwise", leaves, root, attrs={"program": program})
    graph.replace_all_uses(root.output, fused.output)
