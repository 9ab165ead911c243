"""Memory-aware list scheduling and dataflow analysis (reference: src/ml_graph_compiler/schedule.py).

``memory_aware_order`` keeps the set of ready nodes and repeatedly runs the one whose execution
grows the live footprint least, delta(n) = bytes(outputs of n) - bytes(inputs whose last
remaining user is n), ties broken by program order. ``wavefronts`` gives ASAP levels (the
operator-level parallelism a multi-stream executor could use) and ``critical_path_flops`` the
FLOP-weighted longest path.
"""

from __future__ import annotations

from collections.abc import Iterable, Sequence
from dataclasses import dataclass

from . import ops
from .errors import GraphError
from .ir import Graph, Node, Value

VIEW_OPS = frozenset({"Reshape", "Flatten", "Squeeze", "Unsqueeze", "Identity", "Dropout"})


def _bytes(value: Value) -> int:
    return 0 if value.is_constant or value.type is None else value.type.nbytes


def _storage_root(value: Value) -> Value:
    while value.producer is not None and value.producer.op in VIEW_OPS:
        value = value.producer.input(0)
    return value


def peak_live_bytes(graph: Graph, order: Sequence[Node] | None = None) -> int:
    """Peak live bytes of a schedule; a node's inputs and outputs count together, views own no
    storage, graph outputs live to the end."""
    nodes = list(graph.nodes if order is None else order)
    last: dict[int, int] = {}
    for i, node in enumerate(nodes):
        for v in node.inputs:
            if v is not None and not v.is_constant:
                last[id(_storage_root(v))] = i
    for v in graph.outputs:
        last[id(_storage_root(v))] = len(nodes)
    live = sum(_bytes(v) for v in graph.inputs)
    peak = live
    dying: dict[int, list[Value]] = {}
    for v in graph.inputs:
        dying.setdefault(last.get(id(v), -1), []).append(v)
    live -= sum(_bytes(v) for v in dying.pop(-1, []))
    for i, node in enumerate(nodes):
        if node.op not in VIEW_OPS:
            for out in node.outputs:
                live += _bytes(out)
                dying.setdefault(last.get(id(out), i), []).append(out)
        peak = max(peak, live)
        live -= sum(_bytes(v) for v in dying.pop(i, []))
    return peak


def _unique_inputs(node: Node) -> list[Value]:
    return list({id(v): v for v in node.inputs if v is not None}.values())


def memory_aware_order(graph: Graph) -> list[Node]:
    nodes = list(graph.nodes)
    members = {id(n) for n in nodes}
    index = {id(n): i for i, n in enumerate(nodes)}
    waiting = {
        id(n): len({id(v.producer) for v in n.inputs if v is not None and v.producer is not None and id(v.producer) in members})
        for n in nodes
    }
    uses_left: dict[int, int] = {}
    for n in nodes:
        for v in _unique_inputs(n):
            uses_left[id(v)] = uses_left.get(id(v), 0) + 1
    outputs = {id(v) for v in graph.outputs}

    def delta(node: Node) -> int:
        if node.op in VIEW_OPS:
            return 0
        grown = sum(_bytes(o) for o in node.outputs)
        freed = sum(
            _bytes(v) for v in _unique_inputs(node) if uses_left.get(id(v)) == 1 and id(v) not in outputs
        )
        return grown - freed

    ready = [n for n in nodes if waiting[id(n)] == 0]
    order: list[Node] = []
    while ready:
        best = min(ready, key=lambda n: (delta(n), index[id(n)]))
        ready.remove(best)
        order.append(best)
        for v in _unique_inputs(best):
            uses_left[id(v)] -= 1
        released: set[int] = set()
        for out in best.outputs:
            for user in out.users:
                if id(user) in members and id(user) not in released:
                    released.add(id(user))
                    waiting[id(user)] -= 1
                    if waiting[id(user)] == 0:
                        ready.append(user)
    if len(order) != len(nodes):
        raise GraphError("graph has a cycle")
    return order


def apply_order(graph: Graph, order: Iterable[Node]) -> None:
    """Replace the node order with a topological permutation of the same nodes."""
    new = list(order)
    if len(new) != len(graph.nodes) or {id(n) for n in new} != {id(n) for n in graph.nodes}:
        raise GraphError("schedule is not a permutation of the graph's nodes")
    previous = graph.nodes
    graph.nodes = new
    try:
        graph.verify()
    except GraphError:
        graph.nodes = previous
        raise


def wavefronts(graph: Graph) -> list[list[Node]]:
    """ASAP levels: level(n) = 1 + max level of its producers."""
    level: dict[int, int] = {}
    levels: list[list[Node]] = []
    for node in graph.nodes:
        preds = [level[id(v.producer)] for v in node.inputs if v is not None and v.producer is not None]
        lv = 1 + max(preds) if preds else 0
        level[id(node)] = lv
        while len(levels) <= lv:
            levels.append([])
        levels[lv].append(node)
    return levels


def critical_path_flops(graph: Graph) -> tuple[int, int]:
    """(FLOPs on the longest FLOP-weighted path, total FLOPs)."""
    longest: dict[int, int] = {}
    total = 0
    for node in graph.nodes:
        f = ops.flops(node)
        total += f
        preds = [longest[id(v.producer)] for v in node.inputs if v is not None and v.producer is not None]
        longest[id(node)] = f + (max(preds) if preds else 0)
    return (max(longest.values()) if longest else 0), total


@dataclass
class ScheduleReport:
    nodes: int
    peak_before: int
    peak_after: int
    levels: int
    max_width: int
    critical_flops: int
    total_flops: int


def schedule(graph: Graph) -> ScheduleReport:
    """Reorder with memory_aware_order when that lowers the peak live bytes."""
    before = peak_live_bytes(graph)
    order = memory_aware_order(graph)
    after = peak_live_bytes(graph, order)
    if after < before:
        apply_order(graph, order)
    else:
        after = before
    levels = wavefronts(graph)
    crit, total = critical_path_flops(graph)
    return ScheduleReport(
        nodes=len(graph.nodes),
        peak_before=before,
        peak_after=after,
        levels=len(levels),
        max_width=max((len(lv) for lv in levels), default=0),
        critical_flops=crit,
        total_flops=total,
    )
