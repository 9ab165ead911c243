"""Node order: a memory-aware topological order, plus dataflow statistics.

Every topological order computes the same values; orders differ in how many bytes of
intermediate tensors are alive at once, and the planner's arena follows that peak. The order the
reference compiler picks (src/ml_graph_compiler/schedule.py) — which the planner offsets pinned
by tests/golden/reference_plans.json depend on — is a greedy list schedule: among the nodes
whose producers have all run, take the one that grows the live set least,

    growth(n) = bytes written by n - bytes of the inputs whose last remaining reader is n

(views write nothing; constants and graph outputs never free), the earliest in the current
order on ties. The new order is kept only when it lowers the peak of live bytes.

Live bytes count storage owners: a view (Reshape, Flatten, ...) owns nothing and keeps its
source alive while it is read. A node's inputs and outputs are alive together while it runs.
"""

from __future__ import annotations

from collections.abc import Iterable, Sequence
from dataclasses import dataclass

from . import ops
from .errors import GraphError
from .ir import Graph, Node, Value

VIEW_OPS = frozenset({"Reshape", "Flatten", "Squeeze", "Unsqueeze", "Identity", "Dropout"})


def _nbytes(value: Value) -> int:
    return 0 if value.is_constant or value.type is None else value.type.nbytes


def _owner(value: Value) -> Value:
    """The value whose storage ``value`` uses (itself unless it is a view's output)."""
    while value.producer is not None and value.producer.op in VIEW_OPS:
        value = value.producer.input(0)
    return value


def _distinct_inputs(node: Node) -> list[Value]:
    return list({id(v): v for v in node.inputs if v is not None}.values())


def peak_live_bytes(graph: Graph, order: Sequence[Node] | None = None) -> int:
    """Peak of live bytes over ``order`` (default: the graph's order). Graph inputs are alive
    from the start until their last read (unread inputs only at the very start), a node's
    outputs from its step to their storage's last read, graph outputs to the end."""
    steps = list(graph.nodes if order is None else order)
    n = len(steps)
    last_read: dict[int, int] = {}
    for i, node in enumerate(steps):
        for v in node.inputs:
            if v is not None and not v.is_constant:
                last_read[id(_owner(v))] = i
    for v in graph.outputs:
        last_read[id(_owner(v))] = n
    # bytes alive at each step: +size at the first step, -size after the last
    delta = [0] * (n + 2)
    at_start = 0
    for v in graph.inputs:
        size = _nbytes(v)
        at_start += size
        last = last_read.get(id(v), -1)
        if last >= 0:
            delta[0] += size
            delta[last + 1] -= size
    for i, node in enumerate(steps):
        if node.op in VIEW_OPS:
            continue
        for out in node.outputs:
            size = _nbytes(out)
            delta[i] += size
            delta[max(last_read.get(id(out), i), i) + 1] -= size
    peak, live = at_start, 0
    for i in range(n):
        live += delta[i]
        peak = max(peak, live)
    return peak


class _ListScheduler:
    """Greedy list scheduling by live-set growth (see the module docstring)."""

    def __init__(self, graph: Graph):
        self.graph = graph
        self.nodes = list(graph.nodes)
        self.rank = {id(n): i for i, n in enumerate(self.nodes)}
        self.graph_outputs = {id(v) for v in graph.outputs}
        self.readers_left: dict[int, int] = {}  # distinct reader nodes not yet scheduled
        self.blocked: dict[int, int] = {}       # distinct producers not yet scheduled
        self.followers: dict[int, list[Node]] = {id(n): [] for n in self.nodes}
        for node in self.nodes:
            for v in _distinct_inputs(node):
                self.readers_left[id(v)] = self.readers_left.get(id(v), 0) + 1
            producers = {id(v.producer): v.producer for v in node.inputs
                         if v is not None and v.producer is not None and id(v.producer) in self.rank}
            self.blocked[id(node)] = len(producers)
            for p in producers.values():
                self.followers[id(p)].append(node)

    def growth(self, node: Node) -> int:
        if node.op in VIEW_OPS:
            return 0
        freed = sum(_nbytes(v) for v in _distinct_inputs(node)
                    if self.readers_left.get(id(v)) == 1 and id(v) not in self.graph_outputs)
        return sum(_nbytes(o) for o in node.outputs) - freed

    def run(self) -> list[Node]:
        ready = {id(n): n for n in self.nodes if self.blocked[id(n)] == 0}
        order: list[Node] = []
        while ready:
            pick = min(ready.values(), key=lambda n: (self.growth(n), self.rank[id(n)]))
            del ready[id(pick)]
            order.append(pick)
            for v in _distinct_inputs(pick):
                self.readers_left[id(v)] -= 1
            for follower in self.followers[id(pick)]:
                self.blocked[id(follower)] -= 1
                if self.blocked[id(follower)] == 0:
                    ready[id(follower)] = follower
        if len(order) != len(self.nodes):
            raise GraphError("graph has a cycle")
        return order


def memory_aware_order(graph: Graph) -> list[Node]:
    """A topological order that keeps the live set small (greedy; see the module docstring)."""
    return _ListScheduler(graph).run()


def apply_order(graph: Graph, order: Iterable[Node]) -> None:
    """Install ``order`` (a permutation of the nodes); the graph is left unchanged when the
    order is not a permutation or not topological."""
    proposed = list(order)
    if len(proposed) != len(graph.nodes) or {id(n) for n in proposed} != {id(n) for n in graph.nodes}:
        raise GraphError("schedule is not a permutation of the graph's nodes")
    previous, graph.nodes = graph.nodes, proposed
    try:
        graph.verify()
    except GraphError:
        graph.nodes = previous
        raise


def _depths(graph: Graph) -> dict[int, int]:
    """ASAP level of every node: one more than its deepest producer, 0 without producers."""
    depth: dict[int, int] = {}
    for node in graph.nodes:
        above = [depth[id(v.producer)] for v in node.inputs if v is not None and v.producer is not None]
        depth[id(node)] = max(above) + 1 if above else 0
    return depth


def wavefronts(graph: Graph) -> list[list[Node]]:
    """Nodes grouped by ASAP level; the nodes of one level are independent of each other."""
    depth = _depths(graph)
    levels: list[list[Node]] = [[] for _ in range(max(depth.values(), default=-1) + 1)]
    for node in graph.nodes:
        levels[depth[id(node)]].append(node)
    return levels


def critical_path_flops(graph: Graph) -> tuple[int, int]:
    """(FLOPs of the heaviest producer-to-consumer path, total FLOPs); their ratio bounds what
    running independent operators concurrently can gain."""
    heaviest: dict[int, int] = {}
    for node in graph.nodes:
        above = [heaviest[id(v.producer)] for v in node.inputs if v is not None and v.producer is not None]
        heaviest[id(node)] = ops.flops(node) + max(above, default=0)
    total = sum(ops.flops(n) for n in graph.nodes)
    return max(heaviest.values(), default=0), total


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
    """Reorder ``graph`` by ``memory_aware_order`` when that lowers its peak live bytes."""
    before = peak_live_bytes(graph)
    order = memory_aware_order(graph)
    after = peak_live_bytes(graph, order)
    if after < before:
        apply_order(graph, order)
    else:
        after = before
    levels = wavefronts(graph)
    critical, total = critical_path_flops(graph)
    return ScheduleReport(nodes=len(graph.nodes), peak_before=before, peak_after=after, levels=len(levels),
                          max_width=max((len(level) for level in levels), default=0),
                          critical_flops=critical, total_flops=total)
