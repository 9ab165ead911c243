"""Static memory planning: liveness, aliasing, in-place reuse and offset assignment.

Reference: src/ml_graph_compiler/memory.py:1-316. The hip backend consumes these offsets
verbatim (with alignment 256): every non-constant tensor lives at a fixed byte offset of one
arena inside the model's single HBM allocation, so a compiled forward pass allocates nothing.

1. Storage groups: view operators alias their input; an elementwise operator may write over a
   same-shaped, same-itemsize input that dies at it (in place). Union-find merges them.
2. Liveness: with nodes numbered in schedule order, a group lives on [first definition, last
   use]; graph outputs live to the end; inputs and constants are external. A node's workspace
   (split-K partials of a small GEMM, for example) is a group live on [i, i].
3. Offsets: greedy by size (largest first, ties by start; each at the lowest aligned offset
   clear of every time-overlapping placed group), first fit (definition order) or naive.
4. Bounds: the peak of summed live sizes is a lower bound for any valid arena.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass, field
from typing import Literal

from . import ops
from .errors import GraphError
from .ir import Graph, Node, Value

ALIAS_OPS = frozenset({"Reshape", "Flatten", "Squeeze", "Unsqueeze", "Identity", "Dropout"})
INPLACE_OPS = frozenset(op for op in ops.REGISTRY if ops.is_elementwise(op)) | {"FusedElementwise"}

Strategy = Literal["greedy_by_size", "first_fit", "naive"]
STRATEGIES: tuple[Strategy, ...] = ("greedy_by_size", "first_fit", "naive")
WorkspaceFn = Callable[[Node], int]


def align_up(n: int, alignment: int) -> int:
    return -(-n // alignment) * alignment


@dataclass(frozen=True)
class Location:
    """``arena`` (index = byte offset), ``input`` / ``output`` (index = position) or ``const``."""

    kind: Literal["arena", "input", "output", "const"]
    index: int = 0


@dataclass
class Buffer:
    id: int
    size: int
    start: int
    end: int
    values: list[Value] = field(default_factory=list)
    offset: int = -1
    workspace_of: Node | None = None

    def overlaps_in_time(self, other: Buffer) -> bool:
        return self.start <= other.end and other.start <= self.end


@dataclass
class MemoryPlan:
    strategy: str
    alignment: int
    arena_bytes: int
    lower_bound: int
    naive_bytes: int
    buffers: list[Buffer]
    locations: dict[int, Location]
    workspaces: dict[int, int]
    copies: list[tuple[Value, int]]
    inplace: int
    aliases: int

    def location(self, value: Value) -> Location:
        if value.is_constant:
            return Location("const")
        if id(value) not in self.locations:
            raise GraphError(f"value {value.name!r} has no planned location")
        return self.locations[id(value)]

    def offset(self, value: Value) -> int:
        loc = self.location(value)
        if loc.kind != "arena":
            raise GraphError(f"value {value.name!r} is not in the arena ({loc.kind})")
        return loc.index

    def verify(self) -> None:
        """No two buffers alive at the same time may overlap in the arena."""
        placed = sorted((b for b in self.buffers if b.offset >= 0), key=lambda b: b.offset)
        for i, a in enumerate(placed):
            if a.offset % self.alignment:
                raise GraphError(f"buffer {a.id} is misaligned")
            if a.offset + a.size > self.arena_bytes:
                raise GraphError(f"buffer {a.id} exceeds the arena")
            for b in placed[i + 1 :]:
                if b.offset >= a.offset + a.size:
                    break
                if a.overlaps_in_time(b):
                    raise GraphError(f"buffers {a.id} and {b.id} overlap in time and space")

    def summary(self) -> dict[str, object]:
        return {
            "strategy": self.strategy,
            "arena_bytes": self.arena_bytes,
            "lower_bound_bytes": self.lower_bound,
            "naive_bytes": self.naive_bytes,
            "buffers": len(self.buffers),
            "aliases": self.aliases,
            "inplace": self.inplace,
            "reuse_factor": round(self.naive_bytes / self.arena_bytes, 2) if self.arena_bytes else 1.0,
        }


class _DisjointSets:
    def __init__(self) -> None:
        self.parent: dict[int, int] = {}

    def find(self, x: int) -> int:
        self.parent.setdefault(x, x)
        root = x
        while self.parent[root] != root:
            root = self.parent[root]
        while self.parent[x] != root:
            self.parent[x], x = root, self.parent[x]
        return root

    def union(self, a: int, b: int) -> None:
        ra, rb = self.find(a), self.find(b)
        if ra != rb:
            self.parent[rb] = ra


def _place(order: list[Buffer], alignment: int) -> int:
    placed: list[Buffer] = []
    top = 0
    for buf in order:
        offset = 0
        for p in sorted((p for p in placed if p.overlaps_in_time(buf)), key=lambda p: p.offset):
            if offset + buf.size <= p.offset:
                break
            offset = max(offset, align_up(p.offset + p.size, alignment))
        buf.offset = offset
        placed.append(buf)
        top = max(top, offset + buf.size)
    return align_up(top, alignment)


def plan_memory(
    graph: Graph,
    strategy: Strategy = "greedy_by_size",
    alignment: int = 64,
    inplace: bool = True,
    workspace: WorkspaceFn | None = None,
) -> MemoryPlan:
    """Assign every non-constant value a location."""
    if strategy not in STRATEGIES:
        raise GraphError(f"unknown strategy {strategy!r}; known: {STRATEGIES}")
    n_nodes = len(graph.nodes)
    sets = _DisjointSets()
    values: dict[int, Value] = {}
    external: dict[int, Location] = {}
    for i, v in enumerate(graph.inputs):
        values[id(v)] = v
        external[id(v)] = Location("input", i)

    last_use: dict[int, int] = {}
    for i, node in enumerate(graph.nodes):
        for v in node.inputs:
            if v is not None and not v.is_constant:
                last_use[id(v)] = i
    outputs = {id(v) for v in graph.outputs}
    for v in graph.outputs:
        last_use[id(v)] = n_nodes

    aliases = inplace_count = 0
    for i, node in enumerate(graph.nodes):
        for out in node.outputs:
            values[id(out)] = out
            sets.find(id(out))
        x = node.inputs[0] if node.inputs else None
        if node.op in ALIAS_OPS and x is not None:
            if x.is_constant:
                external[id(node.outputs[0])] = Location("const")
            else:
                sets.union(id(x), id(node.outputs[0]))
                aliases += 1
            continue
        if not inplace or node.op not in INPLACE_OPS or len(node.outputs) != 1:
            continue
        out = node.output
        for cand in node.inputs:
            if cand is None or cand.is_constant or cand.type is None or out.type is None:
                continue
            root = sets.find(id(cand))
            if any(sets.find(e) == root for e in external):
                continue
            if cand.type.shape != out.type.shape or cand.type.itemsize != out.type.itemsize:
                continue
            group = [k for k in values if sets.find(k) == root]
            if any(k in outputs for k in group):
                continue
            if max(last_use.get(k, -1) for k in group) != i:
                continue
            sets.union(root, id(out))
            inplace_count += 1
            break

    groups: dict[int, list[Value]] = {}
    for k, v in values.items():
        groups.setdefault(sets.find(k), []).append(v)
    locations: dict[int, Location] = {}
    copies: list[tuple[Value, int]] = []
    output_slot: dict[int, int] = {}
    for j, v in enumerate(graph.outputs):
        if v.is_constant:
            copies.append((v, j))
            continue
        root = sets.find(id(v))
        if root in output_slot or any(sets.find(e) == root for e in external):
            copies.append((v, j))
        else:
            output_slot[root] = j

    defined_at: dict[int, int] = {}
    for i, node in enumerate(graph.nodes):
        for out in node.outputs:
            defined_at[id(out)] = i
    buffers: list[Buffer] = []
    for root, members in groups.items():
        ext = next((external[id(m)] for m in members if id(m) in external), None)
        if ext is not None:
            for m in members:
                locations[id(m)] = ext
            continue
        if root in output_slot:
            for m in members:
                locations[id(m)] = Location("output", output_slot[root])
            continue
        start = min(defined_at.get(id(m), 0) for m in members)
        end = max(max(last_use.get(id(m), -1) for m in members), start)
        size = align_up(max(m.tensor_type.nbytes for m in members), alignment) if members else 0
        buffers.append(Buffer(len(buffers), size, start, end, members))

    workspaces: dict[int, int] = {}
    if workspace is not None:
        for i, node in enumerate(graph.nodes):
            need = workspace(node)
            if need > 0:
                buffers.append(Buffer(len(buffers), align_up(need, alignment), i, i, [], workspace_of=node))

    events: dict[int, int] = {}
    for b in buffers:
        events[b.start] = events.get(b.start, 0) + b.size
        events[b.end + 1] = events.get(b.end + 1, 0) - b.size
    lower = live = 0
    for t in sorted(events):
        live += events[t]
        lower = max(lower, live)
    naive = sum(b.size for b in buffers)

    if strategy == "naive":
        arena = 0
        for b in buffers:
            b.offset = arena
            arena += b.size
    elif strategy == "first_fit":
        arena = _place(sorted(buffers, key=lambda b: (b.start, -b.size)), alignment)
    else:
        arena = _place(sorted(buffers, key=lambda b: (-b.size, b.start)), alignment)

    for b in buffers:
        for m in b.values:
            locations[id(m)] = Location("arena", b.offset)
        if b.workspace_of is not None:
            workspaces[id(b.workspace_of)] = b.offset
    plan = MemoryPlan(
        strategy=strategy,
        alignment=alignment,
        arena_bytes=arena,
        lower_bound=lower,
        naive_bytes=naive,
        buffers=buffers,
        locations=locations,
        workspaces=workspaces,
        copies=copies,
        inplace=inplace_count,
        aliases=aliases,
    )
    plan.verify()
    return plan
