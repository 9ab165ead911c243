"""Static memory plan: one byte offset per tensor inside a single arena.

The hip backend uses these offsets verbatim (alignment 256): every non-constant tensor of a
compiled model lives at a fixed offset of one arena inside the model's one HBM allocation, so a
forward pass allocates nothing. The offsets must equal the reference planner's
(src/ml_graph_compiler/memory.py) for the same graph, strategy and alignment; they are pinned by
tests/golden/reference_plans.json. The rules that fix them:

* Storage slots. A view operator (ALIAS_OPS) writes nothing: its output shares its input's
  slot (a view of a constant is a constant). An elementwise operator may write over one of its
  inputs in place — the first input, in input order, that is not a constant, has the output's
  shape and element size, whose slot holds no graph input or output, and whose slot's last
  reader is this node.
* Placement. Graph inputs keep their caller buffers, and each graph output gets its caller
  buffer unless another output or an input already owns its slot (then it is copied at the
  end). Every other slot is one arena block alive from its first definition to its last read
  (graph outputs to the end); a node that needs scratch memory gets a block alive during that
  node only. Blocks are placed one by one at the lowest aligned offset that clears every placed
  block alive at an overlapping time — largest first (ties: earliest start) for
  ``greedy_by_size``, earliest first (ties: largest) for ``first_fit``; ``naive`` stacks them.
* Bounds. The largest total size of the blocks alive at one time is a lower bound for any
  valid arena; the sum of all blocks is the naive size.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from dataclasses import dataclass, field
from itertools import accumulate
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
    return (n + alignment - 1) // alignment * alignment


@dataclass(frozen=True)
class Location:
    """Where a value lives: ``arena`` (index = byte offset), ``input`` / ``output`` (index =
    position in the caller's pointer list) or ``const`` (the weights blob)."""

    kind: Literal["arena", "input", "output", "const"]
    index: int = 0


@dataclass
class Buffer:
    """One arena block: the storage of a slot, or the scratch of one node."""

    id: int
    size: int
    start: int
    end: int
    values: list[Value] = field(default_factory=list)
    offset: int = -1
    workspace_of: Node | None = None

    def overlaps_in_time(self, other: Buffer) -> bool:
        return not (self.end < other.start or other.end < self.start)


@dataclass
class MemoryPlan:
    strategy: str
    alignment: int
    arena_bytes: int
    lower_bound: int
    naive_bytes: int
    buffers: list[Buffer]
    locations: dict[int, Location]
    workspaces: dict[int, int]        # id(node) -> byte offset of its scratch block
    copies: list[tuple[Value, int]]   # outputs copied into output slot j at the end
    inplace: int
    aliases: int

    def location(self, value: Value) -> Location:
        if value.is_constant:
            return Location("const")
        found = self.locations.get(id(value))
        if found is None:
            raise GraphError(f"value {value.name!r} has no planned location")
        return found

    def offset(self, value: Value) -> int:
        where = self.location(value)
        if where.kind != "arena":
            raise GraphError(f"value {value.name!r} is not in the arena ({where.kind})")
        return where.index

    def verify(self) -> None:
        """Every block aligned and inside the arena; no two blocks alive together overlap."""
        placed = [b for b in self.buffers if b.offset >= 0]
        for b in placed:
            if b.offset % self.alignment:
                raise GraphError(f"buffer {b.id} is misaligned")
            if b.offset + b.size > self.arena_bytes:
                raise GraphError(f"buffer {b.id} exceeds the arena")
        placed.sort(key=lambda b: b.offset)
        for i, low in enumerate(placed):
            for high in placed[i + 1:]:
                if high.offset >= low.offset + low.size:
                    break  # sorted by offset: nothing further overlaps ``low`` in space
                if low.overlaps_in_time(high):
                    raise GraphError(f"buffers {low.id} and {high.id} overlap in time and space")

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


class _Slot:
    """Values sharing one storage; ``external`` is set when that storage is a graph input or a
    constant (then it is not planned)."""

    __slots__ = ("members", "external", "output")

    def __init__(self, first: Value, external: Location | None = None):
        self.members = [first]
        self.external = external
        self.output: int | None = None


class _Slots:
    def __init__(self) -> None:
        self.order: list[_Slot] = []
        self.of: dict[int, _Slot] = {}

    def new(self, value: Value, external: Location | None = None) -> None:
        slot = _Slot(value, external)
        self.order.append(slot)
        self.of[id(value)] = slot

    def join(self, value: Value, slot: _Slot) -> None:
        slot.members.append(value)
        self.of[id(value)] = slot


def _lowest_gap(size: int, busy: list[tuple[int, int]]) -> int:
    """The lowest offset where ``size`` bytes fit between the busy [begin, end) ranges (all
    aligned), scanning them by begin."""
    candidate = 0
    for begin, end in sorted(busy):
        if candidate + size <= begin:
            break
        candidate = max(candidate, end)
    return candidate


def _place(order: list[Buffer], alignment: int) -> int:
    done: list[Buffer] = []
    top = 0
    for block in order:
        busy = [(b.offset, align_up(b.offset + b.size, alignment)) for b in done if b.overlaps_in_time(block)]
        block.offset = _lowest_gap(block.size, busy)
        done.append(block)
        top = max(top, block.offset + block.size)
    return align_up(top, alignment)


def _peak_concurrent(blocks: list[Buffer], steps: int) -> int:
    """Largest total size of the blocks alive at one step (difference array over the steps)."""
    change = [0] * (steps + 2)
    for b in blocks:
        change[b.start] += b.size
        change[b.end + 1] -= b.size
    return max(accumulate(change), default=0)


def plan_memory(graph: Graph, strategy: Strategy = "greedy_by_size", alignment: int = 64,
                inplace: bool = True, workspace: WorkspaceFn | None = None,
                extra_reads: Mapping[int, int] | None = None) -> MemoryPlan:
    """Assign every non-constant value of a scheduled graph a location.

    ``extra_reads`` maps id(value) to a step at which a code generator reads that value besides
    the graph's own readers (a node fused into a later one reads its inputs there): the value
    then stays alive, and unwritten, through that step."""
    if strategy not in STRATEGIES:
        raise GraphError(f"unknown strategy {strategy!r}; known: {STRATEGIES}")
    steps = len(graph.nodes)
    # step of the last read of every value; graph outputs are read after the last node
    last_read: dict[int, int] = {}
    for step, node in enumerate(graph.nodes):
        for v in node.inputs:
            if v is not None and not v.is_constant:
                last_read[id(v)] = step
    for v in graph.outputs:
        last_read[id(v)] = steps
    for key, step in (extra_reads or {}).items():
        last_read[key] = max(last_read.get(key, -1), step)
    output_ids = {id(v) for v in graph.outputs}

    slots = _Slots()
    for k, v in enumerate(graph.inputs):
        slots.new(v, Location("input", k))
    born: dict[int, int] = {}
    n_alias = n_inplace = 0
    for step, node in enumerate(graph.nodes):
        for out in node.outputs:
            born[id(out)] = step
        source = node.inputs[0] if node.inputs else None
        if node.op in ALIAS_OPS and source is not None:
            if source.is_constant:
                slots.new(node.outputs[0], Location("const"))
                for out in node.outputs[1:]:
                    slots.new(out)
            else:
                slots.join(node.outputs[0], slots.of[id(source)])
                for out in node.outputs[1:]:
                    slots.new(out)
                n_alias += 1
            continue
        target = None
        if inplace and node.op in INPLACE_OPS and len(node.outputs) == 1:
            target = _inplace_target(node, step, slots, last_read, output_ids)
        if target is not None:
            slots.join(node.output, target)
            n_inplace += 1
        else:
            for out in node.outputs:
                slots.new(out)

    copies: list[tuple[Value, int]] = []
    for j, v in enumerate(graph.outputs):
        slot = None if v.is_constant else slots.of.get(id(v))
        if slot is None or slot.external is not None or slot.output is not None:
            copies.append((v, j))
        else:
            slot.output = j

    locations: dict[int, Location] = {}
    buffers: list[Buffer] = []
    for slot in slots.order:
        if slot.external is not None or slot.output is not None:
            where = slot.external if slot.external is not None else Location("output", slot.output or 0)
            locations.update((id(m), where) for m in slot.members)
            continue
        start = min(born.get(id(m), 0) for m in slot.members)
        end = max([start] + [last_read.get(id(m), -1) for m in slot.members])
        size = align_up(max(m.tensor_type.nbytes for m in slot.members), alignment)
        buffers.append(Buffer(len(buffers), size, start, end, list(slot.members)))
    if workspace is not None:
        for step, node in enumerate(graph.nodes):
            need = workspace(node)
            if need > 0:
                buffers.append(Buffer(len(buffers), align_up(need, alignment), step, step, workspace_of=node))

    if strategy == "naive":
        arena = 0
        for b in buffers:
            b.offset, arena = arena, arena + b.size
    else:
        key = (lambda b: (-b.size, b.start)) if strategy == "greedy_by_size" else (lambda b: (b.start, -b.size))
        arena = _place(sorted(buffers, key=key), alignment)

    workspaces: dict[int, int] = {}
    for b in buffers:
        locations.update((id(m), Location("arena", b.offset)) for m in b.values)
        if b.workspace_of is not None:
            workspaces[id(b.workspace_of)] = b.offset
    plan = MemoryPlan(strategy=strategy, alignment=alignment, arena_bytes=arena,
                      lower_bound=_peak_concurrent(buffers, steps), naive_bytes=sum(b.size for b in buffers),
                      buffers=buffers, locations=locations, workspaces=workspaces, copies=copies,
                      inplace=n_inplace, aliases=n_alias)
    plan.verify()
    return plan


def _inplace_target(node: Node, step: int, slots: _Slots, last_read: dict[int, int],
                    output_ids: set[int]) -> _Slot | None:
    """The slot of the first input this elementwise node may overwrite, if any."""
    out_t = node.output.type
    if out_t is None:
        return None
    for cand in node.inputs:
        if cand is None or cand.is_constant or cand.type is None:
            continue
        slot = slots.of[id(cand)]
        if slot.external is not None:
            continue
        if cand.type.shape != out_t.shape or cand.type.itemsize != out_t.itemsize:
            continue
        if any(id(m) in output_ids for m in slot.members):
            continue
        if max(last_read.get(id(m), -1) for m in slot.members) == step:
            return slot
    return None
