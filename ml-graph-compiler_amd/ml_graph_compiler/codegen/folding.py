"""Transposes folded into the operands of batched MatMuls.

The reference lowers a Transpose as its own loop nest (codegen/c.py:558-600), a full read and
write of the tensor, even when its only readers are matrix products that could read the
original through strides. The hip GEMM takes every operand as a base pointer with row, column
and per-batch-dimension strides, so:

* **input folding** — ``Y = Transpose(X)`` whose readers are all MatMuls emits nothing; each
  MatMul reads X with Y's dimensions' strides (e.g. the [B, S, H, D] -> [B, H, S, D] head split
  of attention, or K^T as [B, H, D, S]);
* **output folding** — ``Z = Transpose(MatMul(...))`` with the last axis kept in place has the
  MatMul write Z's memory with permuted strides (the head merge back to [B, S, H, D]).

The memory plan is not touched, so a fold is taken only where the plan allows it. Reading X
later than the plan assumed requires that nothing written between the Transpose and its last
reader overlaps X (the planner was free to reuse X's memory once the Transpose had read it),
including the reading MatMul's own output. Writing Z earlier than planned requires that
nothing read or written between the MatMul and the Transpose overlaps Z.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass, field

from .. import ops
from ..ir import Graph, Node, Value
from ..memory import MemoryPlan


@dataclass
class FoldPlan:
    inputs: dict[int, Node] = field(default_factory=dict)    # id(Transpose output) -> Transpose
    outputs: dict[int, Node] = field(default_factory=dict)   # id(MatMul) -> Transpose it writes for
    skipped: dict[int, str] = field(default_factory=dict)    # id(Transpose) -> why it emits nothing


def _overlap(plan: MemoryPlan, a: Value, b: Value) -> bool:
    la, lb = plan.location(a), plan.location(b)
    if la.kind != lb.kind or la.kind == "const":
        return False
    if la.kind in ("input", "output"):
        return la.index == lb.index
    return la.index < lb.index + b.tensor_type.nbytes and lb.index < la.index + a.tensor_type.nbytes


def _overlaps_workspace(plan: MemoryPlan, node: Node, v: Value, workspace_bytes: Callable[[Node], int]) -> bool:
    off = plan.workspaces.get(id(node))
    if off is None:
        return False
    loc = plan.location(v)
    if loc.kind != "arena":
        return False
    return loc.index < off + workspace_bytes(node) and off < loc.index + v.tensor_type.nbytes


def _keeps_last_axis(t: Node) -> bool:
    rank = t.output.tensor_type.rank
    perm = ops.transpose_perm(t, rank)
    return rank >= 2 and perm[-1] == rank - 1


def plan_folds(graph: Graph, plan: MemoryPlan, workspace_bytes: Callable[[Node], int],
               excluded: set[int]) -> FoldPlan:
    """Folds for the scheduled ``graph``; nodes in ``excluded`` (fused elsewhere) stay as they are."""
    pos = {id(n): i for i, n in enumerate(graph.nodes)}
    nodes = graph.nodes
    folds = FoldPlan()

    def written_between(v: Value, lo: int, hi: int) -> bool:
        """Does a node at position lo < p <= hi write memory overlapping v?"""
        for n in nodes[lo + 1 : hi + 1]:
            if id(n) in folds.skipped:
                continue
            if any(_overlap(plan, o, v) for o in n.outputs if o is not v):
                return True
            if _overlaps_workspace(plan, n, v, workspace_bytes):
                return True
        return False

    for t in nodes:
        if t.op != "Transpose" or id(t) in excluded:
            continue
        x, y = t.input(0), t.output
        if x.type is None or x.type.dtype != "float32" or y in graph.outputs or not y.users:
            continue
        if not all(u.op == "MatMul" and id(u) not in excluded and u.input(0).tensor_type.rank >= 2
                   and u.input(1).tensor_type.rank >= 2 for u in y.users):
            continue
        last = max(pos[id(u)] for u in y.users)
        if written_between(x, pos[id(t)], last):
            continue
        folds.inputs[id(y)] = t
        folds.skipped[id(t)] = "read through strides by the MatMul"

    for mm in nodes:
        if mm.op != "MatMul" or id(mm) in excluded:
            continue
        o = mm.output
        if o in graph.outputs or len(o.users) != 1 or o.tensor_type.rank < 2:
            continue
        if mm.input(0).tensor_type.rank < 2 or mm.input(1).tensor_type.rank < 2:
            continue
        t = o.users[0]
        if t.op != "Transpose" or id(t) in excluded or not _keeps_last_axis(t) or id(t) in folds.skipped:
            continue
        if t.output.tensor_type.dtype != "float32" or id(t.output) in folds.inputs:
            continue
        z = t.output
        lo, hi = pos[id(mm)], pos[id(t)]

        def actual(v: Value) -> Value:  # what a node really reads (a folded operand's source)
            return folds.inputs[id(v)].input(0) if id(v) in folds.inputs else v

        clash = False
        for n in nodes[lo:hi]:
            touched = [actual(v) for v in n.inputs if v is not None]
            touched += [v for v in n.outputs if v is not o]
            if any(_overlap(plan, v, z) for v in touched) or _overlaps_workspace(plan, n, z, workspace_bytes):
                clash = True
                break
        # sources of folded operands still to be read after the MatMul must survive its write
        for src_t in folds.inputs.values():
            last_read = max(pos[id(u)] for u in src_t.output.users)
            if pos[id(src_t)] < lo <= last_read and _overlap(plan, src_t.input(0), z):
                clash = True
        if clash:
            continue
        folds.outputs[id(mm)] = t
        folds.skipped[id(t)] = "written in place by the MatMul"
    return folds
