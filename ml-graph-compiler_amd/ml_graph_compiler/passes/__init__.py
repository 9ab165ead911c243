"""Optimization passes and the pass manager (reference: src/ml_graph_compiler/passes/__init__.py).

Pipelines are cumulative; each level adds one group of passes. O3 = loop fusion level.
"""

from __future__ import annotations

import time
from collections.abc import Callable, Sequence
from dataclasses import dataclass, field
from typing import Any

from ..errors import CompilerError
from ..ir import Graph
from .basic import eliminate_common_subexpressions, eliminate_dead_code, fold_constants
from .fusion import fuse
from .layout import to_nhwc
from .loopfuse import fuse_elementwise
from .simplify import simplify

PassFn = Callable[[Graph], int]

PASSES: dict[str, PassFn] = {
    "fold": fold_constants,
    "dce": eliminate_dead_code,
    "cse": eliminate_common_subexpressions,
    "simplify": simplify,
    "fuse": fuse,
    "layout": to_nhwc,
    "loopfuse": fuse_elementwise,
}

_FOLD = ["fold", "dce"]
_CSE = [*_FOLD, "cse", "dce"]
_SIMPLIFY = ["fold", "dce", "cse", "simplify", "fold", "cse", "dce"]
_FUSE = ["fold", "dce", "cse", "simplify", "fold", "cse", "fuse", "simplify", "dce"]
_LAYOUT = ["fold", "dce", "cse", "simplify", "fold", "cse", "fuse", "simplify", "layout", "cse", "dce"]
_LOOPFUSE = [*_LAYOUT, "loopfuse", "dce"]

PIPELINES: dict[str, list[str]] = {
    "O0": [],
    "fold": _FOLD,
    "cse": _CSE,
    "simplify": _SIMPLIFY,
    "fuse": _FUSE,
    "layout": _LAYOUT,
    "loopfuse": _LOOPFUSE,
    "O1": _SIMPLIFY,
    "O2": _FUSE,
    "O3": _LOOPFUSE,
}


@dataclass
class PassRecord:
    name: str
    changes: int
    nodes_after: int
    seconds: float


@dataclass
class PassReport:
    nodes_before: int
    records: list[PassRecord] = field(default_factory=list)

    @property
    def nodes_after(self) -> int:
        return self.records[-1].nodes_after if self.records else self.nodes_before

    def to_dict(self) -> dict[str, Any]:
        return {
            "nodes_before": self.nodes_before,
            "nodes_after": self.nodes_after,
            "passes": [r.__dict__ for r in self.records],
        }


def resolve(passes: str | Sequence[str]) -> list[str]:
    """A pipeline name, a comma-separated pass list, or a sequence of pass names."""
    if isinstance(passes, str):
        if passes in PIPELINES:
            return list(PIPELINES[passes])
        names = [p.strip() for p in passes.split(",") if p.strip()]
    else:
        names = list(passes)
    unknown = [n for n in names if n not in PASSES]
    if unknown:
        raise CompilerError(f"unknown passes {unknown}; known: {sorted(PASSES)} or {sorted(PIPELINES)}")
    return names


def optimize(graph: Graph, passes: str | Sequence[str] = "O3", verify: bool = True) -> PassReport:
    """Run passes in place, verifying the graph after each by default."""
    report = PassReport(nodes_before=len(graph.nodes))
    for name in resolve(passes):
        t0 = time.perf_counter()
        changes = PASSES[name](graph)
        if verify:
            graph.verify()
        report.records.append(PassRecord(name, changes, len(graph.nodes), round(time.perf_counter() - t0, 4)))
    return report


__all__ = [
    "PASSES",
    "PIPELINES",
    "PassReport",
    "eliminate_common_subexpressions",
    "eliminate_dead_code",
    "fold_constants",
    "fuse",
    "fuse_elementwise",
    "optimize",
    "resolve",
    "simplify",
    "to_nhwc",
]
