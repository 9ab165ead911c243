"""Graph optimization passes and the pass manager.

Pass names and cumulative pipelines are the reference's interface
(src/ml_graph_compiler/passes/__init__.py): ``O0`` runs nothing, ``O1`` = ``simplify``,
``O2`` = ``fuse``, ``O3`` = ``loopfuse`` (NHWC layout plus loop fusion). ``optimize`` runs a
pipeline in place, verifies the graph after every pass and reports what each pass did.

Modules: ``cleanup`` (fold, dce, cse), ``algebra`` (simplify), ``patterns`` (LayerNorm and
GELU recognition), ``epilogue`` (Conv/GEMM fusion with bias, residual and activation),
``nhwc`` (layout), ``loops`` (elementwise loop fusion), ``graph_tools`` (shared helpers).
"""

from __future__ import annotations

import time
from collections.abc import Callable, Sequence
from dataclasses import dataclass, field
from typing import Any

from ..errors import CompilerError
from ..ir import Graph
from .algebra import simplify
from .cleanup import eliminate_common_subexpressions, eliminate_dead_code, fold_constants
from .epilogue import fuse_conv, fuse_gemm
from .loops import fuse_elementwise
from .nhwc import to_nhwc
from .patterns import fuse_gelu, fuse_layer_norm


def fuse(graph: Graph) -> int:
    """LayerNorm and GELU recognition, then Conv and GEMM fusion; returns the rewrites."""
    return fuse_layer_norm(graph) + fuse_gelu(graph) + fuse_conv(graph) + fuse_gemm(graph)


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


def _levels() -> dict[str, list[str]]:
    """Each level extends the one before it."""
    front = ["fold", "dce", "cse"]
    simplified = front + ["simplify", "fold", "cse"]
    fused = simplified + ["fuse", "simplify"]
    layout = fused + ["layout", "cse", "dce"]
    levels = {
        "O0": [],
        "fold": ["fold", "dce"],
        "cse": front + ["dce"],
        "simplify": simplified + ["dce"],
        "fuse": fused + ["dce"],
        "layout": layout,
        "loopfuse": layout + ["loopfuse", "dce"],
    }
    levels.update(O1=levels["simplify"], O2=levels["fuse"], O3=levels["loopfuse"])
    return levels


PIPELINES: dict[str, list[str]] = _levels()


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
        return {"nodes_before": self.nodes_before, "nodes_after": self.nodes_after,
                "passes": [vars(r) for r in self.records]}


def resolve(passes: str | Sequence[str]) -> list[str]:
    """A pipeline name, a comma-separated list of pass names, or a sequence of pass names."""
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
    """Run ``passes`` on ``graph`` in place (verifying after each one unless told not to)."""
    report = PassReport(nodes_before=len(graph.nodes))
    for name in resolve(passes):
        began = time.perf_counter()
        changes = PASSES[name](graph)
        if verify:
            graph.verify()
        report.records.append(PassRecord(name, changes, len(graph.nodes), round(time.perf_counter() - began, 4)))
    return report


__all__ = ["PASSES", "PIPELINES", "PassReport", "eliminate_common_subexpressions", "eliminate_dead_code",
           "fold_constants", "fuse", "fuse_elementwise", "optimize", "resolve", "simplify", "to_nhwc"]
