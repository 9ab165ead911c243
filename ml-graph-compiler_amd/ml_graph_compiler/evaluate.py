"""Node-by-node evaluation of a graph with the operator table's numpy semantics.

What the reference's interpreter does (src/ml_graph_compiler/interpreter.py): every node runs
through its ``ops.run`` in graph order. ``mgc compile --check`` uses it on the unoptimized graph
as the baseline for the compiled model's outputs. It is a plain CPU evaluator for checking;
no compiled model ever falls back to it.
"""

from __future__ import annotations

from collections.abc import Mapping

import numpy as np

from . import ops
from .errors import GraphError
from .ir import Graph, Value


def evaluate_graph(graph: Graph, feeds: Mapping[str, np.ndarray]) -> dict[str, np.ndarray]:
    """The named outputs of ``graph`` for ``feeds`` (one array per graph input, by name)."""
    wanted = {v.name: v for v in graph.inputs}
    if set(feeds) != set(wanted):
        raise GraphError(f"inputs: expected {sorted(wanted)}, got {sorted(feeds)}")
    values: dict[int, np.ndarray] = {}
    for name, v in wanted.items():
        array = np.asarray(feeds[name])
        if v.type is not None and (array.shape != v.type.shape or array.dtype != np.dtype(v.type.dtype)):
            raise GraphError(f"input {name!r}: expected {v.type}, got {array.dtype}{list(array.shape)}")
        values[id(v)] = array

    def read(v: Value | None) -> np.ndarray | None:
        if v is None:
            return None
        return v.data if v.data is not None else values[id(v)]

    for node in graph.nodes:
        for out, array in zip(node.outputs, ops.run(node, [read(v) for v in node.inputs]), strict=True):
            values[id(out)] = array
    return {name: read(v) for name, v in graph.named_outputs()}
