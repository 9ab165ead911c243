"""The graph IR the compiler stages pass along: SSA values, operator nodes, one graph.

Interface of the reference IR (src/ml_graph_compiler/ir.py): the class and method names, the
``Value`` / ``Node`` fields and the observable orders — ``values()`` lists graph inputs, then
node inputs, node outputs and graph outputs, each value once; ``topological_sort`` is stable
(when several nodes are ready, the one that currently comes first runs first); fresh names are
``<hint>_<n>`` from one counter. The implementation is this package's own.

Every value is defined exactly once: as a graph input, as a constant (its ``data`` is set), or
as an output of one node. Values keep their readers in ``users`` (a node appears once per input
slot that reads the value), so passes can rewrite without rebuilding indexes.
"""

from __future__ import annotations

import heapq
import itertools
from collections.abc import Iterable, Iterator
from dataclasses import dataclass
from typing import Any

import numpy as np

from .errors import GraphError

# element types the IR accepts, by name
SUPPORTED_DTYPES = ("float32", "float64", "float16", "int64", "int32", "int8", "uint8", "bool")
_BY_NAME = {name: np.dtype(name) for name in SUPPORTED_DTYPES}


def contiguous(array: Any, dtype: Any = None) -> np.ndarray:
    """A C-ordered ndarray of ``array`` (a view when already one); rank is preserved."""
    return np.asarray(array, dtype=dtype, order="C")


def numpy_dtype(name: str) -> np.dtype:
    try:
        return _BY_NAME[name]
    except KeyError:
        raise GraphError(f"unsupported dtype {name!r}") from None


def dtype_name(dtype: Any) -> str:
    wanted = np.dtype(dtype)
    for name, candidate in _BY_NAME.items():
        if candidate == wanted:
            return name
    raise GraphError(f"unsupported numpy dtype {wanted}")


@dataclass(frozen=True)
class TensorType:
    """A dtype name and a static shape."""

    dtype: str
    shape: tuple[int, ...]

    def __post_init__(self) -> None:
        numpy_dtype(self.dtype)
        if not all(isinstance(d, int) and d >= 0 for d in self.shape):
            raise GraphError(f"shape must be non-negative integers, got {self.shape}")

    @property
    def rank(self) -> int:
        return len(self.shape)

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def itemsize(self) -> int:
        return _BY_NAME[self.dtype].itemsize

    @property
    def nbytes(self) -> int:
        return self.size * self.itemsize

    def __str__(self) -> str:
        return self.dtype + "[" + "x".join(str(d) for d in self.shape) + "]"

    @staticmethod
    def of(array: np.ndarray) -> TensorType:
        return TensorType(dtype_name(array.dtype), tuple(int(d) for d in array.shape))


class Value:
    """An SSA value: a graph input, a constant (``data`` set) or a node output."""

    __slots__ = ("data", "name", "producer", "type", "users")

    def __init__(self, name: str, type: TensorType | None = None, data: np.ndarray | None = None):
        self.name = name
        self.type = type
        self.data = data
        self.producer: Node | None = None
        self.users: list[Node] = []

    @property
    def is_constant(self) -> bool:
        return self.data is not None

    @property
    def tensor_type(self) -> TensorType:
        if self.type is None:
            raise GraphError(f"value {self.name!r} has no inferred type")
        return self.type

    def __repr__(self) -> str:
        return f"Value({self.name!r}, {self.type})"


class Node:
    """One operator application; an omitted optional input is ``None``."""

    __slots__ = ("attrs", "inputs", "name", "op", "outputs")

    def __init__(self, op: str, inputs: list[Value | None], outputs: list[Value],
                 attrs: dict[str, Any] | None = None, name: str = ""):
        self.op = op
        self.inputs = inputs
        self.outputs = outputs
        self.attrs: dict[str, Any] = dict(attrs or {})
        self.name = name

    def input(self, i: int) -> Value:
        """Input ``i``, which must be present."""
        value = self.optional_input(i)
        if value is None:
            raise GraphError(f"{self.op} node {self.name!r} is missing input {i}")
        return value

    def optional_input(self, i: int) -> Value | None:
        return self.inputs[i] if 0 <= i < len(self.inputs) else None

    @property
    def output(self) -> Value:
        return self.outputs[0]

    def __repr__(self) -> str:
        reads = ", ".join("_" if v is None else v.name for v in self.inputs)
        writes = ", ".join(v.name for v in self.outputs)
        suffix = f" {self.attrs}" if self.attrs else ""
        return f"{writes} = {self.op}({reads}){suffix}"


class _NameTable:
    """Names handed out in one graph: requested names when free, else ``<hint>_<n>``."""

    def __init__(self) -> None:
        self.taken: set[str] = set()
        self.serial = itertools.count()

    def fresh(self, hint: str) -> str:
        name = f"{hint}_{next(self.serial)}"
        while name in self.taken:
            name = f"{hint}_{next(self.serial)}"
        self.taken.add(name)
        return name

    def claim(self, wanted: str) -> str:
        if not wanted or wanted in self.taken:
            return self.fresh(wanted or "v")
        self.taken.add(wanted)
        return wanted


class Graph:
    """Nodes in execution order, graph inputs, and outputs under fixed public names."""

    def __init__(self, name: str = "graph"):
        self.name = name
        self.opset = 17
        self.inputs: list[Value] = []
        self.outputs: list[Value] = []
        self.output_names: list[str] = []  # the public names; passes may swap the values
        self.nodes: list[Node] = []
        self._table = _NameTable()

    # -- names ---------------------------------------------------------------------------------
    def fresh_name(self, hint: str = "v") -> str:
        return self._table.fresh(hint)

    def _claim(self, name: str) -> str:
        return self._table.claim(name)

    # -- building ------------------------------------------------------------------------------
    def add_input(self, name: str, type: TensorType) -> Value:
        value = Value(self._claim(name), type)
        self.inputs.append(value)
        return value

    def constant(self, array: np.ndarray, name: str = "const") -> Value:
        """A constant value; it belongs to no node and lives as long as something reads it."""
        data = contiguous(array)
        return Value(self._claim(name), TensorType.of(data), data)

    def add_node(self, op: str, inputs: list[Value | None], n_outputs: int = 1,
                 attrs: dict[str, Any] | None = None, name: str = "",
                 output_names: list[str] | None = None, index: int | None = None) -> Node:
        """A node with fresh output values, appended or inserted before position ``index``."""
        wanted = list(output_names) if output_names else [f"{name or op.lower()}_out"] * n_outputs
        node = Node(op, list(inputs), [], attrs, name or self.fresh_name(op.lower()))
        for out_name in wanted:
            value = Value(self._claim(out_name))
            value.producer = node
            node.outputs.append(value)
        for value in node.inputs:
            if value is not None:
                value.users.append(node)
        self.nodes.insert(len(self.nodes) if index is None else index, node)
        return node

    # -- rewriting -----------------------------------------------------------------------------
    def set_input(self, node: Node, i: int, value: Value | None) -> None:
        """Point input slot ``i`` of ``node`` at ``value``, keeping use lists right."""
        _drop_use(node.inputs[i], node)
        node.inputs[i] = value
        if value is not None:
            value.users.append(node)

    def remove_node(self, node: Node) -> None:
        """Delete a node nothing reads any more."""
        for out in node.outputs:
            if out.users or any(out is o for o in self.outputs):
                raise GraphError(f"cannot remove {node.op} {node.name!r}: output still used")
        for value in node.inputs:
            _drop_use(value, node)
        self.nodes.remove(node)

    def remove_nodes(self, dead: Iterable[Node]) -> int:
        """Delete a set of nodes whose outputs are read only inside the set; returns how many."""
        doomed = {id(n): n for n in dead}
        for node in doomed.values():
            for value in node.inputs:
                if value is not None and node in value.users:
                    value.users.remove(node)
        if doomed:
            self.nodes = [n for n in self.nodes if id(n) not in doomed]
        return len(doomed)

    def replace_all_uses(self, old: Value, new: Value) -> None:
        """Every reader of ``old``, graph outputs included, reads ``new`` instead."""
        if old is new:
            return
        readers, old.users = old.users, []
        for reader in dict.fromkeys(readers):  # a node once, however many slots it has
            for slot, value in enumerate(reader.inputs):
                if value is old:
                    reader.inputs[slot] = new
                    new.users.append(reader)
        self.outputs = [new if v is old else v for v in self.outputs]

    def add_output(self, value: Value, name: str | None = None) -> None:
        self.outputs.append(value)
        self.output_names.append(name or value.name)

    def named_outputs(self) -> list[tuple[str, Value]]:
        names = self.output_names or [v.name for v in self.outputs]
        if len(names) != len(self.outputs):
            raise GraphError("output names and outputs differ in length")
        return list(zip(names, self.outputs))

    # -- queries -------------------------------------------------------------------------------
    def values(self) -> Iterator[Value]:
        """Graph inputs, values the nodes read, values they write, graph outputs; each once."""
        ordered: dict[int, Value] = {}
        for value in self.inputs:
            ordered.setdefault(id(value), value)
        for node in self.nodes:
            for value in node.inputs:
                if value is not None:
                    ordered.setdefault(id(value), value)
        for node in self.nodes:
            for value in node.outputs:
                ordered.setdefault(id(value), value)
        for value in self.outputs:
            ordered.setdefault(id(value), value)
        return iter(list(ordered.values()))

    def constants(self) -> list[Value]:
        return [v for v in self.values() if v.is_constant]

    def op_counts(self) -> dict[str, int]:
        """Operator histogram, most frequent first, ties by name."""
        counts: dict[str, int] = {}
        for node in self.nodes:
            counts[node.op] = counts.get(node.op, 0) + 1
        return {op: counts[op] for op in sorted(counts, key=lambda op: (-counts[op], op))}

    def constant_bytes(self) -> int:
        return sum(int(v.data.nbytes) for v in self.constants())

    # -- order and checks ----------------------------------------------------------------------
    def topological_sort(self) -> None:
        """Reorder the nodes so that producers come before readers; among the nodes whose
        inputs are all available, the one earliest in the current order goes next, so an order
        that is already valid is kept unchanged."""
        index = {id(n): i for i, n in enumerate(self.nodes)}
        successors: list[set[int]] = [set() for _ in self.nodes]
        waiting = [0] * len(self.nodes)
        for i, node in enumerate(self.nodes):
            producers = {index[id(v.producer)] for v in node.inputs
                         if v is not None and v.producer is not None and id(v.producer) in index}
            waiting[i] = len(producers)
            for p in producers:
                successors[p].add(i)
        ready = [i for i, count in enumerate(waiting) if count == 0]
        heapq.heapify(ready)
        order: list[int] = []
        while ready:
            i = heapq.heappop(ready)
            order.append(i)
            for j in successors[i]:
                waiting[j] -= 1
                if waiting[j] == 0:
                    heapq.heappush(ready, j)
        if len(order) != len(self.nodes):
            raise GraphError("graph has a cycle")
        self.nodes = [self.nodes[i] for i in order]

    def verify(self) -> None:
        """Raise GraphError unless the graph is in SSA form, ordered, and its use lists agree."""
        available = {id(v) for v in self.inputs}
        for node in self.nodes:
            for value in node.inputs:
                if value is None:
                    continue
                if not (value.is_constant or id(value) in available):
                    raise GraphError(f"{node.op} {node.name!r} uses undefined {value.name!r}")
                if node not in value.users:
                    raise GraphError(f"use list of {value.name!r} misses {node.name!r}")
            for value in node.outputs:
                if id(value) in available:
                    raise GraphError(f"value {value.name!r} is defined twice")
                if value.producer is not node:
                    raise GraphError(f"producer of {value.name!r} is wrong")
                available.add(id(value))
        present = {id(n) for n in self.nodes}
        for value in self.values():
            stale = next((u for u in value.users if id(u) not in present), None)
            if stale is not None:
                raise GraphError(f"{value.name!r} lists removed user {stale.name!r}")
        for value in self.outputs:
            if not value.is_constant and id(value) not in available:
                raise GraphError(f"graph output {value.name!r} is undefined")

    def summary(self) -> dict[str, Any]:
        return {
            "name": self.name,
            "nodes": len(self.nodes),
            "inputs": {v.name: str(v.type) for v in self.inputs},
            "outputs": {n: str(v.type) for n, v in self.named_outputs()},
            "constants": len(self.constants()),
            "constant_bytes": self.constant_bytes(),
            "ops": self.op_counts(),
        }

    def __str__(self) -> str:
        body = [f"  {v.name}: {v.type}," for v in self.inputs]
        body.append(") {")
        body += [f"  {n!r}  -> {', '.join(str(o.type) for o in n.outputs)}" for n in self.nodes]
        body.append("  return " + ", ".join(f"{k}={v.name}" for k, v in self.named_outputs()))
        return "\n".join([f"graph {self.name}(", *body, "}"])


def _drop_use(value: Value | None, node: Node) -> None:
    if value is not None:
        value.users.remove(node)


def comment_text(text: str) -> str:
    """Model-supplied text made safe inside a generated C/C++ comment: non-printable
    characters become spaces and comment delimiters are broken apart."""
    safe = "".join(ch if ch.isprintable() else " " for ch in text)
    return safe.replace("*/", "* /").replace("/*", "/ *")
