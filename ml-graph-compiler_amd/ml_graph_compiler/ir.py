"""SSA graph IR with static shapes (reference: src/ml_graph_compiler/ir.py:1-396).

Each Value is defined once: as a graph input, as a constant (it carries ``data``), or as one
output of one Node. Nodes hold their input Values (None for an omitted optional ONNX input)
and every Value keeps the list of Nodes that read it, so rewrites never rebuild an index.
The behaviour that other stages depend on is kept exactly: the naming counter, the order of
``values()`` (inputs, node inputs, node outputs, graph outputs), the stable heap-based
``topological_sort`` and the checks of ``verify``.
"""

from __future__ import annotations

import heapq
import itertools
from collections.abc import Iterable, Iterator
from dataclasses import dataclass
from typing import Any

import numpy as np

from .errors import GraphError

_DTYPES: dict[str, np.dtype] = {
    name: np.dtype(t)
    for name, t in (
        ("float32", np.float32),
        ("float64", np.float64),
        ("float16", np.float16),
        ("int64", np.int64),
        ("int32", np.int32),
        ("int8", np.int8),
        ("uint8", np.uint8),
        ("bool", np.bool_),
    )
}


def contiguous(array: Any, dtype: Any = None) -> np.ndarray:
    """C-ordered ndarray view/copy of ``array``; zero-dimensional arrays stay zero-dimensional."""
    return np.asarray(array, dtype=dtype, order="C")


def numpy_dtype(name: str) -> np.dtype:
    if name not in _DTYPES:
        raise GraphError(f"unsupported dtype {name!r}")
    return _DTYPES[name]


def dtype_name(dtype: Any) -> str:
    wanted = np.dtype(dtype)
    for name, dt in _DTYPES.items():
        if dt == wanted:
            return name
    raise GraphError(f"unsupported numpy dtype {wanted}")


@dataclass(frozen=True)
class TensorType:
    """Element dtype name and static shape."""

    dtype: str
    shape: tuple[int, ...]

    def __post_init__(self) -> None:
        numpy_dtype(self.dtype)
        for d in self.shape:
            if not isinstance(d, int) or d < 0:
                raise GraphError(f"shape must be non-negative integers, got {self.shape}")

    @property
    def rank(self) -> int:
        return len(self.shape)

    @property
    def size(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    @property
    def itemsize(self) -> int:
        return numpy_dtype(self.dtype).itemsize

    @property
    def nbytes(self) -> int:
        return self.size * self.itemsize

    def __str__(self) -> str:
        return f"{self.dtype}[{'x'.join(map(str, self.shape))}]"

    @staticmethod
    def of(array: np.ndarray) -> TensorType:
        return TensorType(dtype_name(array.dtype), tuple(int(d) for d in array.shape))


class Value:
    """One SSA value."""

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
    """One operator application."""

    __slots__ = ("attrs", "inputs", "name", "op", "outputs")

    def __init__(
        self,
        op: str,
        inputs: list[Value | None],
        outputs: list[Value],
        attrs: dict[str, Any] | None = None,
        name: str = "",
    ):
        self.op = op
        self.inputs = inputs
        self.outputs = outputs
        self.attrs: dict[str, Any] = dict(attrs) if attrs else {}
        self.name = name

    def input(self, i: int) -> Value:
        v = self.inputs[i] if i < len(self.inputs) else None
        if v is None:
            raise GraphError(f"{self.op} node {self.name!r} is missing input {i}")
        return v

    def optional_input(self, i: int) -> Value | None:
        return self.inputs[i] if i < len(self.inputs) else None

    @property
    def output(self) -> Value:
        return self.outputs[0]

    def __repr__(self) -> str:
        args = ", ".join("_" if v is None else v.name for v in self.inputs)
        res = ", ".join(v.name for v in self.outputs)
        text = f"{res} = {self.op}({args})"
        return f"{text} {self.attrs}" if self.attrs else text


class Graph:
    """Ordered nodes plus graph inputs, outputs (with fixed public names) and constants."""

    def __init__(self, name: str = "graph"):
        self.name = name
        self.opset = 17
        self.inputs: list[Value] = []
        self.outputs: list[Value] = []
        self.output_names: list[str] = []
        self.nodes: list[Node] = []
        self._names: set[str] = set()
        self._counter = itertools.count()

    # -- names ---------------------------------------------------------------------------------
    def fresh_name(self, hint: str = "v") -> str:
        while True:
            candidate = f"{hint}_{next(self._counter)}"
            if candidate not in self._names:
                self._names.add(candidate)
                return candidate

    def _claim(self, name: str) -> str:
        if name and name not in self._names:
            self._names.add(name)
            return name
        return self.fresh_name(name or "v")

    # -- building ------------------------------------------------------------------------------
    def add_input(self, name: str, type: TensorType) -> Value:
        v = Value(self._claim(name), type)
        self.inputs.append(v)
        return v

    def constant(self, array: np.ndarray, name: str = "const") -> Value:
        data = contiguous(array)
        return Value(self._claim(name), TensorType.of(data), data)

    def add_node(
        self,
        op: str,
        inputs: list[Value | None],
        n_outputs: int = 1,
        attrs: dict[str, Any] | None = None,
        name: str = "",
        output_names: list[str] | None = None,
        index: int | None = None,
    ) -> Node:
        if output_names:
            names = list(output_names)
        else:
            names = [f"{name or op.lower()}_out"] * n_outputs
        outs = [Value(self._claim(n)) for n in names]
        node = Node(op, list(inputs), outs, attrs, name or self.fresh_name(op.lower()))
        for v in outs:
            v.producer = node
        for v in inputs:
            if v is not None:
                v.users.append(node)
        if index is None:
            self.nodes.append(node)
        else:
            self.nodes.insert(index, node)
        return node

    # -- rewriting -----------------------------------------------------------------------------
    def set_input(self, node: Node, i: int, value: Value | None) -> None:
        previous = node.inputs[i]
        if previous is not None:
            previous.users.remove(node)
        node.inputs[i] = value
        if value is not None:
            value.users.append(node)

    def remove_node(self, node: Node) -> None:
        if any(o.users or o in self.outputs for o in node.outputs):
            raise GraphError(f"cannot remove {node.op} {node.name!r}: output still used")
        for v in node.inputs:
            if v is not None:
                v.users.remove(node)
        self.nodes.remove(node)

    def remove_nodes(self, dead: Iterable[Node]) -> int:
        doomed = set(dead)
        if not doomed:
            return 0
        for node in doomed:
            for v in node.inputs:
                if v is not None and node in v.users:
                    v.users.remove(node)
        self.nodes = [n for n in self.nodes if n not in doomed]
        return len(doomed)

    def replace_all_uses(self, old: Value, new: Value) -> None:
        if old is new:
            return
        for user in list(old.users):
            for i, v in enumerate(user.inputs):
                if v is old:
                    user.inputs[i] = new
                    new.users.append(user)
        old.users = []
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
        seen: set[int] = set()
        ordered = itertools.chain(
            self.inputs,
            (v for n in self.nodes for v in n.inputs if v is not None),
            (v for n in self.nodes for v in n.outputs),
            self.outputs,
        )
        for v in ordered:
            if id(v) not in seen:
                seen.add(id(v))
                yield v

    def constants(self) -> list[Value]:
        return [v for v in self.values() if v.is_constant]

    def op_counts(self) -> dict[str, int]:
        counts: dict[str, int] = {}
        for n in self.nodes:
            counts[n.op] = counts.get(n.op, 0) + 1
        return dict(sorted(counts.items(), key=lambda kv: (-kv[1], kv[0])))

    def constant_bytes(self) -> int:
        return sum(v.data.nbytes for v in self.constants() if v.data is not None)

    # -- order and checks ----------------------------------------------------------------------
    def topological_sort(self) -> None:
        """Stable topological order: among ready nodes the earliest current position runs first."""
        pos = {id(n): i for i, n in enumerate(self.nodes)}
        pending: dict[int, int] = {}
        for n in self.nodes:
            preds = {
                id(v.producer)
                for v in n.inputs
                if v is not None and v.producer is not None and id(v.producer) in pos
            }
            pending[id(n)] = len(preds)
        heap = [(pos[id(n)], n) for n in self.nodes if pending[id(n)] == 0]
        heapq.heapify(heap)
        order: list[Node] = []
        while heap:
            _, n = heapq.heappop(heap)
            order.append(n)
            done: set[int] = set()
            for out in n.outputs:
                for user in out.users:
                    if id(user) in done or id(user) not in pending:
                        continue
                    if any(v is not None and v.producer is n for v in user.inputs):
                        done.add(id(user))
                        pending[id(user)] -= 1
                        if pending[id(user)] == 0:
                            heapq.heappush(heap, (pos[id(user)], user))
        if len(order) != len(self.nodes):
            raise GraphError("graph has a cycle")
        self.nodes = order

    def verify(self) -> None:
        defined = {id(v) for v in self.inputs}
        produced: set[int] = set()
        for n in self.nodes:
            for v in n.inputs:
                if v is None:
                    continue
                if not v.is_constant and id(v) not in defined:
                    raise GraphError(f"{n.op} {n.name!r} uses undefined {v.name!r}")
                if n not in v.users:
                    raise GraphError(f"use list of {v.name!r} misses {n.name!r}")
            for out in n.outputs:
                if id(out) in produced or id(out) in defined:
                    raise GraphError(f"value {out.name!r} is defined twice")
                if out.producer is not n:
                    raise GraphError(f"producer of {out.name!r} is wrong")
                produced.add(id(out))
                defined.add(id(out))
        alive = {id(n) for n in self.nodes}
        for v in self.values():
            for user in v.users:
                if id(user) not in alive:
                    raise GraphError(f"{v.name!r} lists removed user {user.name!r}")
        for v in self.outputs:
            if not v.is_constant and id(v) not in defined:
                raise GraphError(f"graph output {v.name!r} is undefined")

    def summary(self) -> dict[str, Any]:
        return {
            "name": self.name,
            "nodes": len(self.nodes),
            "inputs": {v.name: str(v.type) for v in self.inputs},
            "outputs": {name: str(v.type) for name, v in self.named_outputs()},
            "constants": len(self.constants()),
            "constant_bytes": self.constant_bytes(),
            "ops": self.op_counts(),
        }

    def __str__(self) -> str:
        lines = [f"graph {self.name}("]
        lines.extend(f"  {v.name}: {v.type}," for v in self.inputs)
        lines.append(") {")
        for n in self.nodes:
            lines.append(f"  {n!r}  -> {', '.join(str(o.type) for o in n.outputs)}")
        lines.append("  return " + ", ".join(f"{k}={v.name}" for k, v in self.named_outputs()))
        lines.append("}")
        return "\n".join(lines)


def comment_text(text: str) -> str:
    """Model-supplied text made safe inside a C/C++ comment: no line breaks, no comment ends."""
    printable = "".join(c if c.isprintable() else " " for c in text)
    return printable.replace("*/", "* /").replace("/*", "/ *")
