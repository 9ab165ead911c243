"""IR invariants (the reference's tests/test_ir.py, restated on IR-built graphs)."""

from __future__ import annotations

import numpy as np
import pytest

from ml_graph_compiler.errors import GraphError
from ml_graph_compiler.ir import Graph, TensorType, comment_text, dtype_name, numpy_dtype

F = TensorType("float32", (4,))


def chain():
    g = Graph("t")
    x = g.add_input("x", F)
    a = g.add_node("Relu", [x])
    b = g.add_node("Neg", [a.output])
    g.add_output(b.output, "y")
    for n in g.nodes:
        n.output.type = F
    return g, x, a, b


def test_tensor_type_properties():
    t = TensorType("float32", (2, 3))
    assert t.rank == 2 and t.size == 6 and t.nbytes == 24 and str(t) == "float32[2x3]"
    assert TensorType("int64", ()).size == 1
    with pytest.raises(GraphError):
        TensorType("float32", (-1,))
    with pytest.raises(GraphError):
        TensorType("complex", (1,))
    assert TensorType.of(np.zeros((2, 5), np.int32)) == TensorType("int32", (2, 5))
    assert dtype_name(numpy_dtype("bool")) == "bool"


def test_names_are_unique():
    g = Graph()
    a = g.add_input("x", F)
    b = g.add_input("x", F)
    assert a.name != b.name
    assert g.fresh_name("v") != g.fresh_name("v")


def test_use_lists_and_replace():
    g, x, a, b = chain()
    assert a in x.users and b in a.output.users
    g.verify()
    c = g.add_node("Abs", [x], index=1)
    c.output.type = F
    g.replace_all_uses(a.output, c.output)
    assert b.inputs[0] is c.output and not a.output.users
    g.remove_node(a)
    g.verify()
    with pytest.raises(GraphError):
        g.remove_node(b)


def test_replace_updates_graph_outputs():
    g, x, a, b = chain()
    g.replace_all_uses(b.output, a.output)
    assert g.outputs == [a.output]
    assert g.named_outputs() == [("y", a.output)]


def test_topological_sort_is_stable_and_detects_cycles():
    g, x, a, b = chain()
    g.nodes = [b, a]
    g.topological_sort()
    assert g.nodes == [a, b]
    g.set_input(a, 0, b.output)
    with pytest.raises(GraphError, match="cycle"):
        g.topological_sort()


def test_verify_catches_violations():
    g, x, a, b = chain()
    g.nodes = [b, a]
    with pytest.raises(GraphError, match="undefined"):
        g.verify()
    g.nodes = [a, b]
    a.output.users.clear()
    with pytest.raises(GraphError, match="use list"):
        g.verify()


def test_summary_and_text():
    g, x, a, b = chain()
    s = g.summary()
    assert s["nodes"] == 2 and s["ops"] == {"Neg": 1, "Relu": 1}
    assert "return y=" in str(g)


def test_comment_text_neutralizes_comment_ends():
    assert "*/" not in comment_text("a */ b \n c")
    assert "\n" not in comment_text("x\ny")
