"""Static memory planner and scheduler: the reference's known answers and properties
(tests/test_memory_schedule.py of the reference, on IR-built graphs)."""

from __future__ import annotations

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from ml_graph_compiler import builders
from ml_graph_compiler.errors import GraphError
from ml_graph_compiler.ir import Graph, TensorType, Value
from ml_graph_compiler.memory import STRATEGIES, Buffer, Location, plan_memory
from ml_graph_compiler.passes import fuse_elementwise, optimize
from ml_graph_compiler.schedule import (
    apply_order,
    critical_path_flops,
    memory_aware_order,
    peak_live_bytes,
    schedule,
    wavefronts,
)
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle

F = TensorType("float32", (256,))  # 1 KiB


def chain_graph(n: int, op: str = "Relu") -> Graph:
    g = Graph()
    v = g.add_input("x", F)
    for _ in range(n):
        node = g.add_node(op, [v])
        node.output.type = F
        v = node.output
    g.add_output(v, "y")
    return g


def test_chain_without_inplace_needs_two_buffers():
    g = chain_graph(6)
    plan = plan_memory(g, inplace=False)
    assert plan.arena_bytes == 2 * 1024
    assert plan.naive_bytes == 5 * 1024
    assert plan.lower_bound == 2 * 1024
    assert plan.location(g.outputs[0]) == Location("output", 0)
    assert plan.location(g.inputs[0]) == Location("input", 0)


def test_chain_inplace_writes_everything_into_the_output():
    g = chain_graph(6)
    plan = plan_memory(g)
    assert plan.inplace == 5
    assert plan.arena_bytes == 0
    assert all(plan.location(n.output).kind == "output" for n in g.nodes)


def test_views_alias_their_input():
    g = Graph()
    x = g.add_input("x", TensorType("float32", (4, 8)))
    a = g.add_node("Relu", [x])
    b = g.add_node("Reshape", [a.output, g.constant(np.asarray([8, 4], np.int64))])
    c = g.add_node("Flatten", [b.output], attrs={"axis": 0})
    y = g.add_node("Neg", [c.output])
    g.add_output(y.output, "y")
    infer_shapes(g)
    plan = plan_memory(g, inplace=False)
    assert plan.offset(a.output) == plan.offset(b.output) == plan.offset(c.output)
    assert plan.aliases == 2
    g2 = Graph()
    x2 = g2.add_input("x", TensorType("float32", (4, 8)))
    r = g2.add_node("Reshape", [x2, g2.constant(np.asarray([8, 4], np.int64))])
    g2.add_output(r.output, "y")
    infer_shapes(g2)
    plan = plan_memory(g2)
    assert plan.location(g2.outputs[0]) == Location("input", 0)
    assert len(plan.copies) == 1 and plan.copies[0][1] == 0


def test_view_of_constant_and_constant_output():
    g = Graph()
    c = g.constant(np.ones((2, 2), np.float32), "c")
    node = g.add_node("Reshape", [c], attrs={"shape": [4]})
    node.output.type = TensorType("float32", (4,))
    g.add_output(node.output, "y")
    g.add_output(c, "c_out")
    plan = plan_memory(g)
    assert plan.location(node.output) == Location("const")
    assert plan.location(c) == Location("const")
    assert [j for _, j in plan.copies] == [0, 1]


def test_same_value_twice_as_output_is_copied():
    g = chain_graph(2)
    g.add_output(g.outputs[0], "again")
    assert [j for _, j in plan_memory(g).copies] == [1]


def test_inplace_requires_same_shape_and_death():
    g = Graph()
    x = g.add_input("x", TensorType("float32", (4, 1)))
    bv = g.add_input("b", TensorType("float32", (4, 8)))
    a = g.add_node("Relu", [x])
    c = g.add_node("Add", [a.output, bv])
    d = g.add_node("Neg", [c.output])
    c2 = g.add_node("Relu", [c.output])
    y = g.add_node("Add", [d.output, c2.output])
    g.add_output(y.output, "y")
    infer_shapes(g)
    plan = plan_memory(g)
    plan.verify()
    assert plan.location(c.output) != plan.location(a.output)
    assert plan.location(d.output) != plan.location(c.output)
    assert plan.location(c2.output) == plan.location(c.output)
    assert plan.inplace == 2


def test_workspace_buffers():
    g = chain_graph(3)
    plan = plan_memory(g, inplace=False, workspace=lambda n: 100 if n is g.nodes[1] else 0)
    assert id(g.nodes[1]) in plan.workspaces
    assert plan.workspaces[id(g.nodes[1])] % 64 == 0
    assert plan.arena_bytes >= 1024 + 128


def test_unknown_strategy_and_missing_location():
    g = chain_graph(2)
    with pytest.raises(GraphError):
        plan_memory(g, strategy="best")  # type: ignore[arg-type]
    plan = plan_memory(g)
    with pytest.raises(GraphError):
        plan.location(Value("ghost", F))
    with pytest.raises(GraphError):
        plan.offset(g.inputs[0])


def test_verify_catches_overlap():
    g = chain_graph(4)
    plan = plan_memory(g, inplace=False)
    plan.buffers.append(Buffer(99, 1024, 0, 10, offset=plan.buffers[0].offset))
    with pytest.raises(GraphError, match="overlap"):
        plan.verify()
    plan.buffers[-1] = Buffer(99, 1024, 50, 60, offset=8)
    with pytest.raises(GraphError, match="misaligned"):
        plan.verify()
    plan.buffers[-1] = Buffer(99, 1024, 50, 60, offset=10**6)
    with pytest.raises(GraphError, match="exceeds"):
        plan.verify()


@pytest.mark.parametrize("name", sorted(builders.SAMPLES))
@pytest.mark.parametrize("strategy", STRATEGIES)
def test_plans_are_valid_on_samples(name, strategy):
    g = builders.SAMPLES[name]()
    optimize(g, "O3")
    plan = plan_memory(g, strategy=strategy, alignment=256)
    plan.verify()
    assert plan.lower_bound <= plan.arena_bytes <= plan.naive_bytes
    assert all(o % 256 == 0 for o in (b.offset for b in plan.buffers))


@st.composite
def random_dags(draw):
    g = Graph()
    values = [g.add_input("x", TensorType("float32", (draw(st.integers(1, 64)),)))]
    for _ in range(draw(st.integers(1, 25))):
        size = draw(st.integers(1, 512))
        k = draw(st.integers(1, min(3, len(values))))
        ins = draw(st.lists(st.sampled_from(values), min_size=k, max_size=k))
        node = g.add_node("Concat", list(ins), attrs={"axis": 0})
        node.output.type = TensorType("float32", (size,))
        values.append(node.output)
    for v in draw(st.lists(st.sampled_from(values[1:]), min_size=1, max_size=3, unique_by=id)):
        g.add_output(v)
    return g


@given(random_dags(), st.sampled_from(STRATEGIES), st.sampled_from([16, 64, 256]))
@settings(max_examples=80, deadline=None)
def test_random_plans_never_overlap(g, strategy, alignment):
    plan = plan_memory(g, strategy=strategy, alignment=alignment)
    plan.verify()
    assert plan.lower_bound <= plan.arena_bytes <= plan.naive_bytes
    for i, a in enumerate(plan.buffers):
        for b in plan.buffers[i + 1 :]:
            if a.overlaps_in_time(b):
                assert a.offset + a.size <= b.offset or b.offset + b.size <= a.offset


@given(random_dags())
@settings(max_examples=40, deadline=None)
def test_greedy_by_size_is_never_worse_than_naive(g):
    assert plan_memory(g, "greedy_by_size").arena_bytes <= plan_memory(g, "naive").arena_bytes


def fan_graph() -> Graph:
    g = Graph()
    x = g.add_input("x", TensorType("float32", (8,)))
    big, small = TensorType("float32", (4096,)), TensorType("float32", (8,))
    a1 = g.add_node("Expand", [x])
    a1.output.type = big
    b1 = g.add_node("Expand", [x])
    b1.output.type = big
    a2 = g.add_node("ReduceSum", [a1.output])
    a2.output.type = small
    b2 = g.add_node("ReduceSum", [b1.output])
    b2.output.type = small
    out = g.add_node("Add", [a2.output, b2.output])
    out.output.type = small
    g.add_output(out.output)
    return g


def test_memory_aware_order_reduces_peak():
    g = fan_graph()
    before = peak_live_bytes(g)
    after = peak_live_bytes(g, memory_aware_order(g))
    assert after < before and before == 2 * 16384 + 32
    report = schedule(g)
    assert report.peak_after == after and report.peak_before == before
    g.verify()
    assert schedule(g).peak_after == after


def test_schedule_keeps_order_when_no_gain():
    g = chain_graph(4)
    before = list(g.nodes)
    report = schedule(g)
    assert g.nodes == before and report.peak_after == report.peak_before


def test_apply_order_rejects_bad_orders():
    g = chain_graph(3)
    with pytest.raises(GraphError, match="permutation"):
        apply_order(g, g.nodes[:2])
    with pytest.raises(GraphError):
        apply_order(g, list(reversed(g.nodes)))
    g.verify()


def test_cycle_detection():
    g = chain_graph(2)
    g.set_input(g.nodes[0], 0, g.nodes[1].output)
    with pytest.raises(GraphError, match="cycle"):
        memory_aware_order(g)


def test_wavefronts_and_critical_path():
    g = fan_graph()
    assert [len(lv) for lv in wavefronts(g)] == [2, 2, 1]
    crit, total = critical_path_flops(g)
    assert total == 4096 * 2 + 8 * 2 + 8 and crit == 4096 + 8 + 8
    assert critical_path_flops(Graph()) == (0, 0)


@given(random_dags())
@settings(max_examples=40, deadline=None)
def test_memory_aware_order_is_topological(g):
    seen: set[int] = set()
    order = memory_aware_order(g)
    for node in order:
        for v in node.inputs:
            if v is not None and v.producer is not None:
                assert id(v.producer) in seen
        seen.add(id(node))
    assert len(order) == len(g.nodes)


def test_loop_fusion_builds_one_program():
    g = Graph()
    x = g.add_input("x", TensorType("float32", (2, 4, 4)))
    m = g.add_input("m", TensorType("float32", (1, 4, 4)))
    a = g.add_node("Mul", [x, g.constant(np.asarray(0.5, np.float32))])
    b = g.add_node("Add", [a.output, m])
    c = g.add_node("Clip", [b.output, None, g.constant(np.asarray(1.0, np.float32))])
    y = g.add_node("Softmax", [c.output], attrs={"axis": -1})
    g.add_output(y.output, "y")
    infer_shapes(g)
    feeds = oracle.random_feeds(g)
    expected = oracle.run_graph(g, feeds)["y"]
    assert fuse_elementwise(g) == 1
    assert g.op_counts() == {"FusedElementwise": 1, "Softmax": 1}
    program = g.nodes[0].attrs["program"]
    assert [p[0] for p in program] == ["Mul", "Add", "Clip"]
    assert -1 in program[2][2]
    np.testing.assert_allclose(oracle.run_graph(g, feeds)["y"], expected, rtol=1e-6)
    assert fuse_elementwise(g) == 0
