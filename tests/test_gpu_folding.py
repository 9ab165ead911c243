"""Transposes folded into MatMul operands (codegen/folding.py) against the oracle.

Each graph is compiled with folding on and off; both must match the oracle, and the folded
build must have emitted no kernel for the folded Transposes. The CPU tests check the safety
rule on plans where a later node reuses the transposed tensor's memory.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip, f32
from ml_graph_compiler import builders
from ml_graph_compiler.codegen import hip as hip_codegen
from ml_graph_compiler.codegen.folding import plan_folds
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.memory import plan_memory
from ml_graph_compiler.passes import optimize
from ml_graph_compiler.schedule import schedule
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle


def chain(a_shape, a_perm, b_shape, b_perm, out_perm=None):
    """MatMul(Transpose(a, a_perm), Transpose(b, b_perm)), optionally transposed after."""
    g = Graph("fold")
    feeds = {"a": f32(*a_shape), "b": f32(*b_shape)}
    a = g.add_input("a", TensorType("float32", a_shape))
    b = g.add_input("b", TensorType("float32", b_shape))
    if a_perm is not None:
        a = g.add_node("Transpose", [a], 1, {"perm": a_perm}, name="ta", output_names=["ta"]).output
    if b_perm is not None:
        b = g.add_node("Transpose", [b], 1, {"perm": b_perm}, name="tb", output_names=["tb"]).output
    y = g.add_node("MatMul", [a, b], 1, {}, name="mm", output_names=["mm"]).output
    if out_perm is not None:
        y = g.add_node("Transpose", [y], 1, {"perm": out_perm}, name="to", output_names=["to"]).output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, feeds


CASES = {
    "head_split_a": ((2, 7, 3, 16), [0, 2, 1, 3], (2, 3, 16, 9), None, None, 1),
    "k_transposed_b": ((2, 3, 7, 16), None, (2, 9, 3, 16), [0, 2, 3, 1], None, 1),
    "both_and_merge": ((2, 7, 3, 16), [0, 2, 1, 3], (2, 9, 3, 16), [0, 2, 3, 1], [0, 2, 1, 3], 3),
    "matrix_transposes": ((24, 10), [1, 0], (33, 24), [1, 0], None, 2),  # A with column stride != 1
    "broadcast_batch": ((5, 12), None, (4, 5, 12), [0, 2, 1], None, 1),
    "merge_only": ((2, 3, 7, 16), None, (2, 3, 16, 8), None, [0, 2, 1, 3], 1),
    "last_axis_moves": ((3, 7, 16), None, (3, 16, 8), None, [0, 2, 1], 0),  # stays a copy
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_folded_matmul_matches_oracle(name, hip_cache, monkeypatch):
    a_shape, a_perm, b_shape, b_perm, out_perm, n_folded = CASES[name]
    g, feeds = chain(a_shape, a_perm, b_shape, b_perm, out_perm)
    want = oracle.run_graph(g, feeds)["y"]
    for fold in (True, False):
        monkeypatch.setattr(hip_codegen, "FOLD_TRANSPOSES", fold)
        model = compile_hip(chain(a_shape, a_perm, b_shape, b_perm, out_perm)[0], hip_cache, "O0")
        try:
            got = model.run(feeds)["y"]
            kernels = dict(model.report.kernels)
        finally:
            model.release()
        assert kernels.get("folded", 0) == (n_folded if fold else 0), kernels
        assert float(np.max(np.abs(got.astype(np.float64) - want))) <= 1e-5 * max(1.0, float(np.abs(want).max()))


@pytest.mark.gpu
@pytest.mark.parametrize("sample", ["tiny-bert", "tiny-gpt"])
def test_unfused_attention_with_folds(sample, hip_cache, monkeypatch):
    """With attention fusion off, the head-split and head-merge transposes fold into the
    batched MatMuls of QK^T and PV."""
    monkeypatch.setattr(hip_codegen, "FUSE_ATTENTION", False)
    build = builders.SAMPLES[sample]
    feeds = oracle.random_feeds(build(), 2, int_high=50)
    expected = oracle.run_graph(build(), feeds)
    model = compile_hip(build(), hip_cache)
    try:
        got = model.run(feeds)
        assert model.report.kernels.get("folded", 0) >= 4
    finally:
        model.release()
    for name, want in expected.items():
        assert float(np.max(np.abs(got[name].astype(np.float64) - want))) <= 5e-5


def _reuse_graph():
    """x -> Transpose -> MatMul, with a same-sized tensor computed in between from another
    input: once the Transpose has read x, the planner may hand x's memory to that tensor."""
    g = Graph("reuse")
    x0 = g.add_input("x0", TensorType("float32", (32, 32)))
    w = g.add_input("w", TensorType("float32", (32, 32)))
    x = g.add_node("Relu", [x0], 1, {}, name="x", output_names=["x"]).output
    t = g.add_node("Transpose", [x], 1, {"perm": [1, 0]}, name="t", output_names=["t"]).output
    e = g.add_node("Sigmoid", [w], 1, {}, name="e", output_names=["e"]).output
    y = g.add_node("MatMul", [t, e], 1, {}, name="mm", output_names=["mm"]).output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, {"x0": f32(32, 32), "w": f32(32, 32)}


def test_fold_respects_memory_reuse():
    """CPU: the fold is taken exactly when the plan leaves x untouched until the MatMul."""
    g, _ = _reuse_graph()
    plan = plan_memory(g, alignment=256)
    x = next(n for n in g.nodes if n.name == "x").output
    e = next(n for n in g.nodes if n.name == "e").output
    reused = plan.location(x).index == plan.location(e).index
    folds = plan_folds(g, plan, lambda n: 0, set())
    assert (len(folds.inputs) == 0) == reused
    # a plan without reuse (naive) always allows the fold
    assert len(plan_folds(g, plan_memory(g, "naive", alignment=256), lambda n: 0, set()).inputs) == 1


@pytest.mark.gpu
def test_reuse_graph_matches_oracle(hip_cache):
    g, feeds = _reuse_graph()
    want = oracle.run_graph(g, feeds)["y"]
    model = compile_hip(_reuse_graph()[0], hip_cache, "O0")
    try:
        got = model.run(feeds)["y"]
    finally:
        model.release()
    assert float(np.max(np.abs(got.astype(np.float64) - want))) <= 1e-4
