"""The compiled-model surface of the hip backend, ported from the reference's backend tests.

* Every planner strategy, with and without in-place reuse, gives bit-identical outputs
  (reference tests/test_codegen.py:416-432).
* save / load / profile / benchmark round trip, and a cached rebuild (:578-600).
* Graph outputs that are views of inputs, or constants, are copied into the output buffers
  (:602-613).
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import f32
from ml_graph_compiler import builders
from ml_graph_compiler.codegen import compile_graph
from ml_graph_compiler.codegen.runtime_lib import HipCompiledModel
from ml_graph_compiler.errors import CodegenError
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.memory import STRATEGIES
from ml_graph_compiler.passes import optimize
from ml_graph_compiler.schedule import schedule
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu


def _compiled(make, cache, **kw):
    g = make()
    optimize(g, "O3")
    schedule(g)
    return compile_graph(g, cache_dir=cache, **kw)


@pytest.mark.parametrize("make", [lambda: builders.transformer(gelu="tanh", causal=True), builders.tiny_cnn],
                         ids=["tiny_transformer", "tiny_cnn"])
@pytest.mark.parametrize("strategy", STRATEGIES)
@pytest.mark.parametrize("inplace", [True, False])
def test_memory_plans_give_identical_results(make, strategy, inplace, hip_cache):
    print(f"[gpu] memory plan {strategy} inplace={inplace}", flush=True)
    feeds = oracle.random_feeds(make(), 2)
    base = _compiled(make, hip_cache)
    try:
        reference = base.run(feeds)
    finally:
        base.release()
    model = _compiled(make, hip_cache, strategy=strategy, inplace=inplace)
    try:
        got = model.run(feeds)
        assert model.report.plan["strategy"] == strategy
    finally:
        model.release()
    for k in reference:
        np.testing.assert_array_equal(got[k], reference[k])


def test_save_load_and_profile(hip_cache, tmp_path):
    print("[gpu] save/load/profile", flush=True)
    graph = builders.tiny_cnn()
    feeds = oracle.random_feeds(graph, 7)
    expected = oracle.run_graph(builders.tiny_cnn(), feeds)["logits"]
    optimize(graph, "O3")
    schedule(graph)
    compiled = compile_graph(graph, cache_dir=hip_cache, profile=True)
    first = compiled.run(feeds)
    np.testing.assert_allclose(first["logits"], expected, rtol=1e-4, atol=2e-5)
    prof = compiled.profile()
    assert len(prof) == len(graph.nodes) and all(t >= 0 for _, _, t in prof)
    assert [(op, name) for op, name, _ in prof] == [(n.op, n.name) for n in graph.nodes]
    # the tiny CNN's nine GEMMs, its classifier computed in the global pooling's launch
    assert compiled.report is not None and compiled.report.kernels["gemm"] == 8
    assert compiled.report.kernels["pool_fc"] == 1
    compiled.save(tmp_path / "saved")
    compiled.release()
    loaded = HipCompiledModel.load(tmp_path / "saved")
    try:
        np.testing.assert_array_equal(loaded.run(feeds)["logits"], first["logits"])
        assert [(op, name) for op, name, _ in loaded.profile()] == [(op, name) for op, name, _ in prof]
        times = loaded.benchmark(feeds, warmup=1, repeat=3)
        assert len(times) == 3 and all(t > 0 for t in times)
    finally:
        loaded.release()
    plain = compile_graph(graph, cache_dir=hip_cache)
    try:
        with pytest.raises(CodegenError, match="profile"):
            plain.profile()
    finally:
        plain.release()
    # a cached rebuild of the same graph
    again = compile_graph(graph, cache_dir=hip_cache, profile=True)
    try:
        assert again.report is not None and again.report.cached
    finally:
        again.release()


def test_output_that_is_an_input_or_constant_is_copied(hip_cache):
    print("[gpu] input and constant outputs", flush=True)
    g = Graph("copies")
    x = g.add_input("x", TensorType("float32", (2, 3)))
    view = g.add_node("Reshape", [x], attrs={"shape": [3, 2]})
    view.output.type = TensorType("float32", (3, 2))
    g.add_output(view.output, "reshaped")
    g.add_output(g.constant(np.arange(4, dtype=np.float32), "c"), "const")
    g.add_output(x, "same")
    compiled = compile_graph(g, cache_dir=hip_cache)
    try:
        for _ in range(2):   # a second run replays the captured graph
            xv = f32(2, 3)
            out = compiled.run({"x": xv})
            np.testing.assert_array_equal(out["reshaped"], xv.reshape(3, 2))
            np.testing.assert_array_equal(out["const"], np.arange(4, dtype=np.float32))
            np.testing.assert_array_equal(out["same"], xv)
    finally:
        compiled.release()
