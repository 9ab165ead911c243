"""hip backend end to end on the GPU: bundled samples and benchmark configs against the oracle.

Every test compiles with ``backend="hip"`` (the kernels of libmgc_hip.so; there is no CPU
fallback) and compares with the numpy oracle (oracle/interpreter.py) run on the unoptimized
graph with the same seeded inputs.
"""

from __future__ import annotations

import numpy as np
import pytest

from ml_graph_compiler import builders
from ml_graph_compiler.codegen import compile_graph
from ml_graph_compiler.passes import PIPELINES, optimize
from ml_graph_compiler.schedule import schedule
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu


def compile_hip(graph, cache, level="O3", **kw):
    optimize(graph, level)
    schedule(graph)
    return compile_graph(graph, cache_dir=cache, **kw)


@pytest.mark.parametrize("level", ["O0", "O2", "O3"])
@pytest.mark.parametrize("name", sorted(builders.SAMPLES))
def test_samples(name, level, hip_cache):
    print(f"[gpu] sample {name} {level}", flush=True)
    g0 = builders.SAMPLES[name]()
    feeds = oracle.random_feeds(g0, 4, int_high=100)
    expected = oracle.run_graph(g0, feeds)
    model = compile_hip(builders.SAMPLES[name](), hip_cache, level)
    got = model.run(feeds)
    for k, v in expected.items():
        assert got[k].shape == v.shape and got[k].dtype == v.dtype
        np.testing.assert_allclose(got[k], v, rtol=1e-4, atol=2e-5, err_msg=k)
    model.release()


def test_single_gemm(hip_cache):
    """Config 1: [128,768] x [768,3072] + bias, relu; max-abs <= 1e-4 against the oracle."""
    print("[gpu] single_gemm", flush=True)
    g0 = builders.single_gemm()
    feeds = oracle.random_feeds(g0, 0)
    expected = oracle.run_graph(g0, feeds)["y"]
    model = compile_hip(builders.single_gemm(), hip_cache)
    got = model.run(feeds)["y"]
    err = float(np.max(np.abs(got.astype(np.float64) - expected)))
    print(f"[gpu] single_gemm max-abs {err:.3e}", flush=True)
    assert err <= 1e-4
    model.release()


@pytest.mark.parametrize("batch", [1, 2])
def test_bottleneck(batch, hip_cache):
    print(f"[gpu] bottleneck b{batch}", flush=True)
    g0 = builders.bottleneck(batch)
    feeds = oracle.random_feeds(g0, 1)
    expected = oracle.run_graph(g0, feeds)["y"]
    model = compile_hip(builders.bottleneck(batch), hip_cache)
    got = model.run(feeds)["y"]
    err = float(np.max(np.abs(got.astype(np.float64) - expected)))
    print(f"[gpu] bottleneck b{batch} max-abs {err:.3e} max|ref| {np.abs(expected).max():.3e}", flush=True)
    assert err <= 1e-4
    model.release()
