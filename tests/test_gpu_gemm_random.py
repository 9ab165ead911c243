"""Seeded random GEMM shapes through the hip MatMul / FusedGemm lowering against float64 numpy:
odd and aligned M, N, K (K from 1 to beyond the split-K threshold), constant (packed, DMA
kernel) and runtime right-hand sides, bias and ReLU epilogues, and batched operands — the tile
choice (64 x 64, 128 x 32, split-K with its reduction) changes across these shapes."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.shape_inference import infer_shapes

pytestmark = pytest.mark.gpu


def _cases(n: int, seed: int = 2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kind = i % 4
        m = int(rng.choice([1, 3, 17, 64, 100, 129, 333, 512, 700]))
        nn = int(rng.choice([1, 5, 16, 24, 32, 40, 64, 96, 130, 256, 384, 777]))
        k = int(rng.choice([1, 2, 7, 16, 20, 32, 33, 96, 256, 513, 1024, 2048, 2600]))
        batch = () if kind < 3 else (int(rng.integers(1, 4)),)
        out.append((i, batch, m, nn, k, kind))
    return out


def _graph(batch, m, n, k, kind, rng):
    g = Graph("rand_gemm")
    x = g.add_input("x", TensorType("float32", (*batch, m, k)))
    feeds = {"x": rng.standard_normal((*batch, m, k)).astype(np.float32)}
    if kind == 1:  # runtime right-hand side
        w = g.add_input("w", TensorType("float32", (*batch, k, n)))
        feeds["w"] = (rng.standard_normal((*batch, k, n)) / np.sqrt(k)).astype(np.float32)
    else:
        w = g.constant((rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32), "w")
    y = g.add_node("MatMul", [x, w], 1, {}, name="mm").output
    if kind in (2, 3):  # bias + ReLU: a FusedGemm epilogue at O3
        b = g.constant(rng.standard_normal(n).astype(np.float32), "b")
        y = g.add_node("Add", [y, b], 1, {}, name="bias").output
        y = g.add_node("Relu", [y], 1, {}, name="relu").output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, feeds


def _reference(feeds, g, kind):
    x = feeds["x"].astype(np.float64)
    w = feeds["w"].astype(np.float64) if kind == 1 else next(v for v in g.values() if v.name == "w").data.astype(np.float64)
    y = x @ w
    if kind in (2, 3):
        y = np.maximum(y + next(v for v in g.values() if v.name == "b").data.astype(np.float64), 0.0)
    return y


@pytest.mark.parametrize("case", _cases(32), ids=lambda c: f"{c[0]}-b{c[1]}-{c[2]}x{c[3]}x{c[4]}-k{c[5]}")
def test_random_gemm(case, hip_cache):
    i, batch, m, n, k, kind = case
    rng = np.random.default_rng(1000 + i)
    g, feeds = _graph(batch, m, n, k, kind, rng)
    want = _reference(feeds, g, kind)
    model = compile_hip(g, hip_cache, "O3")
    try:
        got = model.run(feeds)["y"].astype(np.float64)
    finally:
        model.release()
    err = float(np.max(np.abs(got - want))) if want.size else 0.0
    assert err <= 2e-5 * max(1.0, float(np.abs(want).max()) if want.size else 1.0), (case, err)
