"""Seeded random convolutions (O3: NHWC implicit GEMM, space-to-depth stems, depthwise kernels,
grouped convolutions) with bias, residual and activation epilogues against the oracle."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu


def _cases(n: int, seed: int = 77):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kind = ["dense", "dense", "depthwise", "grouped"][i % 4]
        k = int(rng.choice([1, 3, 3, 5, 7]))
        stride = int(rng.choice([1, 1, 2]))
        dil = int(rng.choice([1, 1, 1, 2])) if k > 1 else 1
        cin = int(rng.choice([1, 3, 4, 8, 12, 16, 24, 32, 64]))
        if kind == "depthwise":
            cin = int(rng.choice([4, 8, 16, 32, 48]))
            cout, group = cin, cin
        elif kind == "grouped":
            group = int(rng.choice([2, 4]))
            cin = group * int(rng.choice([2, 4, 8]))
            cout = group * int(rng.choice([2, 4, 8]))
        else:
            cout, group = int(rng.choice([8, 16, 24, 40, 64, 96])), 1
        hw = (int(rng.integers(5, 30)), int(rng.integers(5, 30)))
        pads = [int(x) for x in rng.integers(0, k // 2 + 1, 4)] if k > 1 else [0, 0, 0, 0]
        act = str(rng.choice(["none", "relu", "clip"]))
        residual = bool(rng.random() < 0.3)
        out.append((i, kind, int(rng.integers(1, 4)), cin, cout, group, hw, k, stride, dil, pads, act, residual))
    return out


def _graph(case):
    i, kind, n, cin, cout, group, (h, w), k, stride, dil, pads, act, residual = case
    rng = np.random.default_rng(500 + i)
    g = Graph("rand_conv")
    x = g.add_input("x", TensorType("float32", (n, cin, h, w)))
    feeds = {"x": rng.standard_normal((n, cin, h, w)).astype(np.float32)}
    wt = g.constant((rng.standard_normal((cout, cin // group, k, k)) * (1.0 / np.sqrt(cin // group * k * k))).astype(np.float32), "w")
    b = g.constant(rng.standard_normal(cout).astype(np.float32) * 0.1, "b")
    attrs = {"kernel_shape": [k, k], "strides": [stride, stride], "pads": pads, "dilations": [dil, dil], "group": group}
    y = g.add_node("Conv", [x, wt, b], 1, attrs, name="conv").output
    infer_shapes(g)
    if residual:
        r = g.add_input("r", TensorType("float32", y.type.shape))
        feeds["r"] = rng.standard_normal(y.type.shape).astype(np.float32)
        y = g.add_node("Add", [y, r], 1, {}, name="res").output
    if act == "relu":
        y = g.add_node("Relu", [y], 1, {}, name="act").output
    elif act == "clip":
        lo = g.constant(np.asarray(0.0, np.float32), "lo")
        hi = g.constant(np.asarray(6.0, np.float32), "hi")
        y = g.add_node("Clip", [y, lo, hi], 1, {}, name="act").output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, feeds


def _valid(case):
    _, _, _, _, _, _, (h, w), k, stride, dil, pads, _, _ = case
    ext = dil * (k - 1) + 1
    return h + pads[0] + pads[2] >= ext and w + pads[1] + pads[3] >= ext


@pytest.mark.parametrize("case", [c for c in _cases(40) if _valid(c)][:32],
                         ids=lambda c: f"{c[0]}-{c[1]}-n{c[2]}c{c[3]}o{c[4]}g{c[5]}-{c[6][0]}x{c[6][1]}-k{c[7]}s{c[8]}d{c[9]}")
def test_random_conv(case, hip_cache):
    g, feeds = _graph(case)
    want = oracle.run_graph(g, feeds)["y"]
    model = compile_hip(_graph(case)[0], hip_cache, "O3")
    try:
        got = model.run(feeds)["y"].astype(np.float64)
    finally:
        model.release()
    err = float(np.max(np.abs(got - want)))
    assert err <= 2e-5 * max(1.0, float(np.abs(want).max())), (case, err)
