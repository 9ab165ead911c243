"""Stride-2 convolutions over few channels run as stride-1 convolutions on a space-to-depth copy
of the input (codegen/hip.py ``_conv_space_to_depth``): every tap of the original kernel must
land on the right sub-pixel and padding must stay zero, for odd and even kernels, symmetric and
asymmetric pads, and inputs read from NCHW (the layout pass's input Transpose folded into the
copy) or from an NHWC tensor.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip
from ml_graph_compiler.codegen import hip as hip_codegen
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.passes import optimize
from ml_graph_compiler.schedule import schedule
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle

def conv_graph(c: int, hw: int, k: int, pads: list[int], kout: int = 16, twice: bool = False):
    """The same weights and input on every call (the graph is built twice: for the oracle and
    for the build, which rewrites it)."""
    rng = np.random.default_rng(11)
    g = Graph("s2d")
    x = g.add_input("x", TensorType("float32", (2, c, hw, hw)))
    outs = []
    for i in range(2 if twice else 1):
        w = g.constant((rng.standard_normal((kout, c, k, k)) * 0.3).astype(np.float32), f"w{i}")
        b = g.constant((rng.standard_normal(kout) * 0.1).astype(np.float32), f"b{i}")
        y = g.add_node("Conv", [x, w, b], 1, {"strides": [2, 2], "pads": pads, "kernel_shape": [k, k]},
                       name=f"conv{i}", output_names=[f"conv{i}"]).output
        outs.append(g.add_node("Relu", [y], 1, {}, name=f"relu{i}", output_names=[f"y{i}"]).output)
    for i, y in enumerate(outs):
        g.add_output(y, f"y{i}")
    infer_shapes(g)
    return g, {"x": rng.standard_normal((2, c, hw, hw)).astype(np.float32)}


CASES = [
    (3, 32, 7, [3, 3, 3, 3], False),   # the ResNet stem shape
    (3, 30, 3, [1, 1, 1, 1], False),   # the MobileNet stem shape
    (1, 16, 5, [2, 2, 2, 2], False),
    (2, 18, 4, [1, 1, 2, 2], False),   # even kernel, asymmetric pads
    (5, 20, 3, [0, 0, 0, 0], False),
    (6, 12, 2, [0, 1, 1, 0], False),
    (3, 24, 7, [3, 3, 3, 3], True),    # input shared by two convolutions: read from NHWC
]


def test_s2d_is_chosen():
    """CPU: the rewrite applies to every case; the input Transpose folds unless shared (with
    one channel the layout pass leaves a Reshape, which is a view, instead of a Transpose)."""
    for c, hw, k, pads, twice in CASES:
        g, _ = conv_graph(c, hw, k, pads, twice=twice)
        optimize(g, "O3")
        schedule(g)
        gen = hip_codegen.generate_hip(g, "greedy_by_size", True, False, lambda *a: 0)
        assert gen.kernels.get("space_to_depth") == (2 if twice else 1), gen.kernels
        assert gen.kernels.get("folded", 0) == (0 if twice or c == 1 else 1)


@pytest.mark.gpu
@pytest.mark.parametrize("c, hw, k, pads, twice", CASES)
def test_s2d_conv_matches_oracle(c, hw, k, pads, twice, hip_cache, monkeypatch):
    g, feeds = conv_graph(c, hw, k, pads, twice=twice)
    want = oracle.run_graph(g, feeds)
    for on in (True, False):
        monkeypatch.setattr(hip_codegen, "SPACE_TO_DEPTH", on)
        model = compile_hip(conv_graph(c, hw, k, pads, twice=twice)[0], hip_cache)
        try:
            got = model.run(feeds)
            assert ("space_to_depth" in model.report.kernels) == on
        finally:
            model.release()
        for name, w in want.items():
            assert float(np.max(np.abs(got[name].astype(np.float64) - w))) <= 2e-5 * max(1.0, float(np.abs(w).max()))
