"""Every activation of the epilogue ABI run inside a fused GEMM / convolution on the GPU.

The reference's activation set (codegen/runtime/mgc_runtime.h:93-114, ops.ACTIVATIONS) is
none, relu, clip, gelu, gelu_tanh, tanh and sigmoid; its fusion pass absorbs a bias Add, a
residual Add and then one activation into a FusedGemm / FusedConv (passes/fusion.py:266-300),
and its closed-form test checks each activation of FusedGemm (tests/test_ops.py:440-465). Here
each activation is absorbed at O3 into every kernel family that runs an epilogue (64 x 64 and
128 x 32 DMA tiles, the wave-split kernel, a K split with its reduction, the register-staged
kernel of grouped and NCHW convolutions, the space-to-depth stem, the depthwise kernels) and
compared with the oracle; the test also asserts that the activation really was fused.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import check_hip
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.shape_inference import infer_shapes

pytestmark = pytest.mark.gpu

ACTIVATIONS = ["relu", "clip", "gelu", "gelu_tanh", "tanh", "sigmoid"]


def _activation(g: Graph, y, act: str):
    if act == "relu":
        return g.add_node("Relu", [y], 1, {}, name="act").output
    if act == "clip":
        lo = g.constant(np.asarray(-0.5, np.float32), "lo")
        hi = g.constant(np.asarray(0.5, np.float32), "hi")
        return g.add_node("Clip", [y, lo, hi], 1, {}, name="act").output
    if act in ("gelu", "gelu_tanh"):
        attrs = {"approximate": "tanh"} if act == "gelu_tanh" else {}
        return g.add_node("Gelu", [y], 1, attrs, name="act").output
    return g.add_node({"tanh": "Tanh", "sigmoid": "Sigmoid"}[act], [y], 1, {}, name="act").output


def _fused_activations(g: Graph, op: str) -> list[str]:
    return [str(n.attrs.get("activation", "none")) for n in g.nodes if n.op == op]


GEMM_SHAPES = [
    (256, 320, 256),    # 64 x 64 DMA tiles
    (300, 24, 64),      # 128 x 32 tiles (narrow N)
    (128, 256, 1024),   # wave-split kernel
    (64, 768, 4096),    # a K split and its reduction
]


@pytest.mark.parametrize("act", ACTIVATIONS)
@pytest.mark.parametrize("m, n, k", GEMM_SHAPES)
@pytest.mark.parametrize("residual", [False, True])
def test_fused_gemm_activation(m, n, k, act, residual, hip_cache):
    rng = np.random.default_rng(m + n + k + len(act))
    g = Graph("gemm_act")
    x = g.add_input("x", TensorType("float32", (m, k)))
    feeds = {"x": rng.standard_normal((m, k)).astype(np.float32)}
    w = g.constant((rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32), "w")
    b = g.constant(rng.standard_normal(n).astype(np.float32) * 0.5, "b")
    y = g.add_node("MatMul", [x, w], 1, {}, name="mm").output
    y = g.add_node("Add", [y, b], 1, {}, name="bias").output
    if residual:
        r = g.add_input("r", TensorType("float32", (m, n)))
        feeds["r"] = rng.standard_normal((m, n)).astype(np.float32)
        y = g.add_node("Add", [y, r], 1, {}, name="res").output
    y = _activation(g, y, act)
    g.add_output(y, "y")
    infer_shapes(g)
    check_hip(g, feeds, hip_cache, opt="O3", rtol=2e-5, atol=2e-5)
    assert _fused_activations(g, "FusedGemm") == [act]


CONV_CASES = [
    # (n, cin, cout, hw, k, stride, group)
    (2, 64, 64, 28, 3, 1, 1),     # implicit-GEMM 3x3, 64 x 64 tiles
    (1, 256, 64, 56, 1, 1, 1),    # pointwise (plain strided A)
    (1, 64, 64, 56, 3, 1, 1),     # batch-1 3x3: wave-split kernel
    (1, 16, 24, 20, 1, 1, 1),     # narrow pointwise: 128 x 32 tiles
    (2, 8, 12, 13, 3, 2, 2),      # grouped: register-staged kernel
    (1, 3, 16, 32, 7, 2, 1),      # C = 3 stride-2 stem: space-to-depth then the DMA kernel
    (2, 32, 32, 17, 3, 1, 32),    # depthwise 3x3, stride 1
    (1, 48, 48, 30, 3, 2, 48),    # depthwise 3x3, stride 2
]


@pytest.mark.parametrize("act", ACTIVATIONS)
@pytest.mark.parametrize("case", CONV_CASES)
def test_fused_conv_activation(case, act, hip_cache):
    n, cin, cout, hw, k, stride, group = case
    rng = np.random.default_rng(cin * 31 + cout + k + len(act))
    g = Graph("conv_act")
    x = g.add_input("x", TensorType("float32", (n, cin, hw, hw)))
    feeds = {"x": rng.standard_normal((n, cin, hw, hw)).astype(np.float32)}
    fan_in = cin // group * k * k
    wt = g.constant((rng.standard_normal((cout, cin // group, k, k)) / np.sqrt(fan_in)).astype(np.float32), "w")
    b = g.constant(rng.standard_normal(cout).astype(np.float32) * 0.5, "b")
    attrs = {"kernel_shape": [k, k], "pads": [k // 2] * 4, "strides": [stride, stride], "group": group}
    y = g.add_node("Conv", [x, wt, b], 1, attrs, name="conv").output
    if stride == 1 and cin == cout:
        y = g.add_node("Add", [y, x], 1, {}, name="res").output
    y = _activation(g, y, act)
    g.add_output(y, "y")
    infer_shapes(g)
    check_hip(g, feeds, hip_cache, opt="O3", rtol=2e-5, atol=2e-5)
    assert _fused_activations(g, "FusedConv") == [act]
