"""Short-K GEMMs over many rows on the streaming kernel (each wave streams 32-row tiles, A
straight into registers, its column group of B held in registers, no LDS).

Selected for a strided A with unit column stride, a constant (packed) B, K <= 32 with K % 4 == 0,
at least 4096 rows and at most 768 columns: the expand and project 1 x 1 convolutions of MobileNet-style blocks at large batch; and
over an NHWC image read through its implicit im2col (one channel group, K <= 48, at most 32
columns): MobileNetV2's stem. The cases cover the k layouts (K <= 16: eight k per lane half;
K <= 32: sixteen; K <= 48: twenty-four), K that leaves part of a lane half unused, one to six
32-column blocks per group and several groups, ragged M and N,
the bias / residual / activation epilogue, and convolution windows with padding and stride;
compared with the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import check_hip
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.shape_inference import infer_shapes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(
    "m, k, n, epilogue",
    [
        (4096, 16, 96, "bias_relu"),     # three blocks, K = 16: eight k per lane half
        (5000, 4, 8, "bias_relu"),       # ragged M, one narrow block, K = 4
        (4100, 12, 200, "none"),         # ragged M, seven blocks in two groups
        (6272, 24, 144, "bias_clip"),    # K = 24: the upper lane half reads k 16 .. 23
        (4096, 32, 192, "bias_relu"),    # six blocks in one group
        (8192, 20, 768, "bias"),         # 24 blocks, four groups
        (6000, 32, 16, "residual"),      # project layer with its residual
        (4096, 28, 33, "residual"),      # N = 33: a second block with one live column
        (4096, 16, 96, "none_nan"),      # a NaN input element: its row stays NaN (no clamp)
        (4096, 24, 40, "residual_nan"),  # NaN in the residual passes through
    ],
)
def test_stream_gemm(m, k, n, epilogue, hip_cache):
    print(f"[gpu] stream gemm {m}x{k}x{n} {epilogue}", flush=True)
    rng = np.random.default_rng(m + 3 * k + n)
    g = Graph("stream")
    x = g.add_input("x", TensorType("float32", (m, k)))
    w = g.constant((rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32), "w")
    y = g.add_node("MatMul", [x, w], 1, {}, name="mm").output
    feeds = {"x": rng.standard_normal((m, k)).astype(np.float32)}
    if epilogue.startswith("bias"):
        b = g.constant(rng.standard_normal(n).astype(np.float32), "b")
        y = g.add_node("Add", [y, b], 1, {}, name="bias").output
    if epilogue == "bias_relu":
        y = g.add_node("Relu", [y], 1, {}, name="relu").output
    elif epilogue == "bias_clip":
        lo = g.constant(np.asarray(0.0, np.float32), "lo")
        hi = g.constant(np.asarray(6.0, np.float32), "hi")
        y = g.add_node("Clip", [y, lo, hi], 1, {}, name="clip").output
    elif epilogue.startswith("residual"):
        r = g.add_input("r", TensorType("float32", (m, n)))
        feeds["r"] = rng.standard_normal((m, n)).astype(np.float32)
        y = g.add_node("Add", [y, r], 1, {}, name="res").output
    if epilogue == "none_nan":
        feeds["x"][5, 3] = np.nan
    elif epilogue == "residual_nan":
        feeds["r"][7, 11] = np.nan
    g.add_output(y, "y")
    infer_shapes(g)
    got = check_hip(g, feeds, hip_cache, opt="O3", rtol=2e-5, atol=2e-5)["y"]
    if epilogue == "none_nan":
        assert np.isnan(got[5]).all() and np.isfinite(np.delete(got, 5, axis=0)).all()
    elif epilogue == "residual_nan":
        assert np.isnan(got[7, 11]) and np.isnan(got).sum() == 1


@pytest.mark.parametrize("n, cin, cout, hw, residual", [(2, 16, 96, 56, False), (1, 24, 144, 64, False),
                                                        (2, 32, 32, 48, True)])
def test_stream_pointwise_conv(n, cin, cout, hw, residual, hip_cache):
    """1 x 1 convolutions (NCHW in the graph, NHWC after O3) with BN-style bias and ReLU6."""
    print(f"[gpu] stream conv {n}x{cin}->{cout} {hw}x{hw} residual={residual}", flush=True)
    rng = np.random.default_rng(cin * cout + hw)
    g = Graph("pw")
    x = g.add_input("x", TensorType("float32", (n, cin, hw, hw)))
    w = g.constant((rng.standard_normal((cout, cin, 1, 1)) / np.sqrt(cin)).astype(np.float32), "w")
    b = g.constant(rng.standard_normal(cout).astype(np.float32) * 0.3, "b")
    y = g.add_node("Conv", [x, w, b], 1, {"kernel_shape": [1, 1]}, name="conv").output
    if residual:
        y = g.add_node("Add", [y, x], 1, {}, name="res").output
    lo = g.constant(np.asarray(0.0, np.float32), "lo")
    hi = g.constant(np.asarray(6.0, np.float32), "hi")
    y = g.add_node("Clip", [y, lo, hi], 1, {}, name="relu6").output
    g.add_output(y, "y")
    infer_shapes(g)
    check_hip(g, feeds={"x": rng.standard_normal((n, cin, hw, hw)).astype(np.float32)}, cache=hip_cache,
              opt="O3", rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize(
    "n, h, w, c, kout, k, stride, pad",
    [
        (8, 64, 64, 12, 32, 2, 1, 0),   # MobileNetV2's stem form: 2 x 2 over a space-to-depth copy (K 48)
        (4, 70, 66, 8, 16, 2, 1, 1),    # K 32 with a padded border, ragged rows
        (5, 61, 63, 4, 24, 3, 2, 1),    # 3 x 3 stride 2 over 4 channels (K 36), ragged rows
    ],
)
def test_stream_convolution(n, h, w, c, kout, k, stride, pad, hip_cache):
    """NHWC convolutions whose im2col K fits the streaming kernel (>= 4096 output pixels)."""
    print(f"[gpu] stream conv {n}x{h}x{w}x{c} -> {kout} k{k} s{stride} p{pad}", flush=True)
    rng = np.random.default_rng(n + h + c + kout)
    g = Graph("stream_conv")
    x = g.add_input("x", TensorType("float32", (n, h, w, c)))
    wt = g.constant((rng.standard_normal((k, k, c, kout)) / np.sqrt(k * k * c)).astype(np.float32), "w")
    b = g.constant(rng.standard_normal(kout).astype(np.float32), "b")
    y = g.add_node("FusedConv", [x, wt, b], 1,
                   {"kernel_shape": [k, k], "pads": [pad] * 4, "strides": [stride, stride], "layout": "NHWC",
                    "activation": "clip", "clip_min": 0.0, "clip_max": 6.0}, name="conv").output
    g.add_output(y, "y")
    infer_shapes(g)
    oh = (h + 2 * pad - k) // stride + 1
    ow = (w + 2 * pad - k) // stride + 1
    assert n * oh * ow >= 4096
    check_hip(g, {"x": rng.standard_normal((n, h, w, c)).astype(np.float32)}, hip_cache, opt="O0")
