"""GEMMs and convolutions shaped like batch-1 layers whose 64 x 64 tiles are too few for the CUs:
the library runs them on the wave-split kernel (32 x 32 tiles, the K range dealt to the four
waves of a workgroup, partial tiles summed in LDS) instead of a K split plus a reduction
launch (or, for deep K over few rows, with a K split of its own, four times as many waves
sharing K). Shapes chosen so that the selection applies: K of at least 512, a K split that the
64 x 64 tiling would take, at most 512 tiles of 32 x 32 (times the split; 768 without a split). Ragged M, N and K, a partial last K
stage, bias / residual / activation epilogues, strided and dilated windows; compared with the
oracle (rtol 1e-4)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import check_hip, f32
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.shape_inference import infer_shapes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(
    "m, n, k, epilogue",
    [
        (128, 256, 1024, "bias_relu"),
        (100, 50, 600, "none"),          # ragged tiles, N not a multiple of 4, partial K stage
        (300, 96, 800, "residual"),
        (128, 2304, 768, "bias_relu"),   # 288 tiles: two workgroups per CU
        (196, 1024, 256, "bias_relu"),   # K below the split threshold on 64 too few tiles
        (6272, 96, 576, "bias_relu"),    # 588 tiles of 32 x 32 (up to three per CU), no K split
        (1, 1000, 2048, "bias_relu"),    # deep K over one row: wave split plus a K split
    ],
)
def test_wave_split_gemm(m, n, k, epilogue, hip_cache):
    rng = np.random.default_rng(m * 7 + n)
    g = Graph("ws_gemm")
    x = g.add_input("x", TensorType("float32", (m, k)))
    w = g.constant((rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32), "w")
    y = g.add_node("MatMul", [x, w], 1, {}, name="mm").output
    feeds = {"x": rng.standard_normal((m, k)).astype(np.float32)}
    if epilogue == "bias_relu":
        b = g.constant(rng.standard_normal(n).astype(np.float32), "b")
        y = g.add_node("Add", [y, b], 1, {}, name="bias").output
        y = g.add_node("Relu", [y], 1, {}, name="relu").output
    elif epilogue == "residual":
        r = g.add_input("r", TensorType("float32", (m, n)))
        feeds["r"] = rng.standard_normal((m, n)).astype(np.float32)
        y = g.add_node("Add", [y, r], 1, {}, name="res").output
    g.add_output(y, "y")
    infer_shapes(g)
    check_hip(g, feeds, hip_cache, opt="O3")


@pytest.mark.parametrize(
    "cin, cout, hw, stride, dil, residual, ksize",
    [
        (64, 64, 56, 1, 1, False, 3),    # the ResNet-50 stage-1 3 x 3 layer at batch 1
        (128, 128, 28, 1, 1, True, 3),   # stage 2, with the residual Add
        (64, 96, 57, 2, 1, False, 3),    # strided, ragged output
        (64, 64, 20, 1, 2, True, 3),     # dilated
        (256, 256, 14, 1, 1, False, 3),  # deep K (2304): the wave-split launch splits K as well
        (512, 512, 7, 1, 1, True, 3),    # K 4608 over 49 pixels
        (256, 1024, 14, 1, 1, False, 1), # 1 x 1, K 256: no split, a quarter of the stages
        (256, 512, 56, 2, 1, False, 1),  # 1 x 1 stride-2 downsample to 28 x 28
    ],
)
def test_wave_split_conv(cin, cout, hw, stride, dil, residual, ksize, hip_cache):
    rng = np.random.default_rng(cin + cout + hw)
    g = Graph("ws_conv")
    x = g.add_input("x", TensorType("float32", (1, cin, hw, hw)))
    feeds = {"x": rng.standard_normal((1, cin, hw, hw)).astype(np.float32)}
    wt = g.constant((rng.standard_normal((cout, cin, ksize, ksize)) / np.sqrt(cin * ksize * ksize)).astype(np.float32), "w")
    b = g.constant(rng.standard_normal(cout).astype(np.float32) * 0.1, "b")
    attrs = {"kernel_shape": [ksize, ksize], "pads": [dil * (ksize // 2)] * 4, "strides": [stride, stride],
             "dilations": [dil, dil]}
    y = g.add_node("Conv", [x, wt, b], 1, attrs, name="conv").output
    if residual:
        y = g.add_node("Add", [y, x], 1, {}, name="res").output
    y = g.add_node("Relu", [y], 1, {}, name="relu").output
    g.add_output(y, "y")
    infer_shapes(g)
    check_hip(g, feeds, hip_cache, opt="O3")
