"""64 x 64 GEMM launches whose tile count is just past a multiple of the 256 CUs: the last r
tiles (0 < r <= 64, K >= 128, or r <= 128 with K >= 512: csrc/gemm.hip kQuarterTiles,
kQuarterMinK, kQuarterTilesDeepK) run as 4 r quarter
tiles of 32 x 32, the four waves of a quarter's
workgroup each taking a quarter of K (16 of every 64 k) and the partial quarters summed in LDS
in wave order (csrc/gemm.hip, gemm_dma_tile with QUARTER). Shapes chosen so that the tail
applies: ragged M and N (quarters partly or wholly past the matrix edge), K not a multiple of
the 64-k quarter stage, N not a multiple of 4 (scalar stores), convolution windows over 64 and
128 channels, and a 96-channel window that keeps whole tiles (quarter stages need channel
groups of a multiple of 64), and launches of between one and two tiles per CU with K >= 512,
whose second half of tiles all run as quarters (kHalfQuarterMinK); compared with the oracle."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import check_hip
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.shape_inference import infer_shapes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(
    "m, n, k, epilogue",
    [
        (16428, 64, 300, "bias_relu"),  # 257 tiles: one tile in quarters, the last 44 rows
        (17000, 120, 264, "residual"),  # 532 tiles (20 in quarters), ragged rows and columns,
                                        # the last 64-k stage holds 8 k
        (5000, 832, 256, "none"),       # 1027 tiles: four full rounds, then 3 tiles in quarters
        (16640, 50, 256, "bias_relu"),  # 260 tiles, N not a multiple of 4
        (3264, 768, 520, "bias_relu"),  # 612 tiles, K >= 512: a 100-tile tail in quarters
        (6272, 256, 1024, "bias_relu"), # 392 tiles (1.5 per CU), K >= 512: 196 whole, 784 quarters
        (7990, 256, 600, "residual"),   # 500 tiles: 250 whole, the last row of quarters past M
    ],
)
def test_quarter_tail_gemm(m, n, k, epilogue, hip_cache):
    rng = np.random.default_rng(m + n + k)
    g = Graph("q_gemm")
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
    "batch, cin, cout, hw, stride, residual",
    [
        (1, 64, 64, 130, 1, True),     # 265 tiles of 16900 pixels: 9 in quarters, with residual
        (11, 128, 128, 56, 2, False),  # strided, 270 tiles: 14 in quarters
        (1, 96, 64, 130, 1, False),    # channel group 96: whole tiles only
    ],
)
def test_quarter_tail_conv(batch, cin, cout, hw, stride, residual, hip_cache):
    rng = np.random.default_rng(batch * 1000 + cin + hw)
    g = Graph("q_conv")
    x = g.add_input("x", TensorType("float32", (batch, cin, hw, hw)))
    feeds = {"x": rng.standard_normal((batch, cin, hw, hw)).astype(np.float32)}
    wt = g.constant((rng.standard_normal((cout, cin, 3, 3)) / np.sqrt(cin * 9)).astype(np.float32), "w")
    b = g.constant(rng.standard_normal(cout).astype(np.float32) * 0.1, "b")
    attrs = {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "strides": [stride, stride]}
    y = g.add_node("Conv", [x, wt, b], 1, attrs, name="conv").output
    if residual:
        y = g.add_node("Add", [y, x], 1, {}, name="res").output
    y = g.add_node("Relu", [y], 1, {}, name="relu").output
    g.add_output(y, "y")
    infer_shapes(g)
    check_hip(g, feeds, hip_cache, opt="O3")
