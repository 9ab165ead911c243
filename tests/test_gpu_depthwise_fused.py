"""Depthwise 3 x 3 convolutions computed inside the GEMM of the pointwise convolution that reads
them (mgc_hip_gemm_dw).

A MobileNet inverted-residual block (the reference's mobilenet_v2 builder,
src/ml_graph_compiler/models.py, whose C backend runs mgc_depthwise_nhwc and then mgc_gemm for
the projection, codegen/c.py:1126-1167) expands with a 1 x 1 convolution, filters every channel
with a 3 x 3 depthwise convolution (stride 1 or 2, ReLU6) and projects with a 1 x 1 convolution,
plus the block input when the shapes allow. The hip backend computes each A tile of the
projection GEMM from the expanded tensor while staging it. Each case builds such a block,
compiles it at O3 with the size threshold lifted (DEPTHWISE_FUSE_MIN_ROWS = 0), asserts that
the pair was fused and compares with the oracle on the unoptimized graph; the same block with
the fusion off gives the reference's two-kernel form, and both must agree with the oracle to
the same bound. Shapes reach both tile widths (64 x 32 for projections of at most 32 channels,
64 x 64 above), channel counts that end a 32-wide K stage early, odd image sizes under stride
2, and row counts that end a 64-row tile early. When the depthwise input is a caller buffer the
generated code checks its 16-byte alignment at run time and runs the two convolutions apart if
it is misaligned; both branches are run.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip
from ml_graph_compiler.codegen import hip as hip_codegen
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu

RTOL = ATOL = 3e-5


def _conv(g: Graph, rng, x, cin: int, cout: int, k: int, stride: int, name: str, group: int = 1):
    w = g.constant((rng.standard_normal((cout, cin // group, k, k)) / np.sqrt(cin // group * k * k)).astype(np.float32),
                   f"{name}_w")
    b = g.constant((rng.standard_normal(cout) * 0.2).astype(np.float32), f"{name}_b")
    attrs = {"kernel_shape": [k, k], "pads": [k // 2] * 4, "strides": [stride, stride], "group": group}
    return g.add_node("Conv", [x, w, b], 1, attrs, name=name).output


def inverted_residual(n: int, cin: int, cexp: int, cout: int, hw: int, stride: int,
                      seed: int = 0) -> tuple[Graph, dict[str, np.ndarray]]:
    """x -> relu6(1x1 expand) -> relu6(3x3 depthwise / stride) -> 1x1 project [+ x]."""
    rng = np.random.default_rng(seed)
    g = Graph("inverted_residual")
    x = g.add_input("x", TensorType("float32", (n, cin, hw, hw)))
    lo = g.constant(np.asarray(0.0, np.float32), "lo")
    hi = g.constant(np.asarray(6.0, np.float32), "hi")
    y = g.add_node("Clip", [_conv(g, rng, x, cin, cexp, 1, 1, "expand"), lo, hi], 1, {}, name="a1").output
    y = g.add_node("Clip", [_conv(g, rng, y, cexp, cexp, 3, stride, "dw", group=cexp), lo, hi], 1, {},
                   name="a2").output
    y = _conv(g, rng, y, cexp, cout, 1, 1, "project")
    if stride == 1 and cin == cout:
        y = g.add_node("Add", [y, x], 1, {}, name="add").output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, {"x": rng.standard_normal((n, cin, hw, hw)).astype(np.float32)}


CASES = [
    # (n, cin, cexp, cout, hw, stride)
    (2, 16, 96, 24, 28, 2),    # MobileNetV2 block 1 shape (scaled): stride 2, 64 x 32 tiles, N = 24
    (2, 24, 144, 24, 21, 1),   # residual block, odd image, 882 rows (last tile partial)
    (1, 32, 192, 64, 14, 1),   # N = 64: one 64 x 64 tile column
    (2, 64, 384, 96, 9, 2),    # stride 2 over an odd image (5 x 5), N = 96 (second tile column partial)
    (3, 8, 36, 40, 11, 1),     # C = 36: the second K stage holds four channels; N = 40
    (1, 160, 960, 320, 7, 1),  # the last block: K = 960, N = 320
    (1, 12, 4, 8, 6, 2),       # four channels, eight outputs, 3 x 3 output
]


def _run(g: Graph, feeds, cache, fuse: bool, monkeypatch) -> tuple[dict[str, np.ndarray], dict[str, int]]:
    monkeypatch.setattr(hip_codegen, "FUSE_INVERTED_RESIDUAL", False)  # the whole-block kernel: test_gpu_mbconv.py
    monkeypatch.setattr(hip_codegen, "FUSE_EXPAND_DEPTHWISE", False)  # expansion + depthwise: test_gpu_expand_dw.py
    monkeypatch.setattr(hip_codegen, "FUSE_DEPTHWISE_POINTWISE", fuse)
    monkeypatch.setattr(hip_codegen, "DEPTHWISE_FUSE_MIN_ROWS", 0)
    model = compile_hip(g, cache, "O3")
    try:
        return model.run(feeds), dict(model.report.kernels)
    finally:
        model.release()


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_depthwise_fused_matches_oracle(case, hip_cache, monkeypatch):
    n, cin, cexp, cout, hw, stride = case
    print(f"[gpu] depthwise -> pointwise block {case}", flush=True)
    g, feeds = inverted_residual(n, cin, cexp, cout, hw, stride, seed=sum(case))
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache, True, monkeypatch)
    assert kernels.get("gemm_depthwise") == 1 and "depthwise" not in kernels, kernels
    np.testing.assert_allclose(got["y"], expected, rtol=RTOL, atol=ATOL)
    g2, _ = inverted_residual(n, cin, cexp, cout, hw, stride, seed=sum(case))
    unfused, kernels = _run(g2, feeds, hip_cache, False, monkeypatch)
    assert "gemm_depthwise" not in kernels and kernels.get("depthwise") == 1
    np.testing.assert_allclose(unfused["y"], expected, rtol=RTOL, atol=ATOL)


def _nhwc_pair(n: int, h: int, c: int, cout: int, stride: int, act: str, seed: int):
    """An already-NHWC depthwise -> pointwise pair whose depthwise input is a graph input, so the
    generated code checks its alignment at run time."""
    rng = np.random.default_rng(seed)
    g = Graph("nhwc_pair")
    x = g.add_input("x", TensorType("float32", (n, h, h, c)))
    wd = g.constant((rng.standard_normal((3, 3, 1, c)) / 3.0).astype(np.float32), "wd")
    bd = g.constant(rng.standard_normal(c).astype(np.float32), "bd")
    wp = g.constant((rng.standard_normal((1, 1, c, cout)) / np.sqrt(c)).astype(np.float32), "wp")
    bp = g.constant(rng.standard_normal(cout).astype(np.float32), "bp")
    d = g.add_node("FusedConv", [x, wd, bd], 1,
                   {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "strides": [stride, stride], "group": c,
                    "layout": "NHWC", "activation": act, "clip_min": 0.0, "clip_max": 6.0}, name="dw").output
    y = g.add_node("FusedConv", [d, wp, bp], 1,
                   {"kernel_shape": [1, 1], "pads": [0, 0, 0, 0], "strides": [1, 1], "layout": "NHWC",
                    "activation": "none"}, name="pw").output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, {"x": rng.standard_normal((n, h, h, c)).astype(np.float32)}


@pytest.mark.parametrize("act", ["none", "relu", "clip"])
def test_depthwise_fused_activations_over_caller_buffer(act, hip_cache, monkeypatch):
    print(f"[gpu] depthwise -> pointwise over a caller buffer, act {act}", flush=True)
    monkeypatch.setattr(hip_codegen, "DEPTHWISE_FUSE_MIN_ROWS", 0)
    g, feeds = _nhwc_pair(2, 13, 48, 56, 1, act, seed=5)
    expected = oracle.run_graph(g, feeds)["y"]
    model = compile_hip(g, hip_cache, "O0")
    try:
        assert model.report.kernels.get("gemm_depthwise") == 1, model.report.kernels
        got = model.run(feeds)["y"]
    finally:
        model.release()
    np.testing.assert_allclose(got, expected, rtol=RTOL, atol=ATOL)


def test_depthwise_fused_over_misaligned_caller_buffer(hip_cache, monkeypatch):
    """The depthwise input 4 bytes off a 16-byte boundary: the generated code sees it at run
    time and runs the depthwise and the pointwise convolutions as two kernels instead."""
    import torch

    print("[gpu] depthwise -> pointwise over a misaligned caller buffer", flush=True)
    monkeypatch.setattr(hip_codegen, "DEPTHWISE_FUSE_MIN_ROWS", 0)
    g, feeds = _nhwc_pair(1, 10, 32, 24, 2, "clip", seed=9)
    expected = oracle.run_graph(g, feeds)["y"]
    model = compile_hip(g, hip_cache, "O0")
    try:
        assert model.report.kernels.get("gemm_depthwise") == 1, model.report.kernels
        dev = torch.device("cuda:0")
        host = torch.from_numpy(np.ascontiguousarray(feeds["x"]).reshape(-1))
        buf = torch.zeros(host.numel() + 1, dtype=torch.float32, device=dev)
        view = buf[1:]  # 4 bytes past the allocation's start
        view.copy_(host)
        assert view.data_ptr() % 16 == 4
        out = torch.empty(expected.size, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        model.run_device([view.data_ptr()], [out.data_ptr()])
        got = out.cpu().numpy().reshape(expected.shape)
    finally:
        model.release()
    np.testing.assert_allclose(got, expected, rtol=RTOL, atol=ATOL)
