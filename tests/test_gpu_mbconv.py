"""Whole inverted-residual blocks as one launch (mgc_hip_mbconv).

A MobileNetV2 block with expansion t > 1 (the reference's C backend runs it as mgc_gemm,
mgc_depthwise_nhwc and mgc_gemm with both intermediates in its arena, codegen/c.py:1102-1226)
expands the input with a 1 x 1 convolution and ReLU6, filters every expanded channel with a
3 x 3 depthwise convolution (stride 1 or 2) and ReLU6, and projects with a 1 x 1 convolution,
plus the block input when the shapes allow. The hip backend evaluates the expansion and the
depthwise convolution per 8 x 8-pixel output tile while it forms the projection GEMM's A operand,
so neither intermediate is written. Each case builds such a block, compiles it at O3 with the
size threshold lifted (MBCONV_MIN_ROWS = 0), asserts that the whole block became one
gemm_mbconv launch, and compares with the oracle on the unoptimized graph (the bound of the
two-kernel form in test_gpu_depthwise_fused.py). Shapes reach both strides, every supported
input width (16, 24, 32 channels), expanded widths that end a 32-channel stage early (36, 4)
and the 256-channel maximum, projections of 5 to 32 channels, odd images whose last tiles are
partial, ReLU and ReLU6, with and without the residual. When the block input is a caller buffer
the generated code checks its alignment at run time and runs the three convolutions apart if it
is misaligned; both branches are run.
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


def block(n: int, cin: int, cexp: int, cout: int, h: int, w: int, stride: int, act: str,
          seed: int = 0) -> tuple[Graph, dict[str, np.ndarray]]:
    """x -> act(1x1 expand) -> act(3x3 depthwise / stride) -> 1x1 project [+ x]."""
    rng = np.random.default_rng(seed)
    g = Graph("inverted_residual")
    x = g.add_input("x", TensorType("float32", (n, cin, h, w)))
    lo = g.constant(np.asarray(0.0, np.float32), "lo")
    hi = g.constant(np.asarray(6.0, np.float32), "hi")

    def activation(v, name):
        if act == "relu":
            return g.add_node("Relu", [v], 1, {}, name=name).output
        return g.add_node("Clip", [v, lo, hi], 1, {}, name=name).output

    y = activation(_conv(g, rng, x, cin, cexp, 1, 1, "expand"), "a1")
    y = activation(_conv(g, rng, y, cexp, cexp, 3, stride, "dw", group=cexp), "a2")
    y = _conv(g, rng, y, cexp, cout, 1, 1, "project")
    if stride == 1 and cin == cout:
        y = g.add_node("Add", [y, x], 1, {}, name="add").output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, {"x": rng.standard_normal((n, cin, h, w)).astype(np.float32)}


CASES = [
    # (n, cin, cexp, cout, h, w, stride, act)
    (2, 16, 96, 24, 28, 28, 2, "clip"),    # MobileNetV2's first expanded block (scaled): stride 2
    (2, 24, 144, 24, 21, 21, 1, "clip"),   # residual, odd image: the last tiles of a row are partial
    (1, 32, 192, 32, 14, 14, 1, "relu"),   # residual, two 8 x 8 tiles per row, the second partial
    (2, 24, 144, 32, 13, 17, 2, "clip"),   # stride 2 over an odd, non-square image
    (3, 16, 36, 5, 11, 9, 1, "relu"),      # 36 expanded channels: the second stage holds four; N = 5
    (1, 32, 256, 32, 9, 9, 1, "clip"),     # the 256-channel maximum: eight stages
    (1, 16, 4, 8, 6, 6, 2, "clip"),        # four expanded channels, 3 x 3 output
    (2, 24, 120, 16, 30, 30, 2, "relu"),   # 120 = 3.75 stages, 15 x 15 output
]


def _run(g: Graph, feeds, cache, monkeypatch, opt: str = "O3") -> tuple[dict[str, np.ndarray], dict[str, int]]:
    monkeypatch.setattr(hip_codegen, "MBCONV_MIN_ROWS", 0)
    model = compile_hip(g, cache, opt)
    try:
        return model.run(feeds), dict(model.report.kernels)
    finally:
        model.release()


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_inverted_residual_block_matches_oracle(case, hip_cache, monkeypatch):
    n, cin, cexp, cout, h, w, stride, act = case
    print(f"[gpu] inverted-residual block {case}", flush=True)
    g, feeds = block(n, cin, cexp, cout, h, w, stride, act, seed=len(CASES) + sum(c for c in case if isinstance(c, int)))
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache, monkeypatch)
    assert kernels.get("gemm_mbconv") == 1 and "depthwise" not in kernels and "gemm_depthwise" not in kernels, kernels
    assert kernels.get("gemm") == 1, kernels  # the one launch is the projection's
    np.testing.assert_allclose(got["y"], expected, rtol=RTOL, atol=ATOL)


def _nhwc_block(n: int, h: int, cin: int, cexp: int, cout: int, stride: int, seed: int):
    """An NHWC block whose input is a graph input, so the generated code checks its alignment."""
    rng = np.random.default_rng(seed)
    g = Graph("nhwc_block")
    x = g.add_input("x", TensorType("float32", (n, h, h, cin)))

    def conv(v, k, c_in, c_out, s, group, name, act):
        w = g.constant((rng.standard_normal((k, k, c_in // group, c_out)) / np.sqrt(k * k * c_in / group))
                       .astype(np.float32), f"{name}_w")
        b = g.constant((rng.standard_normal(c_out) * 0.2).astype(np.float32), f"{name}_b")
        return g.add_node("FusedConv", [v, w, b], 1,
                          {"kernel_shape": [k, k], "pads": [k // 2] * 4, "strides": [s, s], "group": group,
                           "layout": "NHWC", "activation": act, "clip_min": 0.0, "clip_max": 6.0}, name=name).output

    y = conv(x, 1, cin, cexp, 1, 1, "ex", "clip")
    y = conv(y, 3, cexp, cexp, stride, cexp, "dw", "clip")
    y = conv(y, 1, cexp, cout, 1, 1, "pw", "none")
    g.add_output(y, "y")
    infer_shapes(g)
    return g, {"x": rng.standard_normal((n, h, h, cin)).astype(np.float32)}


def test_inverted_residual_over_caller_buffers(hip_cache, monkeypatch):
    """The block input is the caller's buffer: aligned, the fused launch runs; 4 bytes off a
    16-byte boundary, the generated code runs the three convolutions apart instead."""
    import torch

    print("[gpu] inverted-residual block over caller buffers", flush=True)
    monkeypatch.setattr(hip_codegen, "MBCONV_MIN_ROWS", 0)
    g, feeds = _nhwc_block(2, 15, 24, 144, 24, 2, seed=4)
    expected = oracle.run_graph(g, feeds)["y"]
    model = compile_hip(g, hip_cache, "O0")
    try:
        assert model.report.kernels.get("gemm_mbconv") == 1, model.report.kernels
        np.testing.assert_allclose(model.run(feeds)["y"], expected, rtol=RTOL, atol=ATOL)
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


def stem_block(n: int, h: int, w: int, cexp: int, cout: int, stem_stride: int, stride: int, act: str,
               seed: int = 0) -> tuple[Graph, dict[str, np.ndarray]]:
    """image -> act(3x3 stem / stem_stride, 3 -> cexp) -> act(3x3 depthwise / stride) -> 1x1
    project: MobileNetV2's stem and first block (no expansion), over an NCHW graph input."""
    rng = np.random.default_rng(seed)
    g = Graph("stem_block")
    x = g.add_input("x", TensorType("float32", (n, 3, h, w)))
    lo = g.constant(np.asarray(0.0, np.float32), "lo")
    hi = g.constant(np.asarray(6.0, np.float32), "hi")

    def activation(v, name):
        if act == "relu":
            return g.add_node("Relu", [v], 1, {}, name=name).output
        return g.add_node("Clip", [v, lo, hi], 1, {}, name=name).output

    y = activation(_conv(g, rng, x, 3, cexp, 3, stem_stride, "stem"), "a0")
    y = activation(_conv(g, rng, y, cexp, cexp, 3, stride, "dw", group=cexp), "a1")
    y = _conv(g, rng, y, cexp, cout, 1, 1, "project")
    g.add_output(y, "y")
    infer_shapes(g)
    return g, {"x": rng.standard_normal((n, 3, h, w)).astype(np.float32)}


STEM_CASES = [
    # (n, h, w, cexp, cout, stem stride, depthwise stride, act)
    (2, 64, 64, 32, 16, 2, 1, "clip"),   # MobileNetV2's stem and first block (scaled): 32 x 32 output
    (1, 37, 29, 32, 16, 2, 1, "clip"),   # odd image: a 19 x 15 stem output, partial tiles
    (2, 30, 34, 36, 5, 2, 2, "relu"),    # 36 channels (a second stage of four), stride-2 depthwise
    (1, 20, 22, 8, 32, 1, 1, "clip"),    # a stride-1 stem, eight channels, 32 outputs
    (3, 18, 18, 64, 24, 2, 1, "relu"),   # two full stages, three images
]


@pytest.mark.parametrize("case", STEM_CASES, ids=lambda c: "x".join(map(str, c)))
def test_stem_block_matches_oracle(case, hip_cache, monkeypatch):
    """The stem convolution, the depthwise convolution and the projection as one
    mgc_hip_mbconv_stem launch reading the NCHW input in place (the layout pass's input
    Transpose emits nothing)."""
    n, h, w, cexp, cout, s0, s1, act = case
    print(f"[gpu] stem block {case}", flush=True)
    g, feeds = stem_block(n, h, w, cexp, cout, s0, s1, act, seed=3 + sum(c for c in case if isinstance(c, int)))
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache, monkeypatch)
    assert kernels.get("mbconv_stem") == 1 and kernels.get("gemm") == 1, kernels
    # folded: the input Transpose, the stem and the depthwise convolution; the one transpose left
    # is the output's NHWC -> NCHW
    assert kernels.get("folded") == 3 and kernels.get("transpose") == 1, kernels
    assert "depthwise" not in kernels and "space_to_depth" not in kernels, kernels
    np.testing.assert_allclose(got["y"], expected, rtol=RTOL, atol=ATOL)


def test_stem_block_over_an_nhwc_caller_buffer(hip_cache, monkeypatch):
    """An NHWC image that is the caller's buffer, also 4 bytes off a 16-byte boundary: the stem
    block reads it through NHWC strides with four-byte loads, so the fused launch runs either
    way."""
    import torch

    print("[gpu] stem block over an NHWC caller buffer", flush=True)
    monkeypatch.setattr(hip_codegen, "MBCONV_MIN_ROWS", 0)
    rng = np.random.default_rng(11)
    g = Graph("nhwc_stem_block")
    x = g.add_input("x", TensorType("float32", (2, 27, 31, 3)))

    def conv(v, k, c_in, c_out, s, group, name, act):
        wt = g.constant((rng.standard_normal((k, k, c_in // group, c_out)) / np.sqrt(k * k * c_in / group))
                        .astype(np.float32), f"{name}_w")
        b = g.constant((rng.standard_normal(c_out) * 0.2).astype(np.float32), f"{name}_b")
        return g.add_node("FusedConv", [v, wt, b], 1,
                          {"kernel_shape": [k, k], "pads": [k // 2] * 4, "strides": [s, s], "group": group,
                           "layout": "NHWC", "activation": act, "clip_min": 0.0, "clip_max": 6.0}, name=name).output

    y = conv(x, 3, 3, 32, 2, 1, "stem", "clip")
    y = conv(y, 3, 32, 32, 1, 32, "dw", "clip")
    y = conv(y, 1, 32, 16, 1, 1, "pw", "none")
    g.add_output(y, "y")
    infer_shapes(g)
    feeds = {"x": rng.standard_normal((2, 27, 31, 3)).astype(np.float32)}
    expected = oracle.run_graph(g, feeds)["y"]
    model = compile_hip(g, hip_cache, "O0")
    try:
        assert model.report.kernels.get("mbconv_stem") == 1, model.report.kernels
        np.testing.assert_allclose(model.run(feeds)["y"], expected, rtol=RTOL, atol=ATOL)
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
