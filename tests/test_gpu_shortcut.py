"""Projection shortcuts computed inside the GEMM of a residual block's last convolution.

A ResNet downsample block (the reference's resnet50 builder, src/ml_graph_compiler/models.py,
and its C backend's one conv call per node, codegen/c_backend.py) adds a 1 x 1 strided
convolution of the block input x to the output of the block's last 1 x 1 convolution c3. The
hip backend runs both as one GEMM with K = K1 + C2: columns below K1 read c3's input, the
others read x at the shortcut's stride. Each case builds such a block, compiles it at O3,
asserts how many blocks were fused and compares with the oracle on the unoptimized graph; the
shapes reach the 64 x 64 and 128 x 32 DMA tiles and the 32 x 32 and 16 x 16 wave-split
kernels. The same blocks compiled with the fusion off give the reference's two-GEMM form; both
must agree with the oracle to the same bound. When the two GEMM inputs are caller buffers the
generated code checks their 16-byte alignment at run time and runs the two GEMMs apart if
either is misaligned; both branches are run.
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


def _conv(g: Graph, rng, x, cin: int, cout: int, k: int, stride: int, name: str, bias: bool = True):
    w = g.constant((rng.standard_normal((cout, cin, k, k)) / np.sqrt(cin * k * k)).astype(np.float32), f"{name}_w")
    ins = [x, w]
    if bias:
        ins.append(g.constant(rng.standard_normal(cout).astype(np.float32) * 0.2, f"{name}_b"))
    attrs = {"kernel_shape": [k, k], "pads": [k // 2] * 4, "strides": [stride, stride]}
    return g.add_node("Conv", ins, 1, attrs, name=name).output


def downsample_block(n: int, cin: int, cmid: int, cout: int, hw: int, stride: int, act: str = "relu",
                     ds_bias: bool = True, seed: int = 0) -> tuple[Graph, dict[str, np.ndarray]]:
    """x -> relu(c1 1x1) -> relu(c2 3x3 / stride) -> c3 1x1, plus ds 1x1 / stride of x, then act."""
    rng = np.random.default_rng(seed)
    g = Graph("downsample")
    x = g.add_input("x", TensorType("float32", (n, cin, hw, hw)))
    y = g.add_node("Relu", [_conv(g, rng, x, cin, cmid, 1, 1, "c1")], 1, {}, name="r1").output
    y = g.add_node("Relu", [_conv(g, rng, y, cmid, cmid, 3, stride, "c2")], 1, {}, name="r2").output
    y = _conv(g, rng, y, cmid, cout, 1, 1, "c3")
    d = _conv(g, rng, x, cin, cout, 1, stride, "ds", bias=ds_bias)
    y = g.add_node("Add", [y, d], 1, {}, name="add").output
    if act == "relu":
        y = g.add_node("Relu", [y], 1, {}, name="act").output
    elif act == "clip":
        lo = g.constant(np.asarray(0.0, np.float32), "lo")
        hi = g.constant(np.asarray(0.75, np.float32), "hi")
        y = g.add_node("Clip", [y, lo, hi], 1, {}, name="act").output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, {"x": rng.standard_normal((n, cin, hw, hw)).astype(np.float32)}


CASES = [
    # (n, cin, cmid, cout, hw, stride)
    (1, 64, 64, 256, 56, 1),      # ResNet-50 layer1: 64 x 64 tiles, stride 1 shortcut
    (1, 256, 128, 512, 28, 2),    # layer2 at batch 1
    (2, 512, 256, 1024, 14, 2),   # layer3, two images
    (1, 1024, 512, 2048, 14, 2),  # layer4 at batch 1: 49 rows, K = 1536
    (3, 12, 32, 40, 9, 2),        # odd sizes: 5 x 5 output, N = 40 (128 x 32 tiles)
    (1, 4, 32, 8, 5, 1),          # four input channels, eight outputs
]


def _run(g: Graph, feeds, cache, fuse: bool, monkeypatch) -> tuple[dict[str, np.ndarray], dict[str, int]]:
    monkeypatch.setattr(hip_codegen, "FUSE_PROJECTION_SHORTCUT", fuse)
    model = compile_hip(g, cache, "O3")
    try:
        return model.run(feeds), dict(model.report.kernels)
    finally:
        model.release()


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_shortcut_fused_matches_oracle(case, hip_cache, monkeypatch):
    n, cin, cmid, cout, hw, stride = case
    print(f"[gpu] shortcut block {case}", flush=True)
    g, feeds = downsample_block(n, cin, cmid, cout, hw, stride, seed=sum(case))
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache, True, monkeypatch)
    assert kernels.get("gemm_shortcut") == 1, kernels
    np.testing.assert_allclose(got["y"], expected, rtol=RTOL, atol=ATOL)
    g2, _ = downsample_block(n, cin, cmid, cout, hw, stride, seed=sum(case))
    unfused, kernels = _run(g2, feeds, hip_cache, False, monkeypatch)
    assert "gemm_shortcut" not in kernels
    np.testing.assert_allclose(unfused["y"], expected, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("act, ds_bias", [("none", True), ("clip", False), ("relu", False)])
def test_shortcut_epilogues(act, ds_bias, hip_cache, monkeypatch):
    """The block's activation (or none) and a shortcut without a bias of its own."""
    print(f"[gpu] shortcut epilogue {act} ds_bias={ds_bias}", flush=True)
    g, feeds = downsample_block(2, 64, 64, 128, 16, 2, act=act, ds_bias=ds_bias, seed=7)
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache, True, monkeypatch)
    assert kernels.get("gemm_shortcut") == 1, kernels
    np.testing.assert_allclose(got["y"], expected, rtol=RTOL, atol=ATOL)


def test_shortcut_not_fused_when_k1_is_ragged(hip_cache, monkeypatch):
    """K1 = 48 is not a whole number of 32-wide K stages: the block runs as two GEMMs."""
    g, feeds = downsample_block(1, 64, 48, 128, 12, 2, seed=3)
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache, True, monkeypatch)
    assert "gemm_shortcut" not in kernels
    np.testing.assert_allclose(got["y"], expected, rtol=RTOL, atol=ATOL)


def _nhwc_block(n: int, h: int, c2: int, k1: int, cout: int, stride: int, seed: int):
    """An already-NHWC block whose two GEMM inputs are caller buffers: a (the last conv's
    input) and x (the shortcut's input) are graph inputs, so the generated code checks their
    alignment at run time."""
    rng = np.random.default_rng(seed)
    oh = (h - 1) // stride + 1
    g = Graph("nhwc_block")
    a = g.add_input("a", TensorType("float32", (n, oh, oh, k1)))
    x = g.add_input("x", TensorType("float32", (n, h, h, c2)))
    wd = g.constant((rng.standard_normal((1, 1, c2, cout)) / np.sqrt(c2)).astype(np.float32), "wd")
    bd = g.constant(rng.standard_normal(cout).astype(np.float32), "bd")
    w3 = g.constant((rng.standard_normal((1, 1, k1, cout)) / np.sqrt(k1)).astype(np.float32), "w3")
    b3 = g.constant(rng.standard_normal(cout).astype(np.float32), "b3")
    common = {"kernel_shape": [1, 1], "pads": [0, 0, 0, 0], "layout": "NHWC"}
    d = g.add_node("FusedConv", [x, wd, bd], 1, {**common, "strides": [stride, stride], "activation": "none"},
                   name="ds").output
    y = g.add_node("FusedConv", [a, w3, b3, d], 1, {**common, "strides": [1, 1], "activation": "relu"},
                   name="c3").output
    g.add_output(y, "y")
    infer_shapes(g)
    feeds = {"a": rng.standard_normal((n, oh, oh, k1)).astype(np.float32),
             "x": rng.standard_normal((n, h, h, c2)).astype(np.float32)}
    return g, feeds


def test_shortcut_over_caller_buffers(hip_cache, monkeypatch):
    print("[gpu] shortcut over caller buffers", flush=True)
    monkeypatch.setattr(hip_codegen, "FUSE_PROJECTION_SHORTCUT", True)
    g, feeds = _nhwc_block(2, 14, 256, 128, 512, 2, seed=11)
    expected = oracle.run_graph(g, feeds)["y"]
    model = compile_hip(g, hip_cache, "O0")
    try:
        assert model.report.kernels.get("gemm_shortcut") == 1, model.report.kernels
        got = model.run(feeds)["y"]
    finally:
        model.release()
    np.testing.assert_allclose(got, expected, rtol=RTOL, atol=ATOL)


def test_shortcut_over_misaligned_caller_buffers(hip_cache, monkeypatch):
    """Caller buffers 4 bytes off a 16-byte boundary: the generated code sees the misalignment at
    run time and runs the shortcut and the last convolution as two GEMMs instead."""
    import torch

    print("[gpu] shortcut over misaligned caller buffers", flush=True)
    monkeypatch.setattr(hip_codegen, "FUSE_PROJECTION_SHORTCUT", True)
    g, feeds = _nhwc_block(1, 14, 64, 64, 256, 2, seed=13)
    expected = oracle.run_graph(g, feeds)["y"]
    model = compile_hip(g, hip_cache, "O0")
    try:
        assert model.report.kernels.get("gemm_shortcut") == 1, model.report.kernels
        dev = torch.device("cuda:0")
        keep = []
        ptrs = []
        for name, _ in model.inputs:
            host = torch.from_numpy(np.ascontiguousarray(feeds[name]).reshape(-1))
            buf = torch.zeros(host.numel() + 1, dtype=torch.float32, device=dev)
            view = buf[1:]  # 4 bytes past the allocation's start
            view.copy_(host)
            assert view.data_ptr() % 16 == 4
            keep.append(buf)
            ptrs.append(view.data_ptr())
        out = torch.empty(expected.size, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        model.run_device(ptrs, [out.data_ptr()])
        got = out.cpu().numpy().reshape(expected.shape)
    finally:
        model.release()
    np.testing.assert_allclose(got, expected, rtol=RTOL, atol=ATOL)
