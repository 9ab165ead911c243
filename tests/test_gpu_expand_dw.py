"""An inverted-residual block's expansion and depthwise convolution as one launch
(mgc_hip_expand_dw).

A MobileNetV2 block with expansion t > 1 (the reference's C backend runs it as mgc_gemm,
mgc_depthwise_nhwc and mgc_gemm with both intermediates in its arena, codegen/c.py:1102-1226)
expands the input with a 1 x 1 convolution and ReLU6 and filters every expanded channel with a
3 x 3 depthwise convolution (stride 1 or 2) and ReLU6 before the 1 x 1 projection. On small
images the hip backend runs the first two as one launch, a workgroup per image and 32 expanded
channels with the expanded tensor only in LDS, and stores the depthwise output for the
projection GEMM. Each case builds such a block, compiles it at O3 with the workgroup threshold
lifted (EXPAND_DW_MIN_WORKGROUPS = 0) and the depthwise -> projection fusion off, asserts that
the pair became one expand_depthwise launch next to the projection's GEMM, and compares with
the oracle on the unoptimized graph. Shapes reach every input width the kernel takes (64, 96,
160 channels), both strides, MobileNetV2's 14 x 14 and 7 x 7 blocks, odd and non-square images
whose last 16-pixel row block is partial, the largest windows (255 of 256 pixels; 224 image
pixels, four row blocks per wave), expanded widths of one to thirty 32-channel slices, ReLU and
ReLU6, with and without the residual. When the block input or the depthwise output is a caller
buffer the generated code checks its alignment at run time and runs the two convolutions apart
if it is misaligned; both branches are run.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip
from ml_graph_compiler.codegen import hip as hip_codegen
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle
from test_gpu_mbconv import block

pytestmark = pytest.mark.gpu

RTOL = ATOL = 3e-5

CASES = [
    # (n, cin, cexp, cout, h, w, stride, act)
    (2, 64, 384, 64, 14, 14, 1, "clip"),    # MobileNetV2's 14 x 14 block with its residual
    (1, 96, 576, 96, 14, 14, 1, "clip"),    # the 96-channel block
    (2, 96, 576, 160, 14, 14, 2, "clip"),   # the 14 -> 7 block at stride 2
    (2, 160, 960, 160, 7, 7, 1, "clip"),    # the 7 x 7 block: thirty slices
    (1, 64, 128, 64, 13, 11, 1, "relu"),    # odd, non-square: 143 pixels, the last row block partial
    (1, 96, 64, 32, 9, 15, 2, "relu"),      # stride 2 over a non-square image: 5 x 8 output
    (3, 160, 32, 16, 5, 6, 1, "clip"),      # one slice, 30 pixels
    (1, 64, 32, 8, 16, 14, 2, "clip"),      # 224 pixels (four row blocks per wave), a 17 x 15 window
]


def _run(g: Graph, feeds, cache, monkeypatch, opt: str = "O3") -> tuple[dict[str, np.ndarray], dict[str, int]]:
    monkeypatch.setattr(hip_codegen, "EXPAND_DW_MIN_WORKGROUPS", 0)
    monkeypatch.setattr(hip_codegen, "FUSE_DEPTHWISE_POINTWISE", False)
    model = compile_hip(g, cache, opt)
    try:
        return model.run(feeds), dict(model.report.kernels)
    finally:
        model.release()


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_expansion_and_depthwise_match_oracle(case, hip_cache, monkeypatch):
    n, cin, cexp, cout, h, w, stride, act = case
    print(f"[gpu] expansion + depthwise {case}", flush=True)
    g, feeds = block(n, cin, cexp, cout, h, w, stride, act, seed=3 + sum(c for c in case if isinstance(c, int)))
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache, monkeypatch)
    assert kernels.get("expand_depthwise") == 1 and "depthwise" not in kernels, kernels
    assert kernels.get("gemm") == 1 and "gemm_mbconv" not in kernels, kernels  # the projection's
    np.testing.assert_allclose(got["y"], expected, rtol=RTOL, atol=ATOL)


def _nhwc_pair(n: int, h: int, cin: int, cexp: int, stride: int, seed: int):
    """An NHWC expansion -> depthwise pair whose input and output are graph values, so the
    generated code checks both alignments."""
    rng = np.random.default_rng(seed)
    g = Graph("nhwc_pair")
    x = g.add_input("x", TensorType("float32", (n, h, h, cin)))

    def conv(v, k, c_in, c_out, s, group, name):
        w = g.constant((rng.standard_normal((k, k, c_in // group, c_out)) / np.sqrt(k * k * c_in / group))
                       .astype(np.float32), f"{name}_w")
        b = g.constant((rng.standard_normal(c_out) * 0.2).astype(np.float32), f"{name}_b")
        return g.add_node("FusedConv", [v, w, b], 1,
                          {"kernel_shape": [k, k], "pads": [k // 2] * 4, "strides": [s, s], "group": group,
                           "layout": "NHWC", "activation": "clip", "clip_min": 0.0, "clip_max": 6.0},
                          name=name).output

    y = conv(x, 1, cin, cexp, 1, 1, "ex")
    y = conv(y, 3, cexp, cexp, stride, cexp, "dw")
    g.add_output(y, "y")
    infer_shapes(g)
    return g, {"x": rng.standard_normal((n, h, h, cin)).astype(np.float32)}


def test_expansion_and_depthwise_over_caller_buffers(hip_cache, monkeypatch):
    """The pair's input and output are the caller's buffers: aligned, the fused launch runs; the
    input or the output 4 bytes off a 16-byte boundary, the generated code runs the two
    convolutions apart instead."""
    import torch

    print("[gpu] expansion + depthwise over caller buffers", flush=True)
    monkeypatch.setattr(hip_codegen, "EXPAND_DW_MIN_WORKGROUPS", 0)
    g, feeds = _nhwc_pair(2, 14, 96, 192, 2, seed=8)
    expected = oracle.run_graph(g, feeds)["y"]
    model = compile_hip(g, hip_cache, "O0")
    try:
        assert model.report.kernels.get("expand_depthwise") == 1, model.report.kernels
        np.testing.assert_allclose(model.run(feeds)["y"], expected, rtol=RTOL, atol=ATOL)
        dev = torch.device("cuda:0")
        host = torch.from_numpy(np.ascontiguousarray(feeds["x"]).reshape(-1))
        for shift_in, shift_out in ((1, 0), (0, 1), (0, 0)):
            inp = torch.zeros(host.numel() + 4, dtype=torch.float32, device=dev)
            xin = inp[shift_in:shift_in + host.numel()]
            xin.copy_(host)
            out = torch.full((expected.size + 4,), float("nan"), dtype=torch.float32, device=dev)
            yout = out[shift_out:shift_out + expected.size]
            assert xin.data_ptr() % 16 == 4 * shift_in and yout.data_ptr() % 16 == 4 * shift_out
            torch.cuda.synchronize()
            model.run_device([xin.data_ptr()], [yout.data_ptr()])
            got = yout.cpu().numpy().reshape(expected.shape)
            np.testing.assert_allclose(got, expected, rtol=RTOL, atol=ATOL, err_msg=f"shifts {shift_in}, {shift_out}")
    finally:
        model.release()


def test_mobilenet_v2_blocks_fused_and_apart_agree(hip_cache, monkeypatch):
    """MobileNetV2 at batch 32 (its ten 14 x 14 and 7 x 7 expanded blocks fused) against the same
    model with the fusion off: the same depthwise inputs up to the expansion's summation order."""
    from helpers import compile_hip as build
    from ml_graph_compiler import builders

    print("[gpu] mobilenet_v2 b32 with and without expansion + depthwise", flush=True)
    rng = np.random.default_rng(11)
    feeds = {"image": rng.standard_normal((32, 3, 224, 224)).astype(np.float32)}
    outs = {}
    for fused in (True, False):
        monkeypatch.setattr(hip_codegen, "FUSE_EXPAND_DEPTHWISE", fused)
        model = build(builders.mobilenet_v2(batch=32), hip_cache, "O3")
        try:
            assert model.report.kernels.get("expand_depthwise", 0) == (10 if fused else 0), model.report.kernels
            outs[fused] = next(iter(model.run(feeds).values()))
        finally:
            model.release()
    scale = float(np.abs(outs[False]).max())
    np.testing.assert_allclose(outs[True], outs[False], rtol=0, atol=1e-5 * max(scale, 1.0))
    assert (outs[True].argmax(axis=1) == outs[False].argmax(axis=1)).all()
