"""Global average pooling and the fully connected layer that reads it as one launch
(mgc_hip_pool_fc).

ResNet-50, MobileNetV2 and the tiny CNN end GlobalAveragePool -> Flatten -> Gemm; the reference's
C backend runs mgc_reduce_mid's mean (codegen/c.py:1255-1270, runtime/mgc_kernels.c:593-612) and
then mgc_gemm for the classifier (c.py:974-1003). At batch 1-4 the hip backend runs both in one
launch whose workgroups each pool their image into LDS and form 16 of the dot products. Graph
cases compile a convolution -> pooling -> classifier graph at O3, assert the fused launch (or,
above POOL_FC_MAX_BATCH images, the two launches) and compare with the oracle on the unoptimized
graph and with the unfused hip launches. Shapes cover ResNet-50's and MobileNetV2's heads (2048 and
1280 channels of 7 x 7, 1000 classes), odd pixel counts and class counts that end a 16-output
workgroup early, one pixel (C / 4 = 3 quads, so 341 pixel parts of which one does any work),
the 4096-channel limit, both Gemm weight layouts and each activation. The C-ABI cases call the
entry point directly over caller buffers with a padded output row stride (the padding must stay
untouched), with and without a bias, against float64 sums, and check that shapes and alignments
outside its limits are refused with MGC_ERR_ARGS.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from capi import ACTS, MGC_ERR_ARGS, MGC_OK, Hip, bind
from helpers import compile_hip
from ml_graph_compiler.codegen import hip as hip_codegen
from ml_graph_compiler.codegen.build import load_kernel_library
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu

ATOL = 1e-4
RTOL = 1e-5


def head_graph(n: int, cin: int, c: int, h: int, w: int, f: int, trans_b: int, act: str,
               seed: int) -> tuple[Graph, dict[str, np.ndarray]]:
    """image -> 1 x 1 Conv (cin -> c) -> Relu -> GlobalAveragePool -> Flatten -> Gemm (-> act)."""
    rng = np.random.default_rng(seed)
    g = Graph("head")
    x = g.add_input("x", TensorType("float32", (n, cin, h, w)))
    wc = g.constant((rng.standard_normal((c, cin, 1, 1)) / np.sqrt(cin)).astype(np.float32), "wc")
    bc = g.constant((rng.standard_normal(c) * 0.1).astype(np.float32), "bc")
    y = g.add_node("Conv", [x, wc, bc], 1, {"kernel_shape": [1, 1], "pads": [0, 0, 0, 0], "strides": [1, 1]},
                   name="conv").output
    y = g.add_node("Relu", [y], 1, {}, name="relu").output
    y = g.add_node("GlobalAveragePool", [y], 1, {}, name="gap").output
    y = g.add_node("Flatten", [y], 1, {"axis": 1}, name="flatten").output
    wf = (rng.standard_normal((f, c)) / np.sqrt(c)).astype(np.float32)
    wfc = g.constant(wf if trans_b else np.ascontiguousarray(wf.T), "wfc")
    bfc = g.constant((rng.standard_normal(f) * 0.2).astype(np.float32), "bfc")
    y = g.add_node("Gemm", [y, wfc, bfc], 1, {"transB": trans_b}, name="fc").output
    if act == "relu":
        y = g.add_node("Relu", [y], 1, {}, name="fc_relu").output
    elif act == "clip":
        lo = g.constant(np.asarray(-0.25, np.float32), "lo")
        hi = g.constant(np.asarray(0.5, np.float32), "hi")
        y = g.add_node("Clip", [y, lo, hi], 1, {}, name="fc_clip").output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, {"x": rng.standard_normal((n, cin, h, w)).astype(np.float32)}


CASES = [
    # (n, cin, c, h, w, f, trans_b, act)
    (1, 64, 2048, 7, 7, 1000, 1, "none"),   # ResNet-50's head at batch 1
    (2, 32, 1280, 7, 7, 1000, 1, "none"),   # MobileNetV2's head at batch 2
    (3, 16, 64, 5, 3, 10, 0, "relu"),       # 15 pixels, 10 classes: one partial workgroup; [C][F] weights
    (4, 8, 4096, 2, 2, 37, 1, "clip"),      # the channel limit, four images
    (1, 8, 12, 1, 1, 5, 0, "none"),         # one pixel, three channel quads
]


def _compile(g, cache, fuse: bool, monkeypatch):
    monkeypatch.setattr(hip_codegen, "FUSE_POOL_FC", fuse)
    return compile_hip(g, cache, "O3")


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_pool_fc_matches_oracle(case, hip_cache, monkeypatch):
    n, cin, c, h, w, f, trans_b, act = case
    print(f"[gpu] pooling + classifier {case}", flush=True)
    g, feeds = head_graph(n, cin, c, h, w, f, trans_b, act, seed=sum(case[:6]))
    expected = oracle.run_graph(g, feeds)["y"]
    model = _compile(g, hip_cache, True, monkeypatch)
    try:
        assert model.report.kernels.get("pool_fc") == 1 and "reduce" not in model.report.kernels, model.report.kernels
        got = model.run(feeds)["y"]
    finally:
        model.release()
    np.testing.assert_allclose(got, expected, rtol=RTOL, atol=ATOL)
    g2, _ = head_graph(n, cin, c, h, w, f, trans_b, act, seed=sum(case[:6]))
    model = _compile(g2, hip_cache, False, monkeypatch)
    try:
        assert "pool_fc" not in model.report.kernels and model.report.kernels.get("reduce") == 1
        apart = model.run(feeds)["y"]
    finally:
        model.release()
    np.testing.assert_allclose(got, apart, rtol=RTOL, atol=ATOL)


def test_pool_fc_not_above_its_batch_limit(hip_cache, monkeypatch):
    n = hip_codegen.POOL_FC_MAX_BATCH + 1
    print(f"[gpu] pooling + classifier at batch {n} (two launches)", flush=True)
    g, feeds = head_graph(n, 16, 256, 3, 3, 20, 1, "none", seed=9)
    expected = oracle.run_graph(g, feeds)["y"]
    model = _compile(g, hip_cache, True, monkeypatch)
    try:
        assert "pool_fc" not in model.report.kernels and model.report.kernels.get("reduce") == 1
        got = model.run(feeds)["y"]
    finally:
        model.release()
    np.testing.assert_allclose(got, expected, rtol=RTOL, atol=ATOL)


class PoolFcArgs(ctypes.Structure):
    """mgc_hip_pool_fc_args."""

    _fields_ = [
        ("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("out", ctypes.c_void_p),
        ("ldo", ctypes.c_long), ("N", ctypes.c_int), ("P", ctypes.c_int), ("C", ctypes.c_int), ("F", ctypes.c_int),
        ("act", ctypes.c_int), ("lo", ctypes.c_float), ("hi", ctypes.c_float),
    ]


@pytest.fixture
def capi():
    lib = load_kernel_library()
    bind(lib)
    lib.mgc_hip_pool_fc.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.mgc_hip_pool_fc_supported.restype = ctypes.c_int
    lib.mgc_hip_pool_fc_supported.argtypes = [ctypes.c_int] * 4
    hip = Hip()
    x = lib.mgc_hip_exec_create(None)
    assert x, lib.mgc_hip_last_error()
    yield lib, hip, x
    lib.mgc_hip_exec_destroy(x)
    hip.free()


def _reference(img: np.ndarray, wt: np.ndarray, bias: np.ndarray | None, act: str) -> np.ndarray:
    pooled = img.astype(np.float64).mean(axis=1)
    y = pooled @ wt.astype(np.float64).T
    if bias is not None:
        y = y + bias
    return oracle.activation(y, {"activation": act, "clip_min": -0.3, "clip_max": 0.4})


@pytest.mark.parametrize("with_bias", [True, False])
def test_pool_fc_entry_point(capi, with_bias):
    """3 images of 11 pixels x 520 channels (130 quads: seven pixel parts, four of two pixels and
    three of one), 75 outputs in rows of 80 floats (columns 75..79 must stay untouched)."""
    lib, hip, x = capi
    rng = np.random.default_rng(31 + with_bias)
    n, p, c, f, ldo = 3, 11, 520, 75, 80
    img = rng.standard_normal((n, p, c)).astype(np.float32)
    wt = (rng.standard_normal((f, c)) / np.sqrt(c)).astype(np.float32)
    bias = (rng.standard_normal(f) * 0.3).astype(np.float32) if with_bias else None
    xb, wb = hip.upload(img), hip.upload(wt)
    bb = hip.upload(bias) if with_bias else None
    out = hip.alloc(4 * n * ldo)
    assert lib.mgc_hip_pool_fc_supported(n, p, c, f) == 1
    for act in ("none", "relu", "clip"):
        hip.put(out, np.full(n * ldo, np.nan, np.float32))
        a = PoolFcArgs(x=xb, w=wb, bias=bb, out=out, ldo=ldo, N=n, P=p, C=c, F=f, act=ACTS.index(act), lo=-0.3, hi=0.4)
        lib.mgc_hip_pool_fc(x, ctypes.byref(a))
        assert lib.mgc_hip_exec_status(x) == MGC_OK, lib.mgc_hip_last_error()
        got = hip.download(out, (n, ldo))
        np.testing.assert_allclose(got[:, :f], _reference(img, wt, bias, act), rtol=RTOL, atol=ATOL, err_msg=act)
        assert np.isnan(got[:, f:]).all(), "wrote past the F outputs of a row"


def test_pool_fc_entry_point_refuses_unsupported(capi):
    lib, hip, x = capi
    xb, wb, out = hip.alloc(4 * 4 * 5000), hip.alloc(4 * 8 * 5000), hip.alloc(4 * 64)
    ok = dict(x=xb, w=wb, bias=None, out=out, ldo=8, N=1, P=4, C=64, F=8, act=0, lo=0.0, hi=0.0)
    assert lib.mgc_hip_pool_fc_supported(1, 4, 64, 8) == 1
    for bad in (dict(C=66), dict(C=4100), dict(ldo=7), dict(x=xb + 4), dict(w=wb + 8), dict(P=0)):
        a = PoolFcArgs(**{**ok, **bad})
        lib.mgc_hip_pool_fc(x, ctypes.byref(a))
        assert lib.mgc_hip_exec_status(x) == MGC_ERR_ARGS, bad
    assert lib.mgc_hip_pool_fc_supported(1, 4, 66, 8) == 0 and lib.mgc_hip_pool_fc_supported(1, 4, 4100, 8) == 0
    a = PoolFcArgs(**{**ok, "N": 0})  # no images: nothing to do
    lib.mgc_hip_pool_fc(x, ctypes.byref(a))
    assert lib.mgc_hip_exec_status(x) == MGC_OK, lib.mgc_hip_last_error()
