"""The ResNet stem as one launch (mgc_hip_conv_stem).

The stem is a 7 x 7, stride-2 convolution of the 3-channel image into 64 channels with its
folded BatchNorm and ReLU; the reference's C backend runs it as mgc_gemm over an
MGC_OP_CONV_NCHW operand (codegen/c.py:1099-1226, runtime/mgc_kernels.c:86-133, 370-396). The hip
backend reads the image window of each output tile in place (NCHW through its strides when the
layout pass's input Transpose brought it to NHWC, so that Transpose emits nothing) and runs the
contraction on MFMA from LDS. Graph cases compile a stem at O3 and compare with the oracle on the
unoptimized graph at the CNN bound (1e-4 absolute) and with the space-to-depth path it replaces;
shapes cover ResNet-50's 224 x 224 input, odd images whose last tiles are partial in both
directions, asymmetric padding, no padding, and each activation the emitter fuses. The C-ABI
cases call the entry point directly with the persistent workgroups capped at one and seven (so
one workgroup walks every tile through its prefetch loop, or tiles are dealt unevenly) and at
the library's choice, over an NHWC caller image with a padded output row stride, against a
float64 convolution, and check that shapes outside its limits are refused with MGC_ERR_ARGS.
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


def stem_graph(n: int, h: int, w: int, pads, act: str, seed: int) -> tuple[Graph, dict[str, np.ndarray]]:
    """image -> Conv 7 x 7 / 2 (3 -> 64) -> BatchNormalization -> activation, over NCHW."""
    rng = np.random.default_rng(seed)
    g = Graph("stem")
    x = g.add_input("x", TensorType("float32", (n, 3, h, w)))
    wt = g.constant((rng.standard_normal((64, 3, 7, 7)) * np.sqrt(2.0 / 147)).astype(np.float32), "w")
    y = g.add_node("Conv", [x, wt], 1, {"kernel_shape": [7, 7], "pads": list(pads), "strides": [2, 2]},
                   name="conv").output
    bn = [g.constant(v.astype(np.float32), name) for v, name in (
        (rng.uniform(0.5, 1.5, 64), "gamma"), (rng.normal(0, 0.1, 64), "beta"),
        (rng.normal(0, 0.1, 64), "mean"), (rng.uniform(0.5, 1.5, 64), "var"))]
    y = g.add_node("BatchNormalization", [y, *bn], 1, {"epsilon": 1e-5}, name="bn").output
    if act == "relu":
        y = g.add_node("Relu", [y], 1, {}, name="relu").output
    elif act == "clip":
        lo = g.constant(np.asarray(0.0, np.float32), "lo")
        hi = g.constant(np.asarray(6.0, np.float32), "hi")
        y = g.add_node("Clip", [y, lo, hi], 1, {}, name="clip").output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, {"x": rng.standard_normal((n, 3, h, w)).astype(np.float32)}


CASES = [
    # (n, h, w, pads [top, left, bottom, right], act)
    (2, 224, 224, (3, 3, 3, 3), "relu"),   # ResNet-50's stem: 112 x 112 output, whole tiles
    (1, 37, 29, (3, 3, 3, 3), "relu"),     # odd image: 19 x 15 output, partial tiles both ways
    (3, 64, 48, (2, 3, 3, 2), "clip"),     # asymmetric padding
    (1, 40, 70, (0, 0, 0, 0), "none"),     # no padding: 17 x 32 output
    (2, 31, 33, (3, 3, 3, 3), "none"),     # a tile row of one output pixel
]


def _run(g, feeds, cache, opt="O3"):
    model = compile_hip(g, cache, opt)
    try:
        return model.run(feeds), dict(model.report.kernels)
    finally:
        model.release()


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(str(v) for v in c[:3]) + f"-{c[4]}")
def test_stem_matches_oracle(case, hip_cache):
    n, h, w, pads, act = case
    print(f"[gpu] conv stem {case}", flush=True)
    g, feeds = stem_graph(n, h, w, pads, act, seed=h + w)
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache)
    assert kernels.get("gemm_stem") == 1 and "space_to_depth" not in kernels and "gemm" not in kernels, kernels
    # the input Transpose is read in place; the one transpose left is the output's NHWC -> NCHW
    assert kernels.get("transpose") == 1, kernels
    np.testing.assert_allclose(got["y"], expected, rtol=RTOL, atol=ATOL)


def test_stem_matches_space_to_depth_path(hip_cache, monkeypatch):
    """The same stem through the space-to-depth copy and the GEMM (the path this launch
    replaces) gives the same result within the bound."""
    print("[gpu] conv stem vs space-to-depth path", flush=True)
    g, feeds = stem_graph(2, 96, 80, (3, 3, 3, 3), "relu", seed=5)
    got, kernels = _run(g, feeds, hip_cache)
    assert kernels.get("gemm_stem") == 1, kernels
    monkeypatch.setattr(hip_codegen, "CONV_STEM", False)
    g2, _ = stem_graph(2, 96, 80, (3, 3, 3, 3), "relu", seed=5)
    ref, kernels2 = _run(g2, feeds, hip_cache)
    assert "gemm_stem" not in kernels2 and kernels2.get("space_to_depth") == 1, kernels2
    np.testing.assert_allclose(got["y"], ref["y"], rtol=RTOL, atol=ATOL)


def test_stem_over_nhwc_input(hip_cache):
    """An NHWC graph input (no Transpose to read through): the image is read with NHWC strides.
    The max pooling after it (as in ResNet) keeps the stem's output in the arena: a graph
    output may be a caller buffer of any alignment, so a stem writing one runs the
    space-to-depth path instead."""
    print("[gpu] conv stem over an NHWC input", flush=True)
    rng = np.random.default_rng(9)
    g = Graph("nhwc_stem")
    x = g.add_input("x", TensorType("float32", (2, 45, 51, 3)))
    wt = g.constant((rng.standard_normal((7, 7, 3, 64)) * 0.1).astype(np.float32), "w")
    b = g.constant((rng.standard_normal(64) * 0.2).astype(np.float32), "b")
    y = g.add_node("FusedConv", [x, wt, b], 1,
                   {"kernel_shape": [7, 7], "pads": [3, 3, 3, 3], "strides": [2, 2], "group": 1,
                    "layout": "NHWC", "activation": "relu"}, name="stem").output
    y = g.add_node("MaxPool", [y], 1, {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "strides": [2, 2],
                                       "layout": "NHWC"}, name="pool").output
    g.add_output(y, "y")
    infer_shapes(g)
    feeds = {"x": rng.standard_normal((2, 45, 51, 3)).astype(np.float32)}
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache, "O0")
    assert kernels.get("gemm_stem") == 1, kernels
    np.testing.assert_allclose(got["y"], expected, rtol=RTOL, atol=ATOL)


# -- the C ABI ---------------------------------------------------------------------------------
class StemArgs(ctypes.Structure):
    """mgc_hip_stem_args."""

    _fields_ = [("img", ctypes.c_void_p), ("C", ctypes.c_int), ("H", ctypes.c_int), ("W", ctypes.c_int),
                ("sn", ctypes.c_long), ("sc", ctypes.c_long), ("sh", ctypes.c_long), ("sw", ctypes.c_long)] + [
        (f, ctypes.c_int) for f in ("KH", "KW", "SH", "SW", "PT", "PL")]


class ConvStemArgs(ctypes.Structure):
    """mgc_hip_conv_stem_args."""

    _fields_ = [("w", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("out", ctypes.c_void_p), ("ldc", ctypes.c_long),
                ("N", ctypes.c_int), ("OH", ctypes.c_int), ("OW", ctypes.c_int), ("act", ctypes.c_int),
                ("lo", ctypes.c_float), ("hi", ctypes.c_float), ("workgroups", ctypes.c_int)]


def pack_weights(w_oihw: np.ndarray) -> np.ndarray:
    """The documented packing, written from its formula (an independent restatement of the
    emitter's transpose): w[((e 32 + l) 2 + h) 2 + b] = W[32 b + l][c][i][2 q + h], e = (c 7 + i) 4 + q."""
    out = np.zeros(84 * 128, np.float32)
    for c in range(3):
        for i in range(7):
            for q in range(4):
                e = (c * 7 + i) * 4 + q
                for lane in range(32):
                    for half in range(2):
                        j = 2 * q + half
                        if j >= 7:
                            continue
                        for blk in range(2):
                            out[((e * 32 + lane) * 2 + half) * 2 + blk] = w_oihw[32 * blk + lane, c, i, j]
    return out


@pytest.fixture(scope="module")
def capi():
    lib = load_kernel_library()
    bind(lib)
    lib.mgc_hip_conv_stem.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.mgc_hip_conv_stem_weight_floats.restype = ctypes.c_long
    hip = Hip()
    x = lib.mgc_hip_exec_create(None)
    assert x, lib.mgc_hip_last_error()
    yield lib, hip, x
    lib.mgc_hip_exec_destroy(x)
    hip.free()


@pytest.mark.parametrize("workgroups", [0, 1, 7])
def test_stem_entry_point(capi, workgroups):
    """NHWC caller image of 2 x 53 x 38, pads (3, 2), output rows of 68 floats (channels 64..67
    must stay untouched), each activation the entry point applies; the persistent workgroups
    capped at one (every tile through one workgroup's prefetch loop) and at seven (tiles dealt
    unevenly) as well as the library's choice."""
    lib, hip, x = capi
    assert lib.mgc_hip_conv_stem_weight_floats() == 84 * 128
    rng = np.random.default_rng(20 + workgroups)
    n, h, w, pt, pl, ldc = 2, 53, 38, 3, 2, 68
    oh, ow = (h + 2 * pt - 7) // 2 + 1, (w + 2 * pl - 7) // 2 + 1
    img = rng.standard_normal((n, h, w, 3)).astype(np.float32)
    wt = (rng.standard_normal((64, 3, 7, 7)) * 0.1).astype(np.float32)
    bias = (rng.standard_normal(64) * 0.3).astype(np.float32)
    conv = oracle.conv_nchw(img.transpose(0, 3, 1, 2).astype(np.float64), wt.astype(np.float64),
                            bias.astype(np.float64), {"kernel_shape": [7, 7], "strides": [2, 2],
                                                      "pads": [pt, pl, pt, pl]}).transpose(0, 2, 3, 1)
    assert conv.shape == (n, oh, ow, 64)
    st = StemArgs(img=hip.upload(img), C=3, H=h, W=w, sn=h * w * 3, sc=1, sh=w * 3, sw=3, KH=7, KW=7, SH=2, SW=2,
                  PT=pt, PL=pl)
    wbuf, bbuf = hip.upload(pack_weights(wt)), hip.upload(bias)
    out = hip.alloc(4 * n * oh * ow * ldc)
    for act in ("none", "relu", "clip"):
        hip.put(out, np.full(n * oh * ow * ldc, np.nan, np.float32))
        a = ConvStemArgs(w=wbuf, bias=bbuf, out=out, ldc=ldc, N=n, OH=oh, OW=ow, act=ACTS.index(act), lo=-0.5,
                         hi=0.75, workgroups=workgroups)
        lib.mgc_hip_conv_stem(x, ctypes.byref(st), ctypes.byref(a))
        assert lib.mgc_hip_exec_status(x) == MGC_OK, lib.mgc_hip_last_error()
        got = hip.download(out, (n, oh, ow, ldc))
        want = oracle.activation(conv, {"activation": act, "clip_min": -0.5, "clip_max": 0.75})
        np.testing.assert_allclose(got[..., :64], want, rtol=RTOL, atol=ATOL, err_msg=act)
        assert np.isnan(got[..., 64:]).all(), "wrote past the 64 channels of a pixel"


def test_stem_entry_point_refuses_unsupported(capi):
    lib, hip, x = capi
    img = hip.upload(np.zeros((1, 4, 16, 16), np.float32))
    wbuf, out = hip.alloc(4 * 84 * 128), hip.alloc(4 * 64 * 64)
    ok = dict(C=3, H=16, W=16, sn=4 * 256, sc=256, sh=16, sw=1, KH=7, KW=7, SH=2, SW=2, PT=3, PL=3)
    for bad in (dict(C=4), dict(KH=5), dict(SW=1), dict(PT=-1)):
        st = StemArgs(img=img, **{**ok, **bad})
        a = ConvStemArgs(w=wbuf, out=out, ldc=64, N=1, OH=8, OW=8, act=0, workgroups=0)
        lib.mgc_hip_conv_stem(x, ctypes.byref(st), ctypes.byref(a))
        assert lib.mgc_hip_exec_status(x) == MGC_ERR_ARGS, bad
    st = StemArgs(img=img, **ok)
    for bad in (dict(ldc=62), dict(workgroups=-1)):
        a = ConvStemArgs(**{**dict(w=wbuf, out=out, ldc=64, N=1, OH=8, OW=8, act=0, workgroups=0), **bad})
        lib.mgc_hip_conv_stem(x, ctypes.byref(st), ctypes.byref(a))
        assert lib.mgc_hip_exec_status(x) == MGC_ERR_ARGS, bad
