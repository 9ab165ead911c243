"""Pins the numpy oracle before it is trusted as the GPU checker.

Each check is chosen so a plausible slip (dropped term, wrong sign or index, transposed
operand, off-by-one window) fails: the reference's known answers (erf accuracy, truncating
integer division, first-max argmax, Gather wrap/raise), brute-force loops for convolution and
pooling on small inputs, textbook float64 formulas for softmax/LayerNorm/GELU, and the
reference's own C kernels (oracle/_ref, built from /root/reference) run on whole graphs.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

from helpers import named_graph
from ml_graph_compiler import builders
from ml_graph_compiler.passes import optimize
from ml_graph_compiler.schedule import schedule
from oracle import interpreter as oracle

rng = np.random.default_rng(7)
HAVE_REFERENCE = Path("/root/reference/src/ml_graph_compiler/codegen/runtime/mgc_kernels.c").exists()


def run1(op, inputs, attrs=None, const=(), n_out=1):
    names = [f"i{k}" for k in range(len(inputs))]
    ins, inits = [], []
    for k, a in enumerate(inputs):
        if a is None:
            names[k] = ""
        elif k in const:
            inits.append((names[k], a))
        else:
            ins.append((names[k], a.shape, str(a.dtype) if a.dtype != np.bool_ else "bool"))
    outs = [f"o{k}" for k in range(n_out)]
    g = named_graph([(op, names, outs, attrs or {})], ins, outs, inits)
    feeds = {n: a for n, a in zip(names, inputs) if n and int(n[1:]) not in const}
    return oracle.run_graph(g, feeds)


def test_erf_matches_math_erf():
    """Reference known answer: error < 2e-7 on linspace(-6, 6, 2001) (tests/test_ops.py:108-113)."""
    x = np.linspace(-6, 6, 2001)
    got = oracle.erf(x)
    assert np.max(np.abs(got - np.array([math.erf(v) for v in x]))) < 2e-7


def test_integer_division_truncates():
    """Reference known answer: [7, -7, 9] / [2, 2, -4] = [3, -3, -2] (tests/test_ops.py:90-93)."""
    out = run1("Div", [np.asarray([7, -7, 9], np.int64), np.asarray([2, 2, -4], np.int64)])["o0"]
    np.testing.assert_array_equal(out, [3, -3, -2])
    assert out.dtype == np.int64


def test_argmax_takes_first_maximum_and_gather_wraps():
    x = np.asarray([[1.0, 3.0, 3.0, 0.0], [5.0, 5.0, 1.0, 5.0]], np.float32)
    np.testing.assert_array_equal(run1("ArgMax", [x], {"axis": 1, "keepdims": 0})["o0"], [1, 0])
    table = np.arange(12, dtype=np.float32).reshape(4, 3)
    out = run1("Gather", [table, np.asarray([-1, 0], np.int64)], {"axis": 0})["o0"]
    np.testing.assert_array_equal(out, table[[3, 0]])
    with pytest.raises(oracle.OracleError, match="Gather"):
        run1("Gather", [table, np.asarray([4], np.int64)], {"axis": 0})


def _brute_conv(x, w, b, stride, pad, dil, group):
    n, c, h, wd = x.shape
    k, cg, kh, kw = w.shape
    oh = (h + pad[0] + pad[2] - (kh - 1) * dil[0] - 1) // stride[0] + 1
    ow = (wd + pad[1] + pad[3] - (kw - 1) * dil[1] - 1) // stride[1] + 1
    out = np.zeros((n, k, oh, ow))
    kg = k // group
    for ni in range(n):
        for ko in range(k):
            g = ko // kg
            for y in range(oh):
                for xx in range(ow):
                    acc = b[ko]
                    for ci in range(cg):
                        for i in range(kh):
                            for j in range(kw):
                                ih = y * stride[0] - pad[0] + i * dil[0]
                                iw = xx * stride[1] - pad[1] + j * dil[1]
                                if 0 <= ih < h and 0 <= iw < wd:
                                    acc += x[ni, g * cg + ci, ih, iw] * w[ko, ci, i, j]
                    out[ni, ko, y, xx] = acc
    return out


@pytest.mark.parametrize(
    "stride, pad, dil, group",
    [((1, 1), (1, 1, 1, 1), (1, 1), 1), ((2, 1), (0, 1, 2, 0), (1, 2), 1), ((1, 1), (1, 1, 1, 1), (1, 1), 2), ((2, 2), (1, 1, 1, 1), (1, 1), 4)],
)
def test_conv_matches_brute_force(stride, pad, dil, group):
    x = rng.standard_normal((2, 4, 7, 6)).astype(np.float32)
    w = rng.standard_normal((4, 4 // group, 3, 2)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    attrs = {"kernel_shape": [3, 2], "strides": list(stride), "pads": list(pad), "dilations": list(dil), "group": group}
    got = run1("Conv", [x, w, b], attrs, const={1, 2})["o0"]
    np.testing.assert_allclose(got, _brute_conv(x, w, b, stride, pad, dil, group), rtol=1e-5, atol=1e-5)
    # NHWC / HWIO layout gives the same numbers
    attrs_nhwc = {**attrs, "layout": "NHWC"}
    got2 = run1("Conv", [x.transpose(0, 2, 3, 1).copy(), w.transpose(2, 3, 1, 0).copy(), b], attrs_nhwc, const={1, 2})["o0"]
    np.testing.assert_allclose(got2.transpose(0, 3, 1, 2), got, rtol=1e-6, atol=1e-6)


def _brute_pool(x, kind, k, s, p, include, ceil):
    n, c, h, w = x.shape

    def osize(i, d):
        room = d + p[i] + p[i + 2] - k[i]
        o = (-(-room // s[i]) if ceil else room // s[i]) + 1
        if ceil and (o - 1) * s[i] >= d + p[i]:
            o -= 1
        return o

    oh, ow = osize(0, h), osize(1, w)
    out = np.zeros((n, c, oh, ow))
    for y in range(oh):
        for xx in range(ow):
            vals, cnt = [], 0
            for i in range(k[0]):
                for j in range(k[1]):
                    ih, iw = y * s[0] - p[0] + i, xx * s[1] - p[1] + j
                    if 0 <= ih < h and 0 <= iw < w:
                        vals.append(x[:, :, ih, iw])
                        cnt += 1
                    elif include and -p[0] <= ih < h + p[2] and -p[1] <= iw < w + p[3]:
                        cnt += 1
            stack = np.stack(vals)
            out[:, :, y, xx] = stack.max(0) if kind == "max" else stack.sum(0) / cnt
    return out


@pytest.mark.parametrize("kind", ["max", "avg"])
@pytest.mark.parametrize("s, p, include, ceil", [((2, 2), (1, 1, 1, 1), 0, 0), ((2, 2), (0, 0, 0, 0), 0, 1), ((1, 1), (1, 1, 1, 1), 1, 0), ((2, 2), (1, 1, 1, 1), 0, 1)])
def test_pool_matches_brute_force(kind, s, p, include, ceil):
    x = rng.standard_normal((2, 3, 9, 10)).astype(np.float32)
    attrs = {"kernel_shape": [3, 3], "strides": list(s), "pads": list(p), "ceil_mode": ceil}
    if kind == "avg":
        attrs["count_include_pad"] = include
    got = run1("MaxPool" if kind == "max" else "AveragePool", [x], attrs)["o0"]
    np.testing.assert_allclose(got, _brute_pool(x, kind, (3, 3), s, p, include, ceil), rtol=1e-5, atol=1e-6)


def test_softmax_layernorm_gelu_closed_forms():
    x = rng.standard_normal((3, 7)).astype(np.float32) * 3
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(1, keepdims=True))
    np.testing.assert_allclose(run1("Softmax", [x], {"axis": -1})["o0"], e / e.sum(1, keepdims=True), rtol=1e-6)
    g, b = rng.standard_normal(7).astype(np.float32), rng.standard_normal(7).astype(np.float32)
    mu, var = x64.mean(1, keepdims=True), x64.var(1, keepdims=True)
    expected = (x64 - mu) / np.sqrt(var + 1e-5) * g + b
    np.testing.assert_allclose(run1("LayerNormalization", [x, g, b], {"axis": -1, "epsilon": 1e-5}, const={1, 2})["o0"], expected, rtol=1e-5, atol=1e-6)
    gelu = 0.5 * x64 * (1 + np.array([math.erf(v / math.sqrt(2)) for v in x64.ravel()]).reshape(x.shape))
    np.testing.assert_allclose(run1("Gelu", [x])["o0"], gelu, rtol=1e-6, atol=1e-6)


def test_fused_gemm_activations_closed_forms():
    """FusedGemm activations against closed forms (reference tests/test_ops.py:440-465)."""
    a = rng.standard_normal((5, 4)).astype(np.float32)
    w = rng.standard_normal((4, 3)).astype(np.float32)
    bias = rng.standard_normal(3).astype(np.float32)
    y = a.astype(np.float64) @ w + bias
    cases = {"relu": np.maximum(y, 0), "clip": np.clip(y, -0.5, 0.7), "tanh": np.tanh(y), "sigmoid": 1 / (1 + np.exp(-y))}
    for act, want in cases.items():
        attrs = {"activation": act, "trans_b": 0}
        if act == "clip":
            attrs.update(clip_min=-0.5, clip_max=0.7)
        got = run1("FusedGemm", [a, w, bias], attrs, const={1, 2})["o0"]
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5, err_msg=act)


REF_CASES = ["mlp", "tiny-cnn", "tiny-bert", "single_gemm", "bottleneck", "mobilenet_v2"]


@pytest.mark.skipif(not HAVE_REFERENCE, reason="the reference's C kernels are built only where /root/reference exists")
@pytest.mark.parametrize("name", REF_CASES)
def test_oracle_agrees_with_reference_c_kernels(name, tmp_path):
    """The reference's own mgc_kernels.c (oracle/Makefile), driven by the restated emitter,
    against the numpy oracle on the unoptimized graph."""
    from oracle import cbackend

    make = builders.SAMPLES.get(name) or builders.CONFIGS[name]
    g0 = make()
    feeds = oracle.random_feeds(g0, 2)
    expected = oracle.run_graph(g0, feeds)
    g = make()
    optimize(g, "O3")
    schedule(g)
    got = cbackend.compile_c(g, tmp_path / f"{name}.so").run(feeds)
    for k, v in expected.items():
        err = float(np.max(np.abs(got[k].astype(np.float64) - v)))
        assert err <= 1e-4 * max(1.0, float(np.max(np.abs(v)))), (k, err)


def test_batch_norm_calibration_renormalizes_resnet50():
    """The calibration the full-depth parity test uses: after batch_norm_statistics on one
    image, every BatchNormalization of ResNet-50 maps its calibration input to per-channel mean
    beta and standard deviation |gamma| (closed form of BN with the batch's own statistics),
    and the logits of fresh images are O(1) instead of ~4e4."""
    from helpers import batch_norm_statistics, with_batch_norm_statistics

    g = builders.resnet50(1)
    feeds = oracle.random_feeds(g, 11)
    stats = batch_norm_statistics(g, feeds)
    assert len(stats) == 53
    env = dict(zip((id(v) for v in g.inputs), (feeds[v.name] for v in g.inputs)))
    for node in g.nodes:
        xs = [None if v is None else (v.data if v.data is not None else env[id(v)]) for v in node.inputs]
        out = oracle.run_node(node, xs)[0]
        env[id(node.output)] = out
        if node.op == "BatchNormalization":
            y = out.astype(np.float64)
            gamma, beta = xs[1].astype(np.float64), xs[2].astype(np.float64)
            eps = float(node.attrs.get("epsilon", 1e-5))
            var = xs[4].astype(np.float64)
            np.testing.assert_allclose(y.mean(axis=(0, 2, 3)), beta, atol=1e-4)
            np.testing.assert_allclose(y.std(axis=(0, 2, 3)), np.abs(gamma) * np.sqrt(var / (var + eps)), rtol=1e-3)
    fresh = with_batch_norm_statistics(builders.resnet50(1), stats)
    logits = oracle.run_graph(fresh, oracle.random_feeds(fresh, 3))["logits"]
    assert 0.1 < np.abs(logits).max() < 50.0
