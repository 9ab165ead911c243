"""hip backend end to end on the GPU: bundled samples and benchmark configs against the oracle.

Every test compiles with ``backend="hip"`` (the kernels of libmgc_hip.so; there is no CPU
fallback) and compares with the numpy oracle (oracle/interpreter.py) run on the unoptimized
graph with the same seeded inputs.
"""

from __future__ import annotations

import numpy as np
import pytest

from ml_graph_compiler import builders
from ml_graph_compiler.codegen import compile_graph
from ml_graph_compiler.passes import PIPELINES, optimize
from ml_graph_compiler.schedule import schedule
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu


def compile_hip(graph, cache, level="O3", **kw):
    optimize(graph, level)
    schedule(graph)
    return compile_graph(graph, cache_dir=cache, **kw)


@pytest.mark.parametrize("level", ["O0", "O2", "O3"])
@pytest.mark.parametrize("name", sorted(builders.SAMPLES))
def test_samples(name, level, hip_cache):
    print(f"[gpu] sample {name} {level}", flush=True)
    g0 = builders.SAMPLES[name]()
    feeds = oracle.random_feeds(g0, 4, int_high=100)
    expected = oracle.run_graph(g0, feeds)
    model = compile_hip(builders.SAMPLES[name](), hip_cache, level)
    got = model.run(feeds)
    for k, v in expected.items():
        assert got[k].shape == v.shape and got[k].dtype == v.dtype
        np.testing.assert_allclose(got[k], v, rtol=1e-4, atol=2e-5, err_msg=k)
    model.release()


def test_single_gemm(hip_cache):
    """Config 1: [128,768] x [768,3072] + bias, relu; max-abs <= 1e-4 against the oracle."""
    print("[gpu] single_gemm", flush=True)
    g0 = builders.single_gemm()
    feeds = oracle.random_feeds(g0, 0)
    expected = oracle.run_graph(g0, feeds)["y"]
    model = compile_hip(builders.single_gemm(), hip_cache)
    got = model.run(feeds)["y"]
    err = float(np.max(np.abs(got.astype(np.float64) - expected)))
    print(f"[gpu] single_gemm max-abs {err:.3e}", flush=True)
    assert err <= 1e-4
    model.release()


@pytest.mark.parametrize("batch", [1, 2])
def test_bottleneck(batch, hip_cache):
    print(f"[gpu] bottleneck b{batch}", flush=True)
    g0 = builders.bottleneck(batch)
    feeds = oracle.random_feeds(g0, 1)
    expected = oracle.run_graph(g0, feeds)["y"]
    model = compile_hip(builders.bottleneck(batch), hip_cache)
    got = model.run(feeds)["y"]
    err = float(np.max(np.abs(got.astype(np.float64) - expected)))
    print(f"[gpu] bottleneck b{batch} max-abs {err:.3e} max|ref| {np.abs(expected).max():.3e}", flush=True)
    assert err <= 1e-4
    model.release()


def _rel_err(got, expected):
    err = float(np.max(np.abs(got.astype(np.float64) - expected)))
    scale = float(np.max(np.abs(expected)))
    return err, scale


# ResNet-50 with random He-normal weights and BatchNorm statistics that do not renormalize grows
# activations block by block: |logits| reach ~4e4, where one fp32 ulp is ~4e-3, so an absolute
# 1e-4 bound is below float resolution. The bound is relative to max|logit| instead: the
# reference's own C backend sits at ~5e-7 of max|logit| against the same oracle
# (tests/test_oracle.py), and the hip result must stay within 1e-5 with identical top-1.
RESNET_REL_TOL = 1e-5


@pytest.mark.parametrize("batch", [1, 32])
def test_resnet50(batch, hip_cache):
    print(f"[gpu] resnet50 b{batch}", flush=True)
    graph = builders.resnet50(batch)
    feeds = oracle.random_feeds(graph, 3)
    model = compile_hip(builders.resnet50(batch), hip_cache)
    got = model.run(feeds)["logits"]
    model.release()
    # the oracle on every image of b1, on the first and last image of b32 (batch independence)
    images = [0] if batch == 1 else [0, batch - 1]
    single = builders.resnet50(1)
    for i in images:
        expected = oracle.run_graph(single, {"image": feeds["image"][i : i + 1]})["logits"]
        err, scale = _rel_err(got[i : i + 1], expected)
        print(f"[gpu] resnet50 b{batch} image {i}: max-abs {err:.3e} max|logit| {scale:.3e} "
              f"rel {err / scale:.2e}", flush=True)
        assert err <= RESNET_REL_TOL * scale
        assert int(np.argmax(got[i])) == int(np.argmax(expected[0]))


@pytest.mark.parametrize("batch", [1, 32])
def test_mobilenet_v2(batch, hip_cache):
    print(f"[gpu] mobilenet_v2 b{batch}", flush=True)
    feeds = oracle.random_feeds(builders.mobilenet_v2(batch), 5)
    model = compile_hip(builders.mobilenet_v2(batch), hip_cache)
    got = model.run(feeds)["logits"]
    model.release()
    single = builders.mobilenet_v2(1)
    for i in ([0] if batch == 1 else [0, batch - 1]):
        expected = oracle.run_graph(single, {"image": feeds["image"][i : i + 1]})["logits"]
        err, scale = _rel_err(got[i : i + 1], expected)
        print(f"[gpu] mobilenet_v2 b{batch} image {i}: max-abs {err:.3e} max|logit| {scale:.3e}", flush=True)
        assert err <= 1e-4
        assert int(np.argmax(got[i])) == int(np.argmax(expected[0]))


@pytest.mark.parametrize("batch", [1, 16])
def test_bert_base(batch, hip_cache):
    print(f"[gpu] bert_base b{batch}", flush=True)
    graph = builders.bert_base(batch)
    feeds = oracle.random_feeds(graph, 6, int_high=30522)
    model = compile_hip(builders.bert_base(batch), hip_cache)
    got = model.run(feeds)["hidden"]
    model.release()
    single = builders.bert_base(1)
    for i in ([0] if batch == 1 else [0, batch - 1]):
        expected = oracle.run_graph(single, {"input_ids": feeds["input_ids"][i : i + 1]})["hidden"]
        err, scale = _rel_err(got[i : i + 1], expected)
        print(f"[gpu] bert_base b{batch} sequence {i}: max-abs {err:.3e} max|h| {scale:.3e}", flush=True)
        assert err <= 5e-4


@pytest.mark.parametrize("batch", [1, 8])
def test_gpt2(batch, hip_cache):
    """GPT-2 small at sequence 128: fused causal attention and the tied 50257-wide head."""
    print(f"[gpu] gpt2 b{batch}", flush=True)
    graph = builders.gpt2(batch)
    feeds = oracle.random_feeds(graph, 8, int_high=50257)
    model = compile_hip(builders.gpt2(batch), hip_cache)
    assert model.report.kernels.get("attention") == 12
    got = model.run(feeds)["logits"]
    model.release()
    single = builders.gpt2(1)
    for i in ([0] if batch == 1 else [0, batch - 1]):
        expected = oracle.run_graph(single, {"input_ids": feeds["input_ids"][i : i + 1]})["logits"]
        err, scale = _rel_err(got[i : i + 1], expected)
        print(f"[gpu] gpt2 b{batch} sequence {i}: max-abs {err:.3e} max|logit| {scale:.3e}", flush=True)
        assert err <= 5e-4
        assert np.array_equal(np.argmax(got[i], -1), np.argmax(expected[0], -1))


@pytest.mark.parametrize(
    "name, kwargs",
    [
        # BERT-large width (hidden 1024 = the widest row the fused GEMM + LayerNorm takes, 16 heads)
        ("bert_large_2l", dict(batch=2, seq=256, d_model=1024, heads=16, layers=2, vocab=1000, gelu="erf",
                               causal=False, weight_scale=0.02, unit_layer_norm=True, embedding_norm=True,
                               lm_head=False, ln_eps=1e-12)),
        # GPT-2-medium width, a ragged causal sequence and a vocabulary head
        ("gpt2_medium_2l", dict(batch=2, seq=200, d_model=1024, heads=16, layers=2, vocab=3000, gelu="tanh",
                                causal=True, weight_scale=0.02)),
        # hidden 1280 (GPT-2 large): wider than the fused GEMM + LayerNorm, so it stays unfused
        ("gpt2_large_width_1l", dict(batch=1, seq=64, d_model=1280, heads=20, layers=1, vocab=500, gelu="tanh",
                                     causal=True, weight_scale=0.02)),
    ],
)
def test_wider_transformers(name, kwargs, hip_cache):
    print(f"[gpu] {name}", flush=True)
    graph = builders.transformer(name=name, **kwargs)
    feeds = oracle.random_feeds(graph, 12, int_high=kwargs["vocab"])
    expected = oracle.run_graph(graph, feeds)
    model = compile_hip(builders.transformer(name=name, **kwargs), hip_cache)
    kernels = dict(model.report.kernels)
    try:
        got = model.run(feeds)
    finally:
        model.release()
    assert kernels.get("attention") == kwargs["layers"], kernels
    assert (kernels.get("gemm_layer_norm", 0) > 0) == (kwargs["d_model"] <= 1024), kernels
    for k, want in expected.items():
        err, scale = _rel_err(got[k], want)
        print(f"[gpu] {name} {k}: max-abs {err:.3e} max|ref| {scale:.3e}", flush=True)
        assert err <= 5e-4


def test_gather_out_of_range_raises(hip_cache):
    from ml_graph_compiler.errors import GraphError

    model = compile_hip(builders.transformer(vocab=16), hip_cache)
    with pytest.raises(GraphError, match="Gather"):
        model.run({"input_ids": np.full((1, 8), 99, np.int64)})
    with pytest.raises(GraphError, match="missing"):
        model.run({})
    with pytest.raises(GraphError, match="expected"):
        model.run({"input_ids": np.zeros((1, 8), np.int32)})
    # the flag was cleared when the error was reported
    ok = model.run({"input_ids": np.zeros((1, 8), np.int64)})
    assert np.isfinite(ok["logits"]).all()
    # replays without a check: the error of any of them is reported by the next check, once
    model.upload({"input_ids": np.full((1, 8), 99, np.int64)})
    model.launch(2)
    model.upload({"input_ids": np.zeros((1, 8), np.int64)})
    model.launch(1)
    with pytest.raises(GraphError, match="Gather"):
        model.sync()
    model.launch(1)
    model.sync()
    model.release()
