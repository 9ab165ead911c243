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


def _per_item_error(got: np.ndarray, expected: np.ndarray) -> np.ndarray:
    """Max-abs error of every batch element (axis 0)."""
    diff = np.abs(got.astype(np.float64) - np.asarray(expected, np.float64))
    return diff.reshape(diff.shape[0], -1).max(axis=1)


def _check_batch(label: str, got: np.ndarray, expected: np.ndarray, tol: float, top1: bool) -> np.ndarray:
    """Every element of a batched run against the oracle run on the whole batch: max-abs per
    element within ``tol`` and, for logits, the arg-max of every row (every image, every
    sequence position) identical (the reference's parity harness, benchmarks/parity.py:104-125)."""
    assert got.shape == expected.shape and got.dtype == np.float32
    errs = _per_item_error(got, expected)
    worst = int(np.argmax(errs))
    print(f"[gpu] {label}: max-abs {errs.max():.3e} (element {worst} of {len(errs)}), "
          f"max|ref| {np.abs(expected).max():.3e}", flush=True)
    assert np.all(errs <= tol), (label, errs.tolist())
    if top1:
        same = np.argmax(got, axis=-1) == np.argmax(expected, axis=-1)
        print(f"[gpu] {label}: top-1 agreement {same.mean():.4f} over {same.size} rows", flush=True)
        assert same.all()
    return errs


@pytest.mark.parametrize("batch", [1, 2, 32])
def test_bottleneck(batch, hip_cache):
    """Config 2 at batch 1 and 32 (and 2): the batched-offset path of the implicit-GEMM
    convolutions (reference c.py:1144-1167), every image against the oracle."""
    print(f"[gpu] bottleneck b{batch}", flush=True)
    g0 = builders.bottleneck(batch)
    feeds = oracle.random_feeds(g0, 1)
    model = compile_hip(builders.bottleneck(batch), hip_cache)
    got = model.run(feeds)["y"]
    model.release()
    expected = oracle.run_graph(g0, feeds)["y"]
    _check_batch(f"bottleneck b{batch}", got, expected, 1e-4, top1=False)


# ResNet-50 with random He-normal weights and BatchNorm statistics that do not renormalize grows
# activations block by block: |logits| reach ~4e4, where one fp32 ulp is ~4e-3, so an absolute
# 1e-4 bound is below float resolution. The gate is the reference's own C backend instead: run in
# the same test on the same inputs and weights, its error against the oracle is the fp32 floor,
# and the hip error may be at most twice that floor.
RESNET_FLOOR_FACTOR = 2.0


@pytest.mark.parametrize("batch", [1, 32])
def test_resnet50(batch, hip_cache):
    from oracle import cbackend

    print(f"[gpu] resnet50 b{batch}", flush=True)
    graph = builders.resnet50(batch)
    feeds = oracle.random_feeds(graph, 3)
    model = compile_hip(builders.resnet50(batch), hip_cache)
    got = model.run(feeds)["logits"]
    model.release()
    print(f"[gpu] resnet50 b{batch}: reference C backend", flush=True)
    cmodel, _, _ = cbackend.load_baseline("resnet50", batch)
    cref = cmodel.run(feeds)["logits"]
    print(f"[gpu] resnet50 b{batch}: oracle", flush=True)
    expected = oracle.run_graph(graph, feeds)["logits"]
    c_errs = _per_item_error(cref, expected)
    floor = float(c_errs.max())
    print(f"[gpu] resnet50 b{batch}: reference C backend max-abs {floor:.3e} "
          f"(rel {floor / np.abs(expected).max():.2e})", flush=True)
    errs = _check_batch(f"resnet50 b{batch}", got, expected, RESNET_FLOOR_FACTOR * floor, top1=True)
    print(f"[gpu] resnet50 b{batch}: hip / C error {errs.max() / floor:.2f}", flush=True)
    assert np.array_equal(np.argmax(cref, -1), np.argmax(expected, -1))


# The calibrated network's own fp32 floor: the reference's C backend on the same inputs and
# weights measured 9.5e-5 (b1) and 1.09e-4 (b32) max-abs against the oracle on logits of up to
# 6.5, so 1e-4 is the bound wherever fp32 reaches it and 1.5 times the C backend's error where
# the C backend itself does not.
CALIBRATED_FLOOR_FACTOR = 1.5


@pytest.mark.parametrize("batch", [1, 32])
def test_resnet50_calibrated(batch, hip_cache):
    """Full-depth ResNet-50 at the north_star's absolute bound: the same topology and He-normal
    weights, with every BatchNormalization's running statistics calibrated on two other
    N(0, 1) images (helpers.batch_norm_statistics), so each block's output stays O(1) and the
    logits are O(1) too (the uncalibrated network's reach ~4e4). BatchNorm is folded at O3 as
    in config 3; every image against the oracle at max-abs <= 1e-4 (or 1.5 x the reference C
    backend's own error on the same inputs, when that is above 1e-4: the fp32 floor) with
    identical top-1, the C backend run alongside with the calibrated weights (the reference's
    parity harness, benchmarks/parity.py:104-125; its published ResNet-50 parity is 4.0e-5
    max-abs with trained weights, README.md:74)."""
    from helpers import batch_norm_statistics, with_batch_norm_statistics

    print(f"[gpu] resnet50 calibrated b{batch}: calibration", flush=True)
    calib = builders.resnet50(2)
    stats = batch_norm_statistics(calib, oracle.random_feeds(calib, 11))
    graph = with_batch_norm_statistics(builders.resnet50(batch), stats)
    feeds = oracle.random_feeds(graph, 3)
    model = compile_hip(with_batch_norm_statistics(builders.resnet50(batch), stats), hip_cache)
    got = model.run(feeds)["logits"]
    model.release()
    print(f"[gpu] resnet50 calibrated b{batch}: oracle", flush=True)
    expected = oracle.run_graph(graph, feeds)["logits"]
    assert np.abs(expected).max() < 50.0
    from oracle import cbackend

    cgraph = with_batch_norm_statistics(builders.resnet50(batch), stats)
    optimize(cgraph, "O3")
    schedule(cgraph)
    cref = cbackend.load_baseline_with_weights("resnet50", batch, cgraph).run(feeds)["logits"]
    floor = float(_per_item_error(cref, expected).max())
    print(f"[gpu] resnet50 calibrated b{batch}: reference C backend max-abs {floor:.3e}", flush=True)
    errs = _check_batch(f"resnet50 calibrated b{batch}", got, expected, max(1e-4, CALIBRATED_FLOOR_FACTOR * floor),
                        top1=True)
    print(f"[gpu] resnet50 calibrated b{batch}: hip / C error {errs.max() / floor:.2f}", flush=True)
    assert np.array_equal(np.argmax(cref, -1), np.argmax(expected, -1))


@pytest.mark.parametrize("batch", [1, 32])
def test_mobilenet_v2(batch, hip_cache):
    print(f"[gpu] mobilenet_v2 b{batch}", flush=True)
    graph = builders.mobilenet_v2(batch)
    feeds = oracle.random_feeds(graph, 5)
    model = compile_hip(builders.mobilenet_v2(batch), hip_cache)
    got = model.run(feeds)["logits"]
    model.release()
    expected = oracle.run_graph(graph, feeds)["logits"]
    _check_batch(f"mobilenet_v2 b{batch}", got, expected, 1e-4, top1=True)


@pytest.mark.parametrize("batch", [1, 16])
def test_bert_base(batch, hip_cache):
    print(f"[gpu] bert_base b{batch}", flush=True)
    graph = builders.bert_base(batch)
    feeds = oracle.random_feeds(graph, 6, int_high=30522)
    model = compile_hip(builders.bert_base(batch), hip_cache)
    got = model.run(feeds)["hidden"]
    model.release()
    expected = oracle.run_graph(graph, feeds)["hidden"]
    _check_batch(f"bert_base b{batch}", got, expected, 5e-4, top1=False)


@pytest.mark.parametrize("batch", [1, 8])
def test_gpt2(batch, hip_cache):
    """GPT-2 small at sequence 128: fused causal attention and the tied 50257-wide head; the
    next-token arg-max of every position of every sequence must agree."""
    print(f"[gpu] gpt2 b{batch}", flush=True)
    graph = builders.gpt2(batch)
    feeds = oracle.random_feeds(graph, 8, int_high=50257)
    model = compile_hip(builders.gpt2(batch), hip_cache)
    assert model.report.kernels.get("attention") == 12
    got = model.run(feeds)["logits"]
    model.release()
    expected = oracle.run_graph(graph, feeds)["logits"]
    _check_batch(f"gpt2 b{batch}", got, expected, 5e-4, top1=True)


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
        _check_batch(f"{name} {k}", got[k], want, 5e-4, top1=False)


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
