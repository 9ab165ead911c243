"""Optimization passes: each rewrite's effect and preserved numerics (the reference's
tests/test_passes.py, with the numpy oracle as the numerics check)."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import named_graph, same_numerics
from ml_graph_compiler import builders
from ml_graph_compiler.errors import CompilerError
from ml_graph_compiler.passes import (
    PIPELINES,
    eliminate_common_subexpressions,
    eliminate_dead_code,
    fold_constants,
    optimize,
    resolve,
    simplify,
)

F32, I64 = "float32", "int64"


@pytest.mark.parametrize("level", list(PIPELINES))
@pytest.mark.parametrize("name", sorted(builders.SAMPLES))
def test_every_pipeline_preserves_numerics(name, level):
    same_numerics(builders.SAMPLES[name], level, rtol=1e-4, atol=1e-5).verify()


@pytest.mark.parametrize(
    "name, expected",
    [
        ("mlp", {"FusedGemm": 3, "Softmax": 1}),
        ("tiny-cnn", {"FusedConv": 9, "FusedGemm": 1, "GlobalAveragePool": 1, "MaxPool": 1, "Reshape": 1, "Transpose": 1}),
    ],
)
def test_o3_operator_mix(name, expected):
    g = builders.SAMPLES[name]()
    optimize(g, "O3")
    assert g.op_counts() == expected


@pytest.mark.parametrize("name", ["tiny-gpt", "tiny-bert"])
def test_transformer_patterns_are_fused(name):
    g = builders.SAMPLES[name]()
    report = optimize(g, "O2")
    ops = g.op_counts()
    assert ops["LayerNormalization"] in (4, 5)
    assert "Erf" not in ops and "Tanh" not in ops and "Pow" not in ops and "ReduceMean" not in ops
    assert ops["FusedGemm"] == 9
    acts = {n.attrs["activation"] for n in g.nodes if n.op == "FusedGemm"}
    assert acts == {"none", "gelu_tanh" if name == "tiny-gpt" else "gelu"}
    assert report.nodes_after < report.nodes_before / 3


def test_pass_report_and_resolve():
    report = optimize(builders.mlp(), ["fold", "dce", "fuse"], verify=False)
    d = report.to_dict()
    assert d["nodes_before"] == 9 and d["nodes_after"] == 4
    assert [p["name"] for p in d["passes"]] == ["fold", "dce", "fuse"]
    assert resolve("fold, cse") == ["fold", "cse"]
    assert resolve("O0") == []
    with pytest.raises(CompilerError, match="unknown passes"):
        resolve("fold,warp")
    assert optimize(builders.mlp(), "O0").nodes_after == 9


def test_constant_folding_and_shape_folding():
    a = np.arange(6, dtype=np.float32).reshape(2, 3)

    def make():
        return named_graph(
            [
                ("Mul", ["a", "a"], ["sq"], {}),
                ("Shape", ["x"], ["s"], {}),
                ("Size", ["x"], ["n"], {}),
                ("Cast", ["n"], ["nf"], {"to": 1}),
                ("Reshape", ["x", "s"], ["xr"], {}),
                ("Add", ["xr", "sq"], ["y0"], {}),
                ("Add", ["y0", "nf"], ["y"], {}),
            ],
            [("x", (2, 3), F32)],
            ["y"],
            [("a", a)],
        )

    g = make()
    assert fold_constants(g) == 4
    assert g.op_counts() == {"Add": 2, "Reshape": 1}
    same_numerics(make, "fold")


def test_folding_skips_large_growth():
    g = named_graph(
        [("Expand", ["c", "shape"], ["big"], {}), ("Add", ["x", "big"], ["y"], {})],
        [("x", (4096, 2048), F32)],
        ["y"],
        [("c", np.ones((1,), np.float32)), ("shape", np.asarray([4096, 2048], np.int64))],
    )
    fold_constants(g)
    assert "Expand" in g.op_counts()


def test_dead_code_elimination():
    g = named_graph([("Relu", ["x"], ["unused"], {}), ("Neg", ["x"], ["y"], {})], [("x", (3,), F32)], ["y"])
    assert eliminate_dead_code(g) == 1
    assert g.op_counts() == {"Neg": 1}
    assert eliminate_dead_code(g) == 0


def test_cse_merges_nodes_constants_and_commutative_operands():
    c = np.ones(3, np.float32)

    def make():
        return named_graph(
            [
                ("Add", ["x", "c1"], ["a"], {}),
                ("Add", ["c2", "x"], ["b"], {}),
                ("Sub", ["x", "c1"], ["s1"], {}),
                ("Sub", ["c1", "x"], ["s2"], {}),
                ("Mul", ["a", "b"], ["m"], {}),
                ("Mul", ["s1", "s2"], ["n"], {}),
                ("Add", ["m", "n"], ["y"], {}),
            ],
            [("x", (3,), F32)],
            ["y"],
            [("c1", c), ("c2", c.copy())],
        )

    g = make()
    assert eliminate_common_subexpressions(g) == 2
    assert g.op_counts() == {"Add": 2, "Sub": 2, "Mul": 2}
    same_numerics(make, "cse")


def test_cse_distinguishes_attributes():
    g = named_graph(
        [("Softmax", ["x"], ["a"], {"axis": 0}), ("Softmax", ["x"], ["b"], {"axis": 1}), ("Add", ["a", "b"], ["y"], {})],
        [("x", (2, 3), F32)],
        ["y"],
    )
    assert eliminate_common_subexpressions(g) == 0


@pytest.mark.parametrize(
    "op, const, first",
    [("Add", 0.0, False), ("Sub", 0.0, False), ("Mul", 1.0, False), ("Div", 1.0, False), ("Pow", 1.0, False),
     ("Add", 0.0, True), ("Mul", 1.0, True)],
)
def test_neutral_elements_are_removed(op, const, first):
    g = named_graph(
        [(op, ["k", "x"] if first else ["x", "k"], ["t"], {}), ("Neg", ["t"], ["y"], {})],
        [("x", (2, 3), F32)],
        ["y"],
        [("k", np.asarray(const, np.float32))],
    )
    assert simplify(g) >= 1
    assert g.op_counts() == {"Neg": 1}


def test_neutral_add_that_broadcasts_is_kept():
    g = named_graph([("Add", ["x", "k"], ["y"], {})], [("x", (3,), F32)], ["y"], [("k", np.zeros((2, 3), np.float32))])
    simplify(g)
    assert g.op_counts() == {"Add": 1}


@pytest.mark.parametrize("exponent, ops", [(2.0, {"Mul": 1}), (3.0, {"Mul": 2}), (0.5, {"Sqrt": 1})])
def test_pow_strength_reduction(exponent, ops):
    def make():
        return named_graph([("Pow", ["x", "e"], ["y"], {})], [("x", (4,), F32)], ["y"], [("e", np.asarray(exponent, np.float32))])

    g = make()
    optimize(g, "simplify")
    assert g.op_counts() == ops
    # sqrt of negative inputs is nan in both graphs; compare on |x|
    ref = make()
    feeds = {"x": np.abs(np.random.default_rng(0).standard_normal(4)).astype(np.float32)}
    from oracle import interpreter as oracle

    np.testing.assert_allclose(oracle.run_graph(g, feeds)["y"], oracle.run_graph(ref, feeds)["y"], rtol=1e-6)


def test_div_by_constant_becomes_mul_but_not_by_zero_or_integers():
    def make():
        return named_graph([("Div", ["x", "c"], ["y"], {})], [("x", (4,), F32)], ["y"],
                           [("c", np.asarray([2, 4, 8, 16], np.float32))])

    assert same_numerics(make, "simplify").op_counts() == {"Mul": 1}
    g = named_graph([("Div", ["x", "c"], ["y"], {})], [("x", (2,), F32)], ["y"], [("c", np.asarray([0, 1], np.float32))])
    simplify(g)
    assert g.op_counts() == {"Div": 1}
    g = named_graph([("Div", ["x", "c"], ["y"], {})], [("x", (2,), I64)], ["y"], [("c", np.asarray([2, 3], np.int64))])
    simplify(g)
    assert g.op_counts() == {"Div": 1}


def test_identity_like_ops_are_removed():
    def make():
        return named_graph(
            [
                ("Identity", ["x"], ["a"], {}),
                ("Dropout", ["a"], ["b"], {}),
                ("Cast", ["b"], ["c"], {"to": 1}),
                ("Expand", ["c", "shape"], ["d"], {}),
                ("Concat", ["d"], ["e"], {"axis": 0}),
                ("Pad", ["e", "pads"], ["f"], {}),
                ("Relu", ["f"], ["y"], {}),
            ],
            [("x", (2, 3), F32)],
            ["y"],
            [("shape", np.asarray([2, 3], np.int64)), ("pads", np.zeros(4, np.int64))],
        )

    assert same_numerics(make, "simplify").op_counts() == {"Relu": 1}


def test_conv_batchnorm_fold_is_the_closed_form():
    """fusion._fold_batch_norm: W' = W * s / sqrt(v + eps) per output channel (float64),
    b' = (b - mean) * s / sqrt(v + eps) + beta (passes/fusion.py:220-243)."""
    rng = np.random.default_rng(0)
    w = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    s, beta, mean = (rng.standard_normal(4).astype(np.float32) for _ in range(3))
    var = (rng.random(4) + 0.5).astype(np.float32)

    def make():
        return named_graph(
            [("Conv", ["x", "w", "b"], ["c"], {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1]}),
             ("BatchNormalization", ["c", "s", "beta", "m", "v"], ["y"], {"epsilon": 1e-3})],
            [("x", (1, 3, 5, 5), F32)],
            ["y"],
            [("w", w), ("b", b), ("s", s), ("beta", beta), ("m", mean), ("v", var)],
        )

    g = same_numerics(make, "fuse", rtol=1e-4, atol=1e-5)
    conv = [n for n in g.nodes if n.op == "FusedConv"]
    assert len(conv) == 1 and g.op_counts() == {"FusedConv": 1}
    factor = s.astype(np.float64) / np.sqrt(var.astype(np.float64) + 1e-3)
    np.testing.assert_array_equal(conv[0].input(1).data, (w.astype(np.float64) * factor.reshape(4, 1, 1, 1)).astype(np.float32))
    np.testing.assert_array_equal(conv[0].input(2).data, ((b.astype(np.float64) - mean) * factor + beta).astype(np.float32))


def test_nhwc_leaves_one_input_transpose():
    g = builders.tiny_cnn()
    optimize(g, "layout")
    assert g.op_counts()["Transpose"] == 1
    assert all(n.attrs.get("layout") == "NHWC" for n in g.nodes if n.op in ("FusedConv", "MaxPool", "GlobalAveragePool"))
