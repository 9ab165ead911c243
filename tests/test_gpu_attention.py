"""Fused attention (mgc_hip_attention) against the oracle running the unfused chain.

The graphs are the chain the transformer sample builds (head-split Reshape/Transpose, QK^T,
scale, Softmax, PV, head-merge Transpose), at sizes that exercise the kernel's edges: a query
count that is not a multiple of the 64-row block, key counts that span several 64-key blocks
and end mid-block, a head dim below 64, separate Q/K/V tensors and a fused QKV projection.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip, f32
from ml_graph_compiler import builders
from ml_graph_compiler.codegen import attention as attn
from ml_graph_compiler.codegen import hip as hip_codegen
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.memory import plan_memory
from ml_graph_compiler.passes import optimize
from ml_graph_compiler.schedule import schedule
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle


def attention_graph(B: int, H: int, S: int, Skv: int, D: int, fused_qkv: bool, scale: float = 0.125):
    g = Graph("attention")
    HD = H * D
    feeds = {}
    if fused_qkv:
        assert S == Skv
        qkv = g.add_input("qkv", TensorType("float32", (B, S, 3 * HD)))
        feeds["qkv"] = f32(B, S, 3 * HD)
        sizes = g.constant(np.array([HD, HD, HD], np.int64), "sizes")
        sp = g.add_node("Split", [qkv, sizes], 3, {"axis": -1}, name="split", output_names=["q", "k", "v"])
        q, k, v = sp.outputs
    else:
        q = g.add_input("q", TensorType("float32", (B, S, HD)))
        k = g.add_input("k", TensorType("float32", (B, Skv, HD)))
        v = g.add_input("v", TensorType("float32", (B, Skv, HD)))
        feeds.update(q=f32(B, S, HD), k=f32(B, Skv, HD), v=f32(B, Skv, HD))

    def heads(x, n, perm, tag):
        r = g.add_node("Reshape", [x], 1, {"shape": [B, n, H, D]}, name=f"r{tag}", output_names=[f"r{tag}_out"])
        return g.add_node("Transpose", [r.output], 1, {"perm": perm}, name=f"t{tag}", output_names=[f"t{tag}_out"]).output

    tq = heads(q, S, [0, 2, 1, 3], "q")
    tk = heads(k, Skv, [0, 2, 3, 1], "k")
    tv = heads(v, Skv, [0, 2, 1, 3], "v")
    s = g.add_node("MatMul", [tq, tk], 1, {}, name="qk", output_names=["scores"]).output
    c = g.constant(np.array(scale, np.float32), "scale")
    sc = g.add_node("Mul", [s, c], 1, {}, name="scale_mul", output_names=["scaled"]).output
    p = g.add_node("Softmax", [sc], 1, {"axis": -1}, name="softmax", output_names=["probs"]).output
    o = g.add_node("MatMul", [p, tv], 1, {}, name="pv", output_names=["ctx"]).output
    to = g.add_node("Transpose", [o], 1, {"perm": [0, 2, 1, 3]}, name="merge", output_names=["merged"]).output
    y = g.add_node("Reshape", [to], 1, {"shape": [B, S, HD]}, name="flat", output_names=["y"]).output
    g.add_output(y, "y")
    infer_shapes(g)
    return g, feeds


def _run(graph, feeds, cache, opt="O3"):
    model = compile_hip(graph, cache, opt)
    try:
        return model.run(feeds), dict(model.report.kernels)
    finally:
        model.release()


@pytest.mark.gpu
@pytest.mark.parametrize(
    "B, H, S, Skv, D, fused_qkv",
    [
        (2, 3, 77, 77, 48, True),    # ragged query block and key block, D < 64
        (1, 2, 50, 200, 64, False),  # separate Q/K/V, 4 key blocks (last partial), S != Skv
        (3, 4, 128, 128, 64, True),  # BERT's shape per head, two query blocks
        (1, 2, 3, 5, 4, False),      # tiny: one query block, one partial key block, D = 4
        (2, 2, 256, 256, 32, True),  # key limit, D of one MFMA column block
    ],
)
def test_fused_attention_matches_oracle(B, H, S, Skv, D, fused_qkv, hip_cache):
    g, feeds = attention_graph(B, H, S, Skv, D, fused_qkv)
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache)
    assert kernels.get("attention") == 1, kernels
    err = float(np.max(np.abs(got["y"].astype(np.float64) - expected)))
    assert err <= 2e-5 * max(1.0, float(np.max(np.abs(expected)))), err


@pytest.mark.gpu
def test_attention_outside_limits_stays_unfused(hip_cache):
    g, feeds = attention_graph(1, 2, 16, 300, 16, False)  # Skv > 256
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache)
    assert "attention" not in kernels
    assert float(np.max(np.abs(got["y"].astype(np.float64) - expected))) <= 2e-5


@pytest.mark.gpu
def test_fused_and_unfused_tiny_bert_agree(hip_cache, monkeypatch):
    feeds = oracle.random_feeds(builders.tiny_bert(), 0, int_high=50)
    expected = oracle.run_graph(builders.tiny_bert(), feeds)
    outs = {}
    for fuse in (True, False):
        monkeypatch.setattr(hip_codegen, "FUSE_ATTENTION", fuse)
        got, kernels = _run(builders.tiny_bert(), feeds, hip_cache)
        assert ("attention" in kernels) == fuse
        outs[fuse] = got
    for name, want in expected.items():
        for fuse in (True, False):
            assert float(np.max(np.abs(outs[fuse][name].astype(np.float64) - want))) <= 5e-5


def test_matcher_finds_every_bert_layer():
    """CPU: all 12 BERT-base layers match (staged: the planner put the context where the dead
    QKV projection was); the causal GPT sample, whose mask sits between scale and softmax, does
    not."""
    g = builders.bert_base(1)
    optimize(g, "O3")
    schedule(g)
    found = attn.find_attention(g, plan_memory(g, alignment=256))
    assert len(found) == 12
    assert all(m.S == 128 and m.Skv == 128 and m.D == 64 and m.H == 12 for m in found)
    assert all(abs(m.scale - 0.125) < 1e-7 for m in found)
    assert all(len(m.absorbed) == 12 for m in found)  # split, 3 x (reshape, transpose), qk, mul, softmax, pv, merge
    gpt = builders.tiny_gpt()
    optimize(gpt, "O3")
    schedule(gpt)
    assert attn.find_attention(gpt, plan_memory(gpt, alignment=256)) == []
