"""Fused attention (mgc_hip_attention) against the oracle running the unfused chain.

The graphs are the chain the transformer sample builds (head-split Reshape/Transpose, QK^T,
score ops, Softmax, PV, head-merge Transpose), at sizes that exercise the kernel's edges: a
query count that is not a multiple of the 64-row block, key counts that span several 64-key
blocks and end mid-block, long sequences (the keys stream through a running softmax), a head
dim below 64, separate Q/K/V tensors and a fused QKV projection. The score ops cover what the
matcher accepts: Mul or Div by a scalar, an additive bias (constant or computed at run time,
broadcast over heads or queries), and a Where mask in both polarities (constant causal with a
finite or -inf fill, an arbitrary constant mask, a mask fed as an input). With fewer than 256
(batch, head, query block) workgroups the kernel splits each workgroup's key blocks between two
groups of waves and merges their softmax states at the end (odd key-block counts leave the second
group idle in the last step); the many-head cases (512 and more workgroups) run one group.
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

rng = np.random.default_rng(7)


def attention_graph(B: int, H: int, S: int, Skv: int, D: int, fused_qkv: bool, scale: float = 0.125,
                    divide: bool = False, bias: str | None = None, mask: str | None = None,
                    keep_true: bool = False, fill: float = -1e4):
    """``bias``: None, "const" ([1, H, S, Skv]) or "input" ([B, 1, 1, Skv], BERT's padding form);
    ``mask``: None, "causal", "random" (constant [S, Skv]) or "input" ([B, 1, S, Skv] bool);
    ``keep_true``: Where(mask, t, fill) instead of Where(mask, fill, t)."""
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
    if divide:
        c = g.constant(np.array(1.0 / scale, np.float32), "denom")
        s = g.add_node("Div", [s, c], 1, {}, name="scale_div", output_names=["scaled"]).output
    else:
        c = g.constant(np.array(scale, np.float32), "scale")
        s = g.add_node("Mul", [c, s], 1, {}, name="scale_mul", output_names=["scaled"]).output
    if bias == "const":
        bv = g.constant((rng.standard_normal((1, H, S, Skv)) * 0.5).astype(np.float32), "bias")
        s = g.add_node("Add", [s, bv], 1, {}, name="bias_add", output_names=["biased"]).output
    elif bias == "input":
        keep = g.add_input("attention_mask", TensorType("float32", (B, Skv)))
        feeds["attention_mask"] = (rng.random((B, Skv)) < 0.8).astype(np.float32)
        r = g.add_node("Reshape", [keep], 1, {"shape": [B, 1, 1, Skv]}, name="mask_r", output_names=["mask_4d"]).output
        one = g.constant(np.array(1.0, np.float32), "one")
        big = g.constant(np.array(-1e4, np.float32), "big")
        inv = g.add_node("Sub", [one, r], 1, {}, name="mask_inv", output_names=["mask_inv"]).output
        add = g.add_node("Mul", [inv, big], 1, {}, name="mask_scale", output_names=["mask_add"]).output
        s = g.add_node("Add", [add, s], 1, {}, name="bias_add", output_names=["biased"]).output
    if mask is not None:
        if mask == "causal":
            drop = np.triu(np.ones((S, Skv), bool), 1)[None, None]
            m = g.constant(~drop if keep_true else drop, "mask")
        elif mask == "random":
            drop = rng.random((S, Skv)) < 0.3
            drop[:, 0] = False  # every row keeps a key
            m = g.constant(~drop if keep_true else drop, "mask")
        else:
            m = g.add_input("mask", TensorType("bool", (B, 1, S, Skv)))
            drop = rng.random((B, 1, S, Skv)) < 0.3
            drop[..., 0] = False
            feeds["mask"] = ~drop if keep_true else drop
        f = g.constant(np.array(fill, np.float32), "fill")
        args = [m, s, f] if keep_true else [m, f, s]
        s = g.add_node("Where", args, 1, {}, name="mask_where", output_names=["masked"]).output
    p = g.add_node("Softmax", [s], 1, {"axis": -1}, name="softmax", output_names=["probs"]).output
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


def _check(g, feeds, hip_cache, opt="O3", fused=True):
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache, opt)
    assert (kernels.get("attention") == 1) if fused else ("attention" not in kernels), kernels
    err = float(np.max(np.abs(got["y"].astype(np.float64) - expected)))
    assert err <= 2e-5 * max(1.0, float(np.max(np.abs(expected)))), err


@pytest.mark.gpu
@pytest.mark.parametrize(
    "B, H, S, Skv, D, fused_qkv",
    [
        (2, 3, 77, 77, 48, True),    # ragged query block and key block, D < 64
        (1, 2, 50, 200, 64, False),  # separate Q/K/V, 4 key blocks (last partial), S != Skv
        (3, 4, 128, 128, 64, True),  # BERT's shape per head, two query blocks
        (1, 2, 3, 5, 4, False),      # tiny: one query block, one partial key block, D = 4
        (2, 2, 256, 256, 32, True),  # D of one MFMA column block
        (1, 2, 16, 300, 16, False),  # keys past the old 256 limit
        (2, 2, 40, 33, 64, False),   # one-pass kernel: 33 keys (two waves), S != Skv
        (1, 3, 130, 96, 32, False),  # one-pass kernel: three waves, five query blocks
        (1, 3, 700, 700, 64, True),  # long sequence: 11 query blocks x 11 key blocks
        # many (batch, head) pairs: 576 and 512 workgroups, more than two per CU
        (4, 16, 520, 520, 64, True),
        (2, 32, 500, 500, 48, False),
    ],
)
def test_fused_attention_matches_oracle(B, H, S, Skv, D, fused_qkv, hip_cache):
    g, feeds = attention_graph(B, H, S, Skv, D, fused_qkv)
    _check(g, feeds, hip_cache)


@pytest.mark.gpu
@pytest.mark.parametrize(
    "case",
    [
        dict(mask="causal"),                                 # GPT sample form: Where(mask, -1e4, t)
        dict(mask="causal", fill=-np.inf, keep_true=True),   # -inf fill: blocks past the diagonal skipped
        dict(mask="causal", fill=-3.4028235e38),             # finfo.min fill
        dict(mask="random", keep_true=True),
        dict(mask="input"),
        dict(bias="const", divide=True),
        dict(bias="input"),
        dict(bias="input", mask="causal", fill=-np.inf),
    ],
    ids=lambda c: "-".join(f"{k}={v}" for k, v in c.items()),
)
@pytest.mark.parametrize("opt", ["O2", "O3"])  # separate nodes, then one FusedElementwise program
def test_masked_and_biased_attention(case, opt, hip_cache):
    g, feeds = attention_graph(2, 3, 150, 150, 64, True, scale=0.125, **case)
    _check(g, feeds, hip_cache, opt)


@pytest.mark.gpu
@pytest.mark.parametrize(
    "case",
    [
        dict(mask="causal"),
        dict(mask="causal", fill=-np.inf, keep_true=True),
        dict(mask="random", keep_true=True),
        dict(mask="input"),
        dict(bias="const", divide=True),
        dict(bias="input", mask="causal", fill=-np.inf),
    ],
    ids=lambda c: "-".join(f"{k}={v}" for k, v in c.items()),
)
@pytest.mark.parametrize("S, D", [(100, 64), (37, 24)])
def test_masked_and_biased_short_attention(case, S, D, hip_cache):
    """At most 128 keys: the one-pass kernel (a wave per 32 keys, the last one partly past the
    keys; a partial last query block; D below one or two MFMA column blocks)."""
    g, feeds = attention_graph(2, 3, S, S, D, True, scale=0.125, **case)
    _check(g, feeds, hip_cache)


@pytest.mark.gpu
def test_causal_long_sequence(hip_cache):
    g, feeds = attention_graph(1, 2, 1030, 1030, 64, True, mask="causal", fill=-np.inf)
    _check(g, feeds, hip_cache)


@pytest.mark.gpu
def test_causal_and_biased_many_heads(hip_cache):
    """Score ops with 64 (batch, head) pairs of 520 queries (ragged last query block)."""
    g, feeds = attention_graph(2, 32, 520, 520, 64, True, mask="causal", fill=-np.inf)
    _check(g, feeds, hip_cache)
    g, feeds = attention_graph(2, 32, 520, 520, 64, True, bias="input")
    _check(g, feeds, hip_cache)
    g, feeds = attention_graph(2, 32, 520, 520, 64, True, mask="causal")  # finite fill past the diagonal
    _check(g, feeds, hip_cache)


@pytest.mark.gpu
def test_attention_outside_limits_stays_unfused(hip_cache):
    g, feeds = attention_graph(1, 2, 16, 40, 80, False)  # D > 64
    _check(g, feeds, hip_cache, fused=False)


@pytest.mark.gpu
@pytest.mark.parametrize("sample", ["tiny-bert", "tiny-gpt"])
def test_fused_and_unfused_samples_agree(sample, hip_cache, monkeypatch):
    build = builders.SAMPLES[sample]
    feeds = oracle.random_feeds(build(), 0, int_high=50)
    expected = oracle.run_graph(build(), feeds)
    outs = {}
    for fuse in (True, False):
        monkeypatch.setattr(hip_codegen, "FUSE_ATTENTION", fuse)
        got, kernels = _run(build(), feeds, hip_cache)
        assert kernels.get("attention", 0) == (2 if fuse else 0)
        outs[fuse] = got
    for name, want in expected.items():
        for fuse in (True, False):
            assert float(np.max(np.abs(outs[fuse][name].astype(np.float64) - want))) <= 5e-5


def test_matcher_finds_every_bert_and_gpt_layer():
    """CPU: all 12 BERT-base layers match, each with its QKV projection absorbed (the fused
    call runs it into scratch, so the context, which the planner put where the dead projection
    was, is written in place without staging); the causal GPT sample's Where mask is
    recognized as causal."""
    g = builders.bert_base(1)
    optimize(g, "O3")
    schedule(g)
    found = attn.find_attention(g, plan_memory(g, alignment=256))
    assert len(found) == 12
    assert all(m.S == 128 and m.Skv == 128 and m.D == 64 and m.H == 12 for m in found)
    assert all(abs(m.ops.scale - 0.125) < 1e-7 and m.ops.mask is None for m in found)
    # split, 3 x (reshape, transpose), qk, mul, softmax, pv, merge + the QKV FusedGemm
    assert all(len(m.absorbed) == 13 and len(m.qkv_gemms) == 1 and not m.staged for m in found)
    gpt = builders.tiny_gpt()
    optimize(gpt, "O3")
    schedule(gpt)
    found = attn.find_attention(gpt, plan_memory(gpt, alignment=256))
    assert len(found) == 2
    assert all(m.ops.causal and not m.ops.mask_keep and m.ops.fill == -1e4 for m in found)


@pytest.mark.gpu
@pytest.mark.parametrize("sample", ["tiny-bert", "tiny-gpt"])
def test_staged_output(sample, hip_cache, monkeypatch):
    """With the QKV projection left as its own GEMM, the planner puts each layer's context where
    the dead projection was: the fused call writes scratch and a copy moves the result into
    place. Both builds must match the oracle."""
    g = builders.SAMPLES[sample]()
    optimize(g, "O3")
    schedule(g)
    monkeypatch.setattr(attn, "ABSORB_QKV", False)
    found = attn.find_attention(g, plan_memory(g, alignment=256))
    assert found and all(m.staged and not m.qkv_gemms for m in found)
    build = builders.SAMPLES[sample]
    feeds = oracle.random_feeds(build(), 2, int_high=50)
    expected = oracle.run_graph(build(), feeds)
    for absorb in (False, True):
        monkeypatch.setattr(attn, "ABSORB_QKV", absorb)
        got, kernels = _run(build(), feeds, hip_cache)
        assert kernels.get("attention") == len(found), kernels
        for name, want in expected.items():
            assert float(np.max(np.abs(got[name].astype(np.float64) - want))) <= 5e-5


def test_matcher_score_op_forms():
    """CPU: the score ops the matcher takes, and the ones it leaves unfused."""
    def ops_of(opt="O3", **case):
        g, _ = attention_graph(1, 2, 40, 40, 16, True, **case)
        optimize(g, opt)
        schedule(g)
        found = attn.find_attention(g, plan_memory(g, alignment=256))
        return found[0].ops if found else None

    assert ops_of(divide=True, opt="O0").divide and ops_of(divide=True, opt="O0").scale == 8.0
    assert not ops_of(divide=True).divide  # O3 turns the division by a constant into a product
    m = ops_of(mask="causal", keep_true=True)
    assert m.causal and m.mask_keep
    m = ops_of(mask="random")
    assert not m.causal and m.mask is not None and not m.mask_keep
    assert ops_of(bias="input", opt="O2").bias is not None
    assert ops_of(bias="const", mask="input").mask is not None
    # a mask applied before the bias is not the kernel's order
    g, _ = attention_graph(1, 2, 40, 40, 16, True, mask="causal")
    w = next(n for n in g.nodes if n.op == "Where")
    sm = next(n for n in g.nodes if n.op == "Softmax")
    extra = g.constant(np.full((1, 1, 40, 40), 0.5, np.float32), "late_bias")
    late = g.add_node("Add", [w.output, extra], 1, {}, name="late_add", output_names=["late"], index=g.nodes.index(sm))
    g.set_input(sm, 0, late.output)
    infer_shapes(g)
    optimize(g, "O2")
    schedule(g)
    assert attn.find_attention(g, plan_memory(g, alignment=256)) == []


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [False, True])
def test_grouped_qkv_projection(causal, hip_cache, monkeypatch):
    """Separate Q/K/V projections (the Hugging Face export form) run as one GEMM feeding the
    fused attention: 3 GEMM launches per layer become 1."""
    def build():
        return builders.transformer(gelu="tanh" if causal else "erf", causal=causal, separate_qkv=True, seq=40, batch=2)

    feeds = oracle.random_feeds(build(), 3, int_high=100)
    expected = oracle.run_graph(build(), feeds)
    got, kernels = _run(build(), feeds, hip_cache)
    monkeypatch.setattr(hip_codegen, "FUSE_ATTENTION", False)
    plain, plain_kernels = _run(build(), feeds, hip_cache)
    assert kernels["attention"] == 2 and kernels["gemm"] == plain_kernels["gemm"] - 2 * 2 - 2 * 2
    for name, want in expected.items():
        for out in (got, plain):
            assert float(np.max(np.abs(out[name].astype(np.float64) - want))) <= 5e-5


@pytest.mark.gpu
def test_bert_base_separate_qkv(hip_cache):
    graph = builders.bert_base(2, separate_qkv=True)
    feeds = oracle.random_feeds(graph, 4, int_high=30522)
    got, kernels = _run(builders.bert_base(2, separate_qkv=True), feeds, hip_cache)
    assert kernels["attention"] == 12 and kernels["gemm"] == 48
    for i in (0, 1):
        want = oracle.run_graph(builders.bert_base(1, separate_qkv=True), {"input_ids": feeds["input_ids"][i : i + 1]})["hidden"]
        assert float(np.max(np.abs(got["hidden"][i : i + 1].astype(np.float64) - want))) <= 5e-4


def test_matcher_groups_separate_qkv_projections():
    """CPU: the three projections of one input join the match; with two different inputs
    (cross attention) they do not."""
    g = builders.bert_base(1, separate_qkv=True)
    optimize(g, "O3")
    schedule(g)
    found = attn.find_attention(g, plan_memory(g, alignment=256))
    assert len(found) == 12 and all(len(m.qkv_gemms) == 3 and not m.staged for m in found)
    assert all(m.reads() == [m.qkv_gemms[0].input(0)] for m in found)
    g, _ = attention_graph(1, 2, 40, 40, 16, False)  # Q, K, V are graph inputs: nothing to group
    optimize(g, "O3")
    schedule(g)
    (m,) = attn.find_attention(g, plan_memory(g, alignment=256))
    assert m.qkv_gemms == []
