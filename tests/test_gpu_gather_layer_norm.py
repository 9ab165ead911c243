"""An embedding lookup, its addend and the LayerNorm over the sum as one launch
(mgc_hip_gather_layer_norm).

A transformer encoder's input is Gather(token table, ids) + position / segment embeddings ->
LayerNormalization; the reference's C backend runs op_Gather (codegen/c.py:662-688), the Add's
loop nest (c.py:360-529) and mgc_layer_norm. The hip backend runs the three as one launch, a
wavefront per token row. Graph cases compile such a chain at O3, assert the fused launch, compare
with the oracle on the unoptimized graph and bit for bit with the three launches it replaces
(the same single add and the same row LayerNorm code). Cases cover BERT's form (a (1, S, D)
constant addend repeated over the batch), a full-shape addend that is a graph input, a
(D,)-vector addend, int32 and negative indices, the 1024-column limit, a LayerNorm without a
bias, and GPT-2's form, whose sum is also read later as a residual (the launch then stores it). An index out of range raises the Gather error as the unfused gather does; the C-ABI cases
check that shapes, index types and alignments outside the entry point's limits are refused.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from capi import MGC_ERR_ARGS, MGC_OK, Hip, bind
from helpers import compile_hip
from ml_graph_compiler.codegen import hip as hip_codegen
from ml_graph_compiler.codegen.build import load_kernel_library
from ml_graph_compiler.errors import GraphError
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu

ATOL = 2e-5
RTOL = 1e-5


def embed_graph(b: int, s: int, vocab: int, d: int, addend: str, idx_dtype: str, ln_bias: bool,
                residual: bool, seed: int) -> tuple[Graph, dict[str, np.ndarray]]:
    """ids -> Gather(table) -> Add(addend) -> LayerNormalization(gamma[, beta]) [+ the sum, as
    GPT-2's first residual]."""
    rng = np.random.default_rng(seed)
    g = Graph("embed")
    ids = g.add_input("ids", TensorType(idx_dtype, (b, s)))
    table = g.constant(rng.standard_normal((vocab, d)).astype(np.float32), "table")
    y = g.add_node("Gather", [table, ids], 1, {"axis": 0}, name="gather").output
    feeds: dict[str, np.ndarray] = {}
    if addend == "position":
        other = g.constant(rng.standard_normal((1, s, d)).astype(np.float32), "pos")
    elif addend == "input":
        other = g.add_input("extra", TensorType("float32", (b, s, d)))
        feeds["extra"] = rng.standard_normal((b, s, d)).astype(np.float32)
    else:
        other = g.constant(rng.standard_normal(d).astype(np.float32), "vec")
    total = y = g.add_node("Add", [y, other], 1, {}, name="add").output
    gamma = g.constant(rng.uniform(0.5, 1.5, d).astype(np.float32), "gamma")
    inputs = [y, gamma]
    if ln_bias:
        inputs.append(g.constant(rng.normal(0, 0.1, d).astype(np.float32), "beta"))
    y = g.add_node("LayerNormalization", inputs, 1, {"axis": -1, "epsilon": 1e-12}, name="ln").output
    if residual:
        y = g.add_node("Add", [y, total], 1, {}, name="residual").output
    g.add_output(y, "y")
    infer_shapes(g)
    ids_v = rng.integers(-vocab, vocab, (b, s)).astype(np.dtype(idx_dtype))
    feeds["ids"] = ids_v
    return g, feeds


CASES = [
    # (b, s, vocab, d, addend, idx dtype, ln bias, sum read later)
    (3, 128, 1000, 768, "position", "int64", True, False),  # BERT's form, negative indices too
    (2, 17, 50, 1024, "input", "int32", True, False),       # the column limit, a full-shape graph-input addend
    (1, 9, 7, 12, "vector", "int64", False, False),         # three quads per row, no LayerNorm bias
    (2, 64, 300, 768, "position", "int64", True, True),     # GPT-2's form: the sum is also the first residual
]


def _run(g, feeds, cache, fuse: bool, monkeypatch):
    monkeypatch.setattr(hip_codegen, "FUSE_GATHER_LAYER_NORM", fuse)
    model = compile_hip(g, cache, "O3")
    try:
        return model.run(feeds)["y"], dict(model.report.kernels)
    finally:
        model.release()


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_gather_layer_norm_matches_oracle(case, hip_cache, monkeypatch):
    print(f"[gpu] gather + add + layer norm {case}", flush=True)
    g, feeds = embed_graph(*case, seed=sum(case[:4]))
    expected = oracle.run_graph(g, feeds)["y"]
    got, kernels = _run(g, feeds, hip_cache, True, monkeypatch)
    assert kernels.get("gather_layer_norm") == 1 and "gather" not in kernels and "layer_norm" not in kernels, kernels
    np.testing.assert_allclose(got, expected, rtol=RTOL, atol=ATOL)
    g2, _ = embed_graph(*case, seed=sum(case[:4]))
    apart, kernels = _run(g2, feeds, hip_cache, False, monkeypatch)
    assert "gather_layer_norm" not in kernels and kernels.get("gather") == 1, kernels
    np.testing.assert_array_equal(got, apart)


def test_gather_layer_norm_index_out_of_range(hip_cache, monkeypatch):
    print("[gpu] gather + add + layer norm with an index out of range", flush=True)
    g, feeds = embed_graph(2, 8, 16, 64, "position", "int64", True, False, seed=5)
    monkeypatch.setattr(hip_codegen, "FUSE_GATHER_LAYER_NORM", True)
    model = compile_hip(g, hip_cache, "O3")
    try:
        assert model.report.kernels.get("gather_layer_norm") == 1, model.report.kernels
        bad = dict(feeds, ids=np.full((2, 8), 16, np.int64))
        with pytest.raises(GraphError, match="Gather"):
            model.run(bad)
        ok = model.run(feeds)["y"]  # the flag was cleared when the error was reported
        np.testing.assert_allclose(ok, oracle.run_graph(g, feeds)["y"], rtol=RTOL, atol=ATOL)
    finally:
        model.release()


class GatherLnArgs(ctypes.Structure):
    """mgc_hip_gather_ln_args."""

    _fields_ = [
        ("table", ctypes.c_void_p), ("dim", ctypes.c_long), ("idx", ctypes.c_void_p), ("idx_dtype", ctypes.c_int),
        ("addend", ctypes.c_void_p), ("add_rows", ctypes.c_long), ("scale", ctypes.c_void_p),
        ("bias", ctypes.c_void_p), ("eps", ctypes.c_float), ("out", ctypes.c_void_p), ("rows", ctypes.c_long),
        ("cols", ctypes.c_int), ("sum", ctypes.c_void_p),
    ]


def test_gather_layer_norm_entry_point_refuses_unsupported():
    lib = load_kernel_library()
    bind(lib)
    lib.mgc_hip_gather_layer_norm.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip = Hip()
    x = lib.mgc_hip_exec_create(None)
    assert x, lib.mgc_hip_last_error()
    try:
        table, out = hip.alloc(4 * 8 * 1100), hip.alloc(4 * 4 * 1100)
        idx = hip.upload(np.zeros(4, np.int64))
        ok = dict(table=table, dim=8, idx=idx, idx_dtype=2, addend=None, add_rows=0, scale=None, bias=None,
                  eps=1e-5, out=out, rows=4, cols=64)
        for bad in (dict(cols=66), dict(cols=1028), dict(out=out + 4), dict(idx_dtype=0), dict(dim=0),
                    dict(addend=table, add_rows=0), dict(sum=out + 8)):
            a = GatherLnArgs(**{**ok, **bad})
            lib.mgc_hip_gather_layer_norm(x, ctypes.byref(a))
            assert lib.mgc_hip_exec_status(x) == MGC_ERR_ARGS, bad
        a = GatherLnArgs(**{**ok, "rows": 0})  # no rows: nothing to do
        lib.mgc_hip_gather_layer_norm(x, ctypes.byref(a))
        assert lib.mgc_hip_exec_status(x) == MGC_OK, lib.mgc_hip_last_error()
    finally:
        lib.mgc_hip_exec_destroy(x)
        hip.free()
