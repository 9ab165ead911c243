"""The oracle against vectors the reference's own operator semantics produced.

tests/golden/reference_ops.{npz,json} were written by tests/golden/make_reference_op_fixtures.py,
which ran the reference's numpy ``ops.run`` (src/ml_graph_compiler/ops.py:122-1202) on seeded
inputs for every operator the oracle implements (212 cases: broadcasting, integer and float
dtypes, omitted optional inputs, attribute and input forms of the same parameter, edge cases
such as truncating integer Div, first-max ArgMax ties, negative Gather indices, empty Range).
Integer and bool outputs must match exactly; float outputs within ``ULPS`` units in the last
place, except where the oracle accumulates in float64 on purpose and the reference in float32
— the contractions (np.matmul / einsum) and average pooling (a float32 window sum,
ops.py:1091-1124): there the bound is fp32 accumulation error.
"""

from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest

from oracle import interpreter as oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
MANIFEST = json.loads((GOLDEN / "reference_ops.json").read_text())
ACCUMULATING = {"MatMul", "Gemm", "FusedGemm", "Conv", "FusedConv", "AveragePool"}
ULPS = 2


def decode_attrs(attrs: dict) -> dict:
    out = {}
    for k, v in attrs.items():
        if isinstance(v, dict) and "__array__" in v:
            out[k] = np.asarray(v["__array__"], dtype=v["dtype"])
        else:
            out[k] = v
    return out


def load_case(case: dict, arrays) -> tuple[list, list]:
    inputs = [arrays[f"{case['name']}/in{i}"] if present else None for i, present in enumerate(case["inputs"])]
    outputs = [arrays[f"{case['name']}/out{j}"] for j in range(case["outputs"])]
    return inputs, outputs


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Units in the last place between two float arrays of one dtype (NaN == NaN counts as 0)."""
    bits = {np.dtype(np.float32): np.int32, np.dtype(np.float64): np.int64}[a.dtype]
    ia, ib = a.view(bits).astype(np.int64), b.view(bits).astype(np.int64)
    # map the sign-magnitude float order onto a monotonic integer line
    top = np.int64(np.iinfo(bits).min)
    ia = np.where(ia < 0, top - ia, ia)
    ib = np.where(ib < 0, top - ib, ib)
    d = np.abs(ia - ib)
    return np.where(np.isnan(a) & np.isnan(b), 0, d)


def compare(op: str, got: np.ndarray, want: np.ndarray, label: str) -> None:
    got = np.asarray(got)
    assert got.shape == want.shape, (label, got.shape, want.shape)
    assert got.dtype == want.dtype, (label, got.dtype, want.dtype)
    if not np.issubdtype(want.dtype, np.floating):
        np.testing.assert_array_equal(got, want, err_msg=label)
    elif op in ACCUMULATING:
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-6, err_msg=label)
    else:
        assert np.array_equal(np.isnan(got), np.isnan(want)), label
        worst = int(ulp_distance(got, want).max()) if got.size else 0
        assert worst <= ULPS, f"{label}: {worst} ulp"


@pytest.fixture(scope="module")
def arrays():
    with np.load(GOLDEN / "reference_ops.npz", allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def test_every_oracle_operator_has_reference_vectors():
    covered = {c["op"] for c in MANIFEST}
    assert set(oracle.OPS) <= covered, sorted(set(oracle.OPS) - covered)


@pytest.mark.parametrize("case", MANIFEST, ids=[c["name"] for c in MANIFEST])
def test_oracle_matches_reference_ops(case, arrays):
    inputs, want = load_case(case, arrays)
    node = SimpleNamespace(op=case["op"], attrs=decode_attrs(case["attrs"]), outputs=[None] * case["outputs"],
                           name=case["name"])
    got = oracle.run_node(node, [None if a is None else a.copy() for a in inputs])
    assert len(got) == len(want)
    for j, (g, w) in enumerate(zip(got, want)):
        compare(case["op"], g, w, f"{case['name']} output {j}")


def test_ulp_distance_known_answers():
    one = np.asarray([1.0], np.float32)
    nxt = np.nextafter(one, np.float32(2))
    assert int(ulp_distance(one, nxt)[0]) == 1
    neg = np.asarray([-0.0], np.float32)
    assert int(ulp_distance(np.asarray([0.0], np.float32), neg)[0]) == 0
    tiny = np.asarray([np.float32(1e-45)], np.float32)
    assert int(ulp_distance(tiny, -tiny)[0]) == 2


@pytest.mark.parametrize("case", MANIFEST, ids=[c["name"] for c in MANIFEST])
def test_compiler_evaluator_and_shape_rules_match_reference_ops(case, arrays):
    """The compiler's own operator table (constant folding evaluates through ``ops.run``, shape
    inference through ``ops.infer``) against the same reference vectors: every output type, and
    every output value within the bounds above."""
    from ml_graph_compiler import ops
    from ml_graph_compiler.ir import Node, TensorType, Value

    inputs, want = load_case(case, arrays)
    node = Node(case["op"], [None] * len(inputs), [Value(f"o{j}") for j in range(case["outputs"])],
                decode_attrs(case["attrs"]), name=case["name"])
    types = [None if a is None else TensorType.of(a) for a in inputs]
    consts = [a if (i in case["const"] and a is not None) else None for i, a in enumerate(inputs)]
    inferred = ops.infer(node, types, consts)
    assert [(t.dtype, t.shape) for t in inferred] == [(w.dtype.name, w.shape) for w in want]
    got = ops.run(node, [None if a is None else a.copy() for a in inputs])
    for j, (g, w) in enumerate(zip(got, want)):
        compare(case["op"], g, w, f"{case['name']} output {j}")
