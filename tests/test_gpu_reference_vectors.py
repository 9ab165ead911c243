"""The hip backend against vectors the reference's own operator semantics produced.

Every case of tests/golden/reference_ops.{npz,json} (written by
tests/golden/make_reference_op_fixtures.py from the reference's numpy ``ops.run``) is compiled
as a one-operator graph at O0 — the inputs the case marks constant become graph constants, the
others graph inputs — and run on the GPU. Integer, bool and pure data-movement outputs must
equal the reference's bit for bit; float outputs within rtol 1e-4 / atol 1e-5 (fp32 kernels
against numpy, as the other operator tests). Cases the reference's C backend rejects too are
checked for the same CodegenError (no GPU needed) in tests/test_codegen_cpu.py.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip, op_graph
from test_gpu_ops import COPY_OPS
from test_reference_op_vectors import MANIFEST, decode_attrs, load_case

pytestmark = pytest.mark.gpu

# the reference's C backend rejects these as well (tests/test_codegen.py:616-619 for Trilu;
# c.py _require_f32 for non-float32 MatMul)
UNSUPPORTED = {"Trilu_upper": "Trilu", "Trilu_lower_k": "Trilu", "Trilu_upper_negk": "Trilu",
               "MatMul_i64": "int64"}
CASES = [c for c in MANIFEST if c["name"] not in UNSUPPORTED]


@pytest.fixture(scope="module")
def arrays():
    with np.load(__import__("pathlib").Path(__file__).parent / "golden" / "reference_ops.npz") as data:
        return {k: data[k] for k in data.files}


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_hip_matches_reference_vectors(case, arrays, hip_cache):
    inputs, want = load_case(case, arrays)
    g, feeds = op_graph(case["op"], inputs, const=set(case["const"]), attrs=decode_attrs(case["attrs"]),
                        n_outputs=case["outputs"])
    model = compile_hip(g, hip_cache, "O0")
    try:
        got = model.run(feeds)
    finally:
        model.release()
    exact = case["op"] in COPY_OPS or case["op"] in ("Split", "Concat", "Dropout", "Cast", "Reshape", "Where",
                                                       "Neg", "Abs", "Relu", "Floor", "Ceil", "Max", "Min", "Clip")
    for j, w in enumerate(want):
        label = f"{case['name']} output {j}"
        y = got[f"out{j}"]
        assert y.shape == w.shape and y.dtype == w.dtype, (label, y.shape, y.dtype, w.shape, w.dtype)
        if np.issubdtype(w.dtype, np.floating) and not exact:
            np.testing.assert_allclose(y, w, rtol=1e-4, atol=1e-5, err_msg=label)
        else:
            np.testing.assert_array_equal(y, w, err_msg=label)
