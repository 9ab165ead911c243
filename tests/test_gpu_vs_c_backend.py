"""The hip backend against the reference's own generated-C backend on the same inputs.

The C side is the reference's mgc_kernels.c driven by its emitter's lowering (oracle/cbackend.py),
prebuilt per workload into oracle/_ref (the same libraries bench.py times as its CPU baseline);
it runs on the host of the GPU box. Both compile the same O3 graph (same seeded weights); the
bounds are the north-star tolerances: 1e-4 max-abs for the CNNs (relative to max|logit| for
ResNet-50, whose random-weight logits reach ~1e4), 5e-4 for BERT, integer outputs exact.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip
from ml_graph_compiler import builders
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu

CASES = {
    "single_gemm": ("y", 1e-4, False),
    "bottleneck": ("y", 1e-4, False),
    "mobilenet_v2": ("logits", 1e-4, False),
    "resnet50": ("logits", 1e-5, True),   # relative to max|logit|
    "bert_base": ("hidden", 5e-4, False),
}


@pytest.mark.parametrize("workload", sorted(CASES))
def test_hip_matches_reference_c_backend(workload, hip_cache):
    from oracle import cbackend

    try:
        cmodel, graph, meta = cbackend.load_baseline(workload)
    except (OSError, cbackend.CBackendError) as exc:
        pytest.skip(f"prebuilt reference C backend for {workload} unavailable: {exc}")
    out, tol, relative = CASES[workload]
    print(f"[gpu] {workload} b{meta['batch']} hip vs reference C backend", flush=True)
    feeds = oracle.random_feeds(graph, 9, int_high=30522 if workload == "bert_base" else 100)
    want = cmodel.run(feeds)[out].astype(np.float64)
    build = builders.single_gemm if workload == "single_gemm" else builders.CONFIGS[workload]
    model = compile_hip(build() if workload == "single_gemm" else build(batch=meta["batch"]), hip_cache)
    try:
        got = model.run(feeds)[out]
    finally:
        model.release()
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    scale = float(np.max(np.abs(want)))
    print(f"[gpu] {workload}: max-abs {err:.3e} (max|ref| {scale:.3e})", flush=True)
    assert err <= tol * (scale if relative else 1.0)
    if out == "logits":
        assert np.array_equal(np.argmax(got, axis=-1), np.argmax(want, axis=-1))
