"""The hip backend against the reference's own generated-C backend on the same inputs.

The C side is the reference's mgc_kernels.c driven by its emitter's lowering (oracle/cbackend.py),
prebuilt per workload and batch into oracle/_ref (the libraries bench.py times as its CPU
baseline); it runs on the host of the GPU box. Both compile the same O3 graph (same seeded
weights) at batch 1 and at the GPU batch of each BASELINE config, and every element of the batch
is compared. Bounds: 1e-4 max-abs for the CNNs, 5e-4 for BERT and GPT-2 (the north-star
tolerances for transformers; GPT-2's logits must also agree on the arg-max of every position); for
ResNet-50, whose random-weight logits reach ~4e4, 2e-6 of max|logit| (both backends sit ~5e-7
from the float64 oracle there). Logits must have the same arg-max in every row.

A missing prebuilt library is a failure, not a skip: __graft_entry__.build() makes them where
the reference exists and they travel with the tree.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip
from ml_graph_compiler import builders
from oracle import cbackend
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu

CASES = {
    "single_gemm": ("y", 1e-4, False),
    "bottleneck": ("y", 1e-4, False),
    "mobilenet_v2": ("logits", 1e-4, False),
    "resnet50": ("logits", 2e-6, True),   # relative to max|logit|
    "bert_base": ("hidden", 5e-4, False),
    "gpt2": ("logits", 5e-4, False),
}
VOCAB = {"bert_base": 30522, "gpt2": 50257}
PAIRS = [(wl, b) for wl in sorted(CASES) for b in cbackend.BASELINES[wl]]


@pytest.mark.parametrize("workload, batch", PAIRS)
def test_hip_matches_reference_c_backend(workload, batch, hip_cache):
    print(f"[gpu] {workload} b{batch} hip vs reference C backend", flush=True)
    cmodel, graph, meta = cbackend.load_baseline(workload, batch)
    assert meta["batch"] == batch
    out, tol, relative = CASES[workload]
    feeds = oracle.random_feeds(graph, 9, int_high=VOCAB.get(workload, 100))
    want = cmodel.run(feeds)[out].astype(np.float64)
    build = builders.single_gemm() if workload == "single_gemm" else builders.CONFIGS[workload](batch=batch)
    model = compile_hip(build, hip_cache)
    try:
        got = model.run(feeds)[out]
    finally:
        model.release()
    assert got.shape == want.shape
    diff = np.abs(got.astype(np.float64) - want)
    per_item = diff.reshape(diff.shape[0], -1).max(axis=1)
    scale = float(np.max(np.abs(want)))
    bound = tol * (scale if relative else 1.0)
    print(f"[gpu] {workload} b{batch}: max-abs {per_item.max():.3e} over {len(per_item)} elements "
          f"(max|ref| {scale:.3e}, bound {bound:.3e})", flush=True)
    assert np.all(per_item <= bound), per_item.tolist()
    if out == "logits":
        assert np.array_equal(np.argmax(got, axis=-1), np.argmax(want, axis=-1))
