"""A LayerNormalization fused into the split-K reduction of the FusedGemm right before it
(mgc_hip_gemm_layer_norm): BERT's post-LN pattern (the GEMM output feeds only the LayerNorm,
so it is never stored) and GPT-2's pre-LN pattern (the GEMM output is also the next residual,
so the reduction stores it too), against the oracle and against the unfused build.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import compile_hip
from ml_graph_compiler.codegen import build as native
from ml_graph_compiler.codegen import hip as hip_codegen
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.passes import optimize
from ml_graph_compiler.schedule import schedule
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle


def gemm_ln_graph(B: int, S: int, K: int, N: int, second_reader: bool = False, residual: bool = True,
                  ln_bias: bool = True, seed: int = 5):
    """y = x W + b (+ r); z = LayerNorm(y); outputs z (and Relu(y) when ``second_reader``)."""
    rng = np.random.default_rng(seed)
    g = Graph("gemm_ln")
    x = g.add_input("x", TensorType("float32", (B, S, K)))
    feeds = {"x": rng.standard_normal((B, S, K)).astype(np.float32)}
    w = g.constant((rng.standard_normal((K, N)) * 0.05).astype(np.float32), "w")
    b = g.constant((rng.standard_normal(N) * 0.1).astype(np.float32), "b")
    y = g.add_node("MatMul", [x, w], 1, {}, name="mm").output
    y = g.add_node("Add", [y, b], 1, {}, name="bias").output
    if residual:
        r = g.add_input("r", TensorType("float32", (B, S, N)))
        feeds["r"] = rng.standard_normal((B, S, N)).astype(np.float32)
        y = g.add_node("Add", [y, r], 1, {}, name="res").output
    scale = g.constant((rng.random(N) + 0.5).astype(np.float32), "ln_scale")
    inputs = [y, scale] + ([g.constant((rng.standard_normal(N) * 0.1).astype(np.float32), "ln_bias")] if ln_bias else [])
    z = g.add_node("LayerNormalization", inputs, 1, {"axis": -1, "epsilon": 1e-5}, name="ln").output
    g.add_output(z, "z")
    if second_reader:
        g.add_output(g.add_node("Relu", [y], 1, {}, name="relu").output, "y_relu")
    infer_shapes(g)
    return g, feeds


CASES = {
    "bert_post_ln": (2, 64, 768, 768, False, True, True),
    "gpt_pre_ln": (2, 33, 256, 512, True, True, True),   # GEMM output stored for a second reader
    "no_residual_no_bias": (1, 50, 96, 132, False, False, False),
    "long_k": (1, 40, 3072, 768, False, True, True),     # the library's own split (K >= 2048)
    "widest_row": (1, 17, 64, 1024, False, True, True),
    "ragged_k": (3, 7, 20, 12, False, True, True),       # K below one 32-wide stage per split
}


def test_fusion_is_chosen():
    """CPU: each case fuses (the kernel library answers the workspace query), wider rows and
    rows not a multiple of four do not."""
    for name, case in CASES.items():
        g, _ = gemm_ln_graph(*case)
        optimize(g, "O3")
        schedule(g)
        gen = hip_codegen.generate_hip(g, gemm_workspace=native.gemm_workspace_floats,
                                       gemm_ln_workspace=native.gemm_layer_norm_workspace_floats)
        assert gen.kernels.get("gemm_layer_norm") == 1 and "layer_norm" not in gen.kernels, (name, gen.kernels)
    for n in (1028, 130):
        g, _ = gemm_ln_graph(1, 8, 32, n)
        optimize(g, "O3")
        schedule(g)
        gen = hip_codegen.generate_hip(g, gemm_workspace=native.gemm_workspace_floats,
                                       gemm_ln_workspace=native.gemm_layer_norm_workspace_floats)
        assert "gemm_layer_norm" not in gen.kernels and gen.kernels.get("layer_norm") == 1, (n, gen.kernels)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_gemm_layer_norm_matches_oracle(name, hip_cache, monkeypatch):
    case = CASES[name]
    g, feeds = gemm_ln_graph(*case)
    want = oracle.run_graph(g, feeds)
    got = {}
    for fuse in (True, False):
        monkeypatch.setattr(hip_codegen, "FUSE_GEMM_LAYER_NORM", fuse)
        model = compile_hip(gemm_ln_graph(*case)[0], hip_cache, "O3")
        try:
            got[fuse] = model.run(feeds)
            assert ("gemm_layer_norm" in model.report.kernels) == fuse, model.report.kernels
        finally:
            model.release()
    for out, w in want.items():
        for fuse in (True, False):
            err = float(np.max(np.abs(got[fuse][out].astype(np.float64) - w)))
            assert err <= 5e-5 * max(1.0, float(np.abs(w).max())), (out, fuse, err)
        assert float(np.max(np.abs(got[True][out] - got[False][out]))) <= 2e-5 * max(1.0, float(np.abs(w).max()))
