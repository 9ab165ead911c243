"""ONNX files compiled end to end on the GPU: ``compile_model(path)`` and ``mgc compile``.

The files are the ones PyTorch's exporter wrote (tests/golden/onnx); each compiled model must
reproduce both PyTorch's float32 outputs and the oracle interpreter run on the imported graph.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from ml_graph_compiler.cli import main as cli_main
from ml_graph_compiler.codegen import compile_model
from ml_graph_compiler.onnx_import import from_onnx
from oracle import interpreter as oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "onnx"
MANIFEST = json.loads((GOLDEN / "manifest.json").read_text())


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_torch_exported_model_compiles_and_matches(name, hip_cache):
    path = GOLDEN / f"{name}.onnx"
    z = np.load(GOLDEN / f"{name}.npz")
    feeds = {k[3:]: z[k] for k in z.files if k.startswith("in_")}
    expected = oracle.run_graph(from_onnx(path, dims=MANIFEST[name]["dims"]), feeds)
    model = compile_model(path, dims=MANIFEST[name]["dims"], cache_dir=hip_cache)
    try:
        got = model.run(feeds)
    finally:
        model.release()
    for k in z.files:
        if not k.startswith("out_"):
            continue
        out, torch_out = got[k[4:]].astype(np.float64), z[k]
        scale = max(1.0, float(np.max(np.abs(torch_out))))
        assert float(np.max(np.abs(out - expected[k[4:]]))) <= 2e-5 * scale, k
        assert float(np.max(np.abs(out - torch_out))) <= 2e-5 * scale, k


@pytest.mark.gpu
def test_cli_compile_onnx_file(tmp_path, capsys, hip_cache):
    path = GOLDEN / "encoder_unfolded_dynamic.onnx"
    argv = ["compile", str(path), "--dim", "batch=4", "--dim", "sequence=16", "--check", "--bench", "3",
            "--cache-dir", str(hip_cache), "-o", str(tmp_path / "saved"), "--json"]
    assert cli_main(argv) == 0
    payload = json.loads(capsys.readouterr().out)
    assert payload["backend"] == "hip" and payload["max_abs_diff_vs_interpreter"] <= 1e-4
    assert payload["outputs"]["y"].startswith("float32[4, 16, 32]")
    assert (tmp_path / "saved" / "model.json").exists() and payload["latency_ms_min"] > 0
