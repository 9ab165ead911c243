"""Writes tests/golden/onnx/*.onnx (+ .npz) with PyTorch's ONNX exporter.

Run in the build container (CPU only, a minute or so):

    python tests/golden/make_onnx_fixtures.py

Why these files: this build reads ONNX with its own protobuf decoder, and a decoder checked
only against its own encoder would agree with itself on a wrong field number. PyTorch's
TorchScript exporter serializes models with libtorch's compiled copy of the ONNX schema, an
independent writer of the format. The Python onnx package is not installed, and the exporter's
last step only uses it to merge onnx-script functions into the model (there are none in these
models), so that step is replaced by the identity on the bytes libtorch produced.

Each model is exported with deterministic weights; the .npz holds the inputs (``in_<name>``)
and PyTorch's float32 outputs (``out_<name>``) for them. ``manifest.json`` records each file's
opset, the symbolic dimensions it leaves open and the values the tests bind them to.
"""

from __future__ import annotations

import io
import json
import math
from pathlib import Path

import numpy as np
import torch
from torch import nn
from torch.onnx._internal.torchscript_exporter import onnx_proto_utils

OUT = Path(__file__).resolve().parent / "onnx"


class Mlp(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.net = nn.Sequential(nn.Linear(16, 32), nn.ReLU(), nn.Linear(32, 4))

    def forward(self, x):
        return self.net(x)


class Cnn(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.c1 = nn.Conv2d(3, 8, 3, padding=1)
        self.bn = nn.BatchNorm2d(8)
        self.c2 = nn.Conv2d(8, 16, 3, stride=2, padding=1)
        self.fc = nn.Linear(16, 10)

    def forward(self, x):
        y = torch.max_pool2d(torch.relu(self.bn(self.c1(x))), 2)
        y = torch.relu(self.c2(y))
        y = torch.flatten(torch.nn.functional.adaptive_avg_pool2d(y, 1), 1)
        return self.fc(y)


class Encoder(nn.Module):
    """One pre-norm transformer encoder layer written out op by op (4 heads of 8)."""

    def __init__(self, d: int = 32, heads: int = 4, approximate: str = "none") -> None:
        super().__init__()
        self.h, self.dh = heads, d // heads
        self.ln1, self.ln2 = nn.LayerNorm(d), nn.LayerNorm(d)
        self.qkv, self.proj = nn.Linear(d, 3 * d), nn.Linear(d, d)
        self.fc1, self.fc2 = nn.Linear(d, 4 * d), nn.Linear(4 * d, d)
        self.approximate = approximate

    def forward(self, x):
        b, s, d = x.shape
        q, k, v = self.qkv(self.ln1(x)).split(d, dim=-1)
        q = q.reshape(b, s, self.h, self.dh).transpose(1, 2)
        k = k.reshape(b, s, self.h, self.dh).permute(0, 2, 3, 1)
        v = v.reshape(b, s, self.h, self.dh).transpose(1, 2)
        p = torch.softmax(torch.matmul(q, k) / math.sqrt(self.dh), dim=-1)
        o = torch.matmul(p, v).transpose(1, 2).reshape(b, s, d)
        x = x + self.proj(o)
        return x + self.fc2(nn.functional.gelu(self.fc1(self.ln2(x)), approximate=self.approximate))


class TinyGpt(nn.Module):
    """Token + position embedding, one causal attention layer, tied LM head."""

    def __init__(self, vocab: int = 50, d: int = 32, seq: int = 12) -> None:
        super().__init__()
        self.wte, self.wpe = nn.Embedding(vocab, d), nn.Embedding(seq, d)
        self.ln, self.lnf = nn.LayerNorm(d), nn.LayerNorm(d)
        self.attn, self.proj = nn.Linear(d, 3 * d), nn.Linear(d, d)
        self.register_buffer("mask", torch.tril(torch.ones(seq, seq, dtype=torch.bool)))
        self.h = 2

    def forward(self, ids):
        b, s = ids.shape
        x = self.wte(ids) + self.wpe(torch.arange(s))
        d = x.shape[-1]
        q, k, v = self.attn(self.ln(x)).split(d, dim=-1)
        q, k, v = (t.reshape(b, s, self.h, d // self.h).transpose(1, 2) for t in (q, k, v))
        a = torch.matmul(q, k.transpose(-1, -2)) * (1.0 / math.sqrt(d // self.h))
        a = a.masked_fill(~self.mask[:s, :s], float("-inf")).softmax(-1)
        x = x + self.proj(torch.matmul(a, v).transpose(1, 2).reshape(b, s, d))
        x = nn.functional.gelu(self.lnf(x), approximate="tanh")
        return torch.matmul(x, self.wte.weight.t())


class LegacySoftmax(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.fc = nn.Linear(8, 6)

    def forward(self, x):
        y = self.fc(x)
        return torch.softmax(y, dim=-1), torch.log_softmax(y, dim=-1)


def export(model: nn.Module, args: tuple, path: Path, opset: int, inputs: list[str],
           outputs: list[str], dynamic_axes: dict | None = None, fold: bool = True) -> bytes:
    model.eval()
    buf = io.BytesIO()
    with torch.no_grad():
        torch.onnx.export(model, args, buf, dynamo=False, opset_version=opset, input_names=inputs,
                          output_names=outputs, dynamic_axes=dynamic_axes, do_constant_folding=fold)
    data = buf.getvalue()
    path.write_bytes(data)
    return data


def main() -> None:
    onnx_proto_utils._add_onnxscript_fn = lambda model_bytes, custom_opsets: model_bytes
    OUT.mkdir(exist_ok=True)
    manifest = {}

    def case(name, model, feeds, opset, outputs, dynamic_axes=None, dims=None, export_feeds=None,
             fold=True):
        torch.manual_seed(0)
        for p in model.parameters():  # deterministic, non-trivial weights and BN statistics
            p.data = torch.randn_like(p) * 0.3
        for m in model.modules():
            if isinstance(m, nn.BatchNorm2d):
                m.running_mean = torch.randn_like(m.running_mean) * 0.2
                m.running_var = torch.rand_like(m.running_var) + 0.5
        tensors = tuple(torch.from_numpy(v) for v in feeds.values())
        ex = tuple(torch.from_numpy(v) for v in (export_feeds or feeds).values())
        export(model, ex, OUT / f"{name}.onnx", opset, list(feeds), outputs, dynamic_axes, fold)
        with torch.no_grad():
            got = model(*tensors)
        got = got if isinstance(got, tuple) else (got,)
        arrays = {f"in_{k}": v for k, v in feeds.items()}
        arrays.update({f"out_{k}": t.numpy().astype(np.float32) for k, t in zip(outputs, got)})
        np.savez(OUT / f"{name}.npz", **arrays)
        manifest[name] = {"opset": opset, "dims": dims or {}}

    rng = np.random.default_rng(0)
    f32 = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    case("mlp_dynamic_batch", Mlp(), {"x": f32(3, 16)}, 14, ["y"],
         dynamic_axes={"x": {0: "batch"}, "y": {0: "batch"}}, dims={"batch": 3},
         export_feeds={"x": f32(2, 16)})
    case("cnn", Cnn(), {"image": f32(2, 3, 16, 16)}, 13, ["logits"])
    case("encoder_opset17", Encoder(), {"x": f32(2, 10, 32)}, 17, ["y"])
    case("encoder_opset14", Encoder(), {"x": f32(2, 10, 32)}, 14, ["y"])
    # no constant folding: Constant nodes and Shape -> Gather -> Concat -> Reshape arithmetic
    # over a symbolic batch and sequence
    case("encoder_unfolded_dynamic", Encoder(), {"x": f32(2, 10, 32)}, 13, ["y"],
         dynamic_axes={"x": {0: "batch", 1: "sequence"}, "y": {0: "batch", 1: "sequence"}},
         dims={"batch": 2, "sequence": 10}, export_feeds={"x": f32(3, 5, 32)}, fold=False)
    case("encoder_gelu_tanh_opset20", Encoder(approximate="tanh"), {"x": f32(1, 7, 32)}, 20, ["y"])
    case("tiny_gpt", TinyGpt(), {"ids": rng.integers(0, 50, (2, 12)).astype(np.int64)}, 14, ["logits"])
    case("legacy_softmax_opset11", LegacySoftmax(), {"x": f32(5, 8)}, 11, ["p", "logp"])
    (OUT / "manifest.json").write_text(json.dumps(manifest, indent=1, sort_keys=True) + "\n")
    for f in sorted(OUT.iterdir()):
        print(f"{f.name:36s} {f.stat().st_size:8d} bytes")


if __name__ == "__main__":
    main()
