"""Model builders that construct IR graphs directly (the `onnx` package is not available).

Each builder emits the operator patterns a torch.onnx export at opset 14 produces, the way the
reference's samples do (src/ml_graph_compiler/samples.py:1-253): Conv + BatchNormalization +
Relu blocks with residual adds, depthwise convolutions with Clip(0, 6), decomposed LayerNorm,
erf and tanh GELU subgraphs, Shape-driven Reshape targets, a fused QKV projection with Split and
a tied embedding head. Graphs come back typed (shape inference has run) and unoptimized (O0).

``SAMPLES`` mirrors the reference's bundled samples; ``CONFIGS`` are the benchmark workloads:
single_gemm, bottleneck, resnet50, mobilenet_v2, bert_base.
"""

from __future__ import annotations

import math
from collections.abc import Callable
from typing import Any

import numpy as np

from .ir import Graph, TensorType, Value
from .shape_inference import infer_shapes


class GraphBuilder:
    """Appends nodes to a Graph with ONNX-style naming (``{hint}_{count}``)."""

    def __init__(self, name: str, seed: int) -> None:
        self.graph = Graph(name)
        self.graph.opset = 14
        self.rng = np.random.default_rng(seed)
        self.count = 0

    def name(self, hint: str) -> str:
        self.count += 1
        return f"{hint}_{self.count}"

    def input(self, name: str, dtype: str, shape: tuple[int, ...]) -> Value:
        return self.graph.add_input(name, TensorType(dtype, tuple(shape)))

    def const(self, array: np.ndarray, hint: str = "w") -> Value:
        return self.graph.constant(np.asarray(array), self.name(hint))

    def weight(self, shape: tuple[int, ...], scale: float | None = None, hint: str = "w") -> Value:
        """Normal weights; default scale 1 / sqrt(fan_in) like the reference samples."""
        fan_in = int(np.prod(shape[1:])) if len(shape) > 1 else shape[0]
        s = scale if scale is not None else 1.0 / math.sqrt(max(fan_in, 1))
        return self.const((self.rng.standard_normal(shape) * s).astype(np.float32), hint)

    def scalar(self, value: float) -> Value:
        return self.const(np.asarray(value, dtype=np.float32), "s")

    def op(self, op: str, inputs: list[Value | None], n_out: int = 1, **attrs: Any) -> list[Value]:
        out_names = [self.name(op.lower()) for _ in range(n_out)]
        node = self.graph.add_node(op, inputs, n_out, attrs, name=self.name(op), output_names=out_names)
        return node.outputs

    def op1(self, op: str, inputs: list[Value | None], **attrs: Any) -> Value:
        return self.op(op, inputs, 1, **attrs)[0]

    def finish(self, outputs: list[tuple[str, Value]]) -> Graph:
        for name, v in outputs:
            self.graph.add_output(v, name)
        infer_shapes(self.graph)
        self.graph.verify()
        return self.graph


# ---------------------------------------------------------------------------------------------
# the reference's bundled samples, rebuilt in the IR
# ---------------------------------------------------------------------------------------------
def mlp(batch: int = 4, sizes: tuple[int, ...] = (16, 32, 32, 10), seed: int = 0) -> Graph:
    """MatMul + Add + Relu layers, then Softmax."""
    b = GraphBuilder("mlp", seed)
    x = b.input("x", "float32", (batch, sizes[0]))
    for i in range(len(sizes) - 1):
        x = b.op1("MatMul", [x, b.weight((sizes[i], sizes[i + 1]))])
        x = b.op1("Add", [x, b.weight((sizes[i + 1],), 0.1)])
        if i < len(sizes) - 2:
            x = b.op1("Relu", [x])
    return b.finish([("y", b.op1("Softmax", [x], axis=-1))])


def _conv_bn_sample(b: GraphBuilder, x: Value, cin: int, cout: int, k: int, stride: int = 1, group: int = 1) -> Value:
    w = b.weight((cout, cin // group, k, k))
    y = b.op1("Conv", [x, w], kernel_shape=[k, k], strides=[stride, stride], pads=[k // 2] * 4, group=group)
    scale = b.const((1.0 + 0.1 * b.rng.standard_normal(cout)).astype(np.float32), "bn_s")
    bias = b.const((0.1 * b.rng.standard_normal(cout)).astype(np.float32), "bn_b")
    mean = b.const((0.1 * b.rng.standard_normal(cout)).astype(np.float32), "bn_m")
    var = b.const((0.5 + b.rng.random(cout)).astype(np.float32), "bn_v")
    return b.op1("BatchNormalization", [y, scale, bias, mean, var], epsilon=1e-5)


def tiny_cnn(batch: int = 1, size: int = 32, channels: int = 16, classes: int = 10, seed: int = 0) -> Graph:
    """Stem, residual block, inverted residual with depthwise + ReLU6, strided block, head."""
    b = GraphBuilder("tiny_cnn", seed)
    image = b.input("image", "float32", (batch, 3, size, size))
    x = b.op1("Relu", [_conv_bn_sample(b, image, 3, channels, 3, stride=2)])
    x = b.op1("MaxPool", [x], kernel_shape=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1])
    y = b.op1("Relu", [_conv_bn_sample(b, x, channels, channels, 3)])
    y = _conv_bn_sample(b, y, channels, channels, 3)
    x = b.op1("Relu", [b.op1("Add", [y, x])])
    lo, hi = b.scalar(0.0), b.scalar(6.0)
    e = b.op1("Clip", [_conv_bn_sample(b, x, channels, channels * 2, 1), lo, hi])
    e = b.op1("Clip", [_conv_bn_sample(b, e, channels * 2, channels * 2, 3, group=channels * 2), lo, hi])
    e = _conv_bn_sample(b, e, channels * 2, channels, 1)
    x = b.op1("Add", [x, e])
    y = b.op1("Relu", [_conv_bn_sample(b, x, channels, channels * 2, 3, stride=2)])
    y = _conv_bn_sample(b, y, channels * 2, channels * 2, 3)
    shortcut = _conv_bn_sample(b, x, channels, channels * 2, 1, stride=2)
    x = b.op1("Relu", [b.op1("Add", [y, shortcut])])
    x = b.op1("GlobalAveragePool", [x])
    x = b.op1("Flatten", [x], axis=1)
    logits = b.op1("Gemm", [x, b.weight((classes, channels * 2)), b.weight((classes,), 0.1)], transB=1)
    return b.finish([("logits", logits)])


def _layer_norm_pattern(b: GraphBuilder, x: Value, d: int, gamma: np.ndarray, beta: np.ndarray, eps: float) -> Value:
    """LayerNorm as torch.onnx exports it below opset 17."""
    mean = b.op1("ReduceMean", [x], axes=[-1], keepdims=1)
    diff = b.op1("Sub", [x, mean])
    var = b.op1("ReduceMean", [b.op1("Pow", [diff, b.scalar(2.0)])], axes=[-1], keepdims=1)
    std = b.op1("Sqrt", [b.op1("Add", [var, b.scalar(eps)])])
    y = b.op1("Div", [diff, std])
    return b.op1("Add", [b.op1("Mul", [y, b.const(gamma, "ln_g")]), b.const(beta, "ln_b")])


def _sample_ln(b: GraphBuilder, x: Value, d: int) -> Value:
    gamma = (1.0 + 0.1 * b.rng.standard_normal(d)).astype(np.float32)
    beta = (0.1 * b.rng.standard_normal(d)).astype(np.float32)
    return _layer_norm_pattern(b, x, d, gamma, beta, 1e-5)


def _gelu_pattern(b: GraphBuilder, x: Value, kind: str) -> Value:
    if kind == "erf":  # BERT: x * 0.5 * (1 + erf(x / sqrt(2)))
        e = b.op1("Erf", [b.op1("Div", [x, b.scalar(math.sqrt(2.0))])])
        return b.op1("Mul", [b.op1("Mul", [x, b.op1("Add", [e, b.scalar(1.0)])]), b.scalar(0.5)])
    # GPT-2: 0.5 * x * (1 + tanh(sqrt(2 / pi) * (x + 0.044715 * x^3)))
    cube = b.op1("Pow", [x, b.scalar(3.0)])
    inner = b.op1("Add", [x, b.op1("Mul", [b.scalar(0.044715), cube])])
    t = b.op1("Tanh", [b.op1("Mul", [b.scalar(math.sqrt(2.0 / math.pi)), inner])])
    return b.op1("Mul", [b.op1("Mul", [b.scalar(0.5), x]), b.op1("Add", [b.scalar(1.0), t])])


def _dynamic_reshape(b: GraphBuilder, x: Value, tail: list[int]) -> Value:
    """Reshape whose target is computed from Shape, as torch.onnx exports it."""
    shape = b.op1("Shape", [x])
    dims = [
        b.op1(
            "Unsqueeze",
            [
                b.op1("Gather", [shape, b.const(np.asarray(i, np.int64), "i")], axis=0),
                b.const(np.asarray([0], np.int64), "ax"),
            ],
        )
        for i in (0, 1)
    ]
    target = b.op1("Concat", [*dims, b.const(np.asarray(tail, np.int64), "tail")], axis=0)
    return b.op1("Reshape", [x, target])


def transformer(
    batch: int = 1,
    seq: int = 8,
    d_model: int = 32,
    heads: int = 4,
    layers: int = 2,
    vocab: int = 128,
    gelu: str = "tanh",
    causal: bool = True,
    seed: int = 0,
    weight_scale: float | None = None,
    unit_layer_norm: bool = False,
    embedding_norm: bool = False,
    lm_head: bool = True,
    ln_eps: float = 1e-5,
    name: str = "tiny_transformer",
    separate_qkv: bool = False,
) -> Graph:
    """Pre-LN causal tanh-GELU (GPT-2 style) or post-LN erf-GELU (BERT style) encoder.

    With the defaults this is the reference's tiny_transformer sample. ``weight_scale`` fixes
    the std of every weight (BERT config: 0.02); ``unit_layer_norm`` makes every LN gamma 1 and
    beta 0; ``embedding_norm`` adds BERT's LayerNorm after the embeddings; ``lm_head`` adds the
    tied vocabulary projection (otherwise the output is the last hidden state);
    ``separate_qkv`` projects Q, K and V with three Dense layers, as Hugging Face models export,
    instead of one Dense and a Split.
    """
    b = GraphBuilder(name, seed)
    ids = b.input("input_ids", "int64", (batch, seq))
    dh = d_model // heads

    def w(shape: tuple[int, ...], scale: float | None = None, hint: str = "w") -> Value:
        return b.weight(shape, weight_scale if weight_scale is not None else scale, hint)

    def ln(x: Value) -> Value:
        if unit_layer_norm:
            return _layer_norm_pattern(b, x, d_model, np.ones(d_model, np.float32), np.zeros(d_model, np.float32), ln_eps)
        return _sample_ln(b, x, d_model)

    def dense(x: Value, din: int, dout: int) -> Value:
        return b.op1("Add", [b.op1("MatMul", [x, w((din, dout))]), w((dout,), 0.02)])

    wte = w((vocab, d_model), 0.1, "wte")
    wpe = w((seq, d_model), 0.1, "wpe")
    x = b.op1("Gather", [wte, ids], axis=0)
    positions = b.const(np.arange(seq, dtype=np.int64)[None, :], "pos")
    x = b.op1("Add", [x, b.op1("Gather", [wpe, positions], axis=0)])
    if embedding_norm:
        x = ln(x)
    mask = np.triu(np.ones((seq, seq), dtype=bool), 1)[None, None]
    pre_ln = gelu == "tanh"
    for _ in range(layers):
        h = ln(x) if pre_ln else x
        if separate_qkv:
            q, k, v = (dense(h, d_model, d_model) for _ in range(3))
        else:
            qkv = dense(h, d_model, 3 * d_model)
            q, k, v = b.op("Split", [qkv, b.const(np.asarray([d_model] * 3, np.int64), "split")], 3, axis=-1)

        def heads_first(t: Value) -> Value:
            return b.op1("Transpose", [_dynamic_reshape(b, t, [heads, dh])], perm=[0, 2, 1, 3])

        q, k, v = heads_first(q), heads_first(k), heads_first(v)
        kt = b.op1("Transpose", [k], perm=[0, 1, 3, 2])
        scores = b.op1("Div", [b.op1("MatMul", [q, kt]), b.scalar(math.sqrt(dh))])
        if causal:
            neg = b.const(np.asarray(-1e4, dtype=np.float32), "neg")
            scores = b.op1("Where", [b.const(mask, "mask"), neg, scores])
        else:
            ones = b.const(np.ones((batch, 1, 1, seq), np.float32))
            zero_mask = b.op1("Mul", [b.op1("Sub", [b.scalar(1.0), ones]), b.scalar(-1e4)])
            scores = b.op1("Add", [scores, zero_mask])
        attn = b.op1("MatMul", [b.op1("Softmax", [scores], axis=-1), v])
        attn = b.op1("Transpose", [attn], perm=[0, 2, 1, 3])
        attn = dense(_dynamic_reshape(b, attn, [d_model]), d_model, d_model)
        x = b.op1("Add", [x, attn])
        if not pre_ln:
            x = ln(x)
        h = ln(x) if pre_ln else x
        f = dense(_gelu_pattern(b, dense(h, d_model, 4 * d_model), gelu), 4 * d_model, d_model)
        x = b.op1("Add", [x, f])
        if not pre_ln:
            x = ln(x)
    if pre_ln:
        x = ln(x)
    if lm_head:
        logits = b.op1("MatMul", [x, b.op1("Transpose", [wte], perm=[1, 0])])
        return b.finish([("logits", logits)])
    return b.finish([("hidden", x)])


def tiny_gpt() -> Graph:
    return transformer(gelu="tanh", causal=True)


def tiny_bert() -> Graph:
    return transformer(gelu="erf", causal=False)


SAMPLES: dict[str, Callable[[], Graph]] = {
    "mlp": mlp,
    "tiny-cnn": tiny_cnn,
    "tiny-gpt": tiny_gpt,
    "tiny-bert": tiny_bert,
}


# ---------------------------------------------------------------------------------------------
# benchmark configurations
# ---------------------------------------------------------------------------------------------
def _he(b: GraphBuilder, shape: tuple[int, ...]) -> Value:
    """He-normal convolution / linear weight: std sqrt(2 / fan_in)."""
    fan_in = int(np.prod(shape[1:]))
    return b.const((b.rng.standard_normal(shape) * math.sqrt(2.0 / fan_in)).astype(np.float32), "w")


def _bn(b: GraphBuilder, x: Value, c: int) -> Value:
    """BatchNormalization with gamma ~ U(0.5, 1.5), beta and mean ~ N(0, 0.1), var ~ U(0.5, 1.5)."""
    gamma = b.const(b.rng.uniform(0.5, 1.5, c).astype(np.float32), "bn_s")
    beta = b.const((0.1 * b.rng.standard_normal(c)).astype(np.float32), "bn_b")
    mean = b.const((0.1 * b.rng.standard_normal(c)).astype(np.float32), "bn_m")
    var = b.const(b.rng.uniform(0.5, 1.5, c).astype(np.float32), "bn_v")
    return b.op1("BatchNormalization", [x, gamma, beta, mean, var], epsilon=1e-5)


def _conv_bn(b: GraphBuilder, x: Value, cin: int, cout: int, k: int, stride: int = 1, group: int = 1, pad: int | None = None) -> Value:
    p = k // 2 if pad is None else pad
    y = b.op1(
        "Conv",
        [x, _he(b, (cout, cin // group, k, k))],
        kernel_shape=[k, k],
        strides=[stride, stride],
        pads=[p] * 4,
        dilations=[1, 1],
        group=group,
    )
    return _bn(b, y, cout)


def single_gemm(m: int = 128, k: int = 768, n: int = 3072, seed: int = 0) -> Graph:
    """Config 1: MatMul -> Add(bias) -> Relu; W, bias ~ N(0, 0.02)."""
    b = GraphBuilder("single_gemm", seed)
    a = b.input("a", "float32", (m, k))
    w = b.const((b.rng.standard_normal((k, n)) * 0.02).astype(np.float32), "w")
    bias = b.const((b.rng.standard_normal(n) * 0.02).astype(np.float32), "b")
    y = b.op1("Relu", [b.op1("Add", [b.op1("MatMul", [a, w]), bias])])
    return b.finish([("y", y)])


def _bottleneck(b: GraphBuilder, x: Value, cin: int, width: int, stride: int, downsample: bool) -> Value:
    y = b.op1("Relu", [_conv_bn(b, x, cin, width, 1)])
    y = b.op1("Relu", [_conv_bn(b, y, width, width, 3, stride=stride)])
    y = _conv_bn(b, y, width, width * 4, 1)
    shortcut = _conv_bn(b, x, cin, width * 4, 1, stride=stride) if downsample else x
    return b.op1("Relu", [b.op1("Add", [y, shortcut])])


def bottleneck(batch: int = 1, seed: int = 0) -> Graph:
    """Config 2: ResNet-50 stage-1 identity bottleneck (256 -> 64 -> 64 -> 256 at 56x56)."""
    b = GraphBuilder("bottleneck", seed)
    x = b.input("x", "float32", (batch, 256, 56, 56))
    return b.finish([("y", _bottleneck(b, x, 256, 64, 1, False))])


def resnet50(batch: int = 1, classes: int = 1000, seed: int = 0) -> Graph:
    """Config 3: torchvision ResNet-50 (v1.5: stride on the 3x3 conv), He-normal init."""
    b = GraphBuilder("resnet50", seed)
    image = b.input("image", "float32", (batch, 3, 224, 224))
    x = b.op1("Relu", [_conv_bn(b, image, 3, 64, 7, stride=2, pad=3)])
    x = b.op1("MaxPool", [x], kernel_shape=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1])
    cin = 64
    for width, blocks, stride in ((64, 3, 1), (128, 4, 2), (256, 6, 2), (512, 3, 2)):
        for i in range(blocks):
            s = stride if i == 0 else 1
            x = _bottleneck(b, x, cin, width, s, downsample=(i == 0))
            cin = width * 4
    x = b.op1("GlobalAveragePool", [x])
    x = b.op1("Flatten", [x], axis=1)
    fc_w = _he(b, (classes, cin))
    fc_b = b.const((0.01 * b.rng.standard_normal(classes)).astype(np.float32), "fc_b")
    logits = b.op1("Gemm", [x, fc_w, fc_b], alpha=1.0, beta=1.0, transB=1)
    return b.finish([("logits", logits)])


def mobilenet_v2(batch: int = 1, classes: int = 1000, seed: int = 0) -> Graph:
    """Config 4: torchvision MobileNetV2 width 1.0 (ReLU6 exported as Clip(0, 6))."""
    b = GraphBuilder("mobilenet_v2", seed)
    image = b.input("image", "float32", (batch, 3, 224, 224))
    lo, hi = b.scalar(0.0), b.scalar(6.0)

    def relu6(v: Value) -> Value:
        return b.op1("Clip", [v, lo, hi])

    x = relu6(_conv_bn(b, image, 3, 32, 3, stride=2))
    cin = 32
    for t, c, n, s in ((1, 16, 1, 1), (6, 24, 2, 2), (6, 32, 3, 2), (6, 64, 4, 2), (6, 96, 3, 1), (6, 160, 3, 2), (6, 320, 1, 1)):
        for i in range(n):
            stride = s if i == 0 else 1
            hidden = cin * t
            y = x
            if t != 1:
                y = relu6(_conv_bn(b, y, cin, hidden, 1))
            y = relu6(_conv_bn(b, y, hidden, hidden, 3, stride=stride, group=hidden))
            y = _conv_bn(b, y, hidden, c, 1)
            x = b.op1("Add", [x, y]) if stride == 1 and cin == c else y
            cin = c
    x = relu6(_conv_bn(b, x, cin, 1280, 1))
    x = b.op1("GlobalAveragePool", [x])
    x = b.op1("Flatten", [x], axis=1)
    fc_w = b.const((b.rng.standard_normal((classes, 1280)) * 0.01).astype(np.float32), "fc_w")
    fc_b = b.const(np.zeros(classes, np.float32), "fc_b")
    logits = b.op1("Gemm", [x, fc_w, fc_b], alpha=1.0, beta=1.0, transB=1)
    return b.finish([("logits", logits)])


def bert_base(batch: int = 1, seq: int = 128, layers: int = 12, seed: int = 0, separate_qkv: bool = False) -> Graph:
    """Config 5: BERT-base encoder, post-LN, erf GELU, weights ~ N(0, 0.02), LN gamma 1 beta 0.

    The embeddings (word + position, then LayerNorm) feed 12 encoder layers; the output is the
    last hidden state [batch, seq, 768] (no pooler, no vocabulary head). ``separate_qkv`` gives
    the Hugging Face export's three Q/K/V projections instead of the sample's fused one.
    """
    return transformer(
        batch=batch,
        seq=seq,
        d_model=768,
        heads=12,
        layers=layers,
        vocab=30522,
        gelu="erf",
        causal=False,
        seed=seed,
        weight_scale=0.02,
        unit_layer_norm=True,
        embedding_norm=True,
        lm_head=False,
        ln_eps=1e-12,
        name="bert_base",
        separate_qkv=separate_qkv,
    )


def gpt2(batch: int = 1, seq: int = 128, layers: int = 12, seed: int = 0) -> Graph:
    """GPT-2 small (124M parameters): pre-LN decoder stack with the causal Where mask, tanh
    GELU, weights ~ N(0, 0.02), and the tied vocabulary head x @ wte^T ([.., 768] x [768, 50257],
    a FusedGemm with trans_b after O3), the pattern of the reference's causal sample
    (samples.py:178-245) at GPT-2 size."""
    return transformer(
        batch=batch,
        seq=seq,
        d_model=768,
        heads=12,
        layers=layers,
        vocab=50257,
        gelu="tanh",
        causal=True,
        seed=seed,
        weight_scale=0.02,
        lm_head=True,
        name="gpt2",
    )


CONFIGS: dict[str, Callable[..., Graph]] = {
    "single_gemm": single_gemm,
    "bottleneck": bottleneck,
    "resnet50": resnet50,
    "mobilenet_v2": mobilenet_v2,
    "bert_base": bert_base,
    "gpt2": gpt2,
}


def random_feeds(graph: Graph, seed: int = 0, int_high: int = 100) -> dict[str, np.ndarray]:
    """Seeded inputs like the reference's interpreter.random_feeds (interpreter.py:128-141):
    standard normal floats, booleans in {0, 1}, integers in [0, int_high)."""
    rng = np.random.default_rng(seed)
    feeds: dict[str, np.ndarray] = {}
    for v in graph.inputs:
        t = v.tensor_type
        dt = np.dtype({"float32": np.float32, "float64": np.float64, "int64": np.int64, "int32": np.int32,
                       "int8": np.int8, "uint8": np.uint8, "bool": np.bool_, "float16": np.float16}[t.dtype])
        if np.issubdtype(dt, np.floating):
            feeds[v.name] = rng.standard_normal(t.shape).astype(dt)
        elif dt == np.bool_:
            feeds[v.name] = rng.integers(0, 2, t.shape).astype(np.bool_)
        else:
            feeds[v.name] = rng.integers(0, int_high, t.shape).astype(dt)
    return feeds
