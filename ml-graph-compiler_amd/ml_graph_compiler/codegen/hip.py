"""hip code generation: the counterpart of the reference's C emitter (codegen/c.py:1-1340).

The emitter walks the scheduled graph once and writes one C++ translation unit of host code:
a forward function with one libmgc_hip.so launcher call per node, every arena, weights, input
and output pointer a constant offset, plus the exports of include/mgc_model.h. Device work is
all in the prebuilt kernel library (hand-written gfx950 kernels), so a model builds with g++ in
about a second and the runtime captures the forward into a hipGraph on first use.

Lowering per operator family:

* MatMul, Gemm, FusedGemm, Conv, FusedConv -> mgc_hip_gemm (fp32 MFMA). Constant right-hand
  sides are stored transposed ([N][K], k contiguous) in the weights blob so the kernel reads
  them in 16-byte k quads; NHWC convolutions are implicit GEMMs over M = N * OH * OW (batch
  folded into M), pointwise ones plain strided GEMMs; NCHW convolutions (below O3) read the image
  through im2col on the B side with a per-row bias. A small GEMM that cannot fill the chip splits
  K into a workspace that the memory planner places (its workspace hook).
* Depthwise convolution -> mgc_hip_depthwise (NHWC float4 over channels).
* Elementwise nodes and FusedElementwise programs -> mgc_hip_elementwise: leaves with element
  strides over the collapsed output dims plus a typed instruction list.
* Transpose/Expand/Slice/Concat/Split/Pad/Tile and output copies -> mgc_hip_copy / mgc_hip_fill.
* Gather -> mgc_hip_gather (device flag on a bad index -> mgc_run returns 1).
* Scaled dot-product attention chains (head-split Reshape/Transpose, MatMul, scale, Softmax,
  MatMul, head-merge Transpose; see codegen/attention.py) -> one mgc_hip_attention call that
  reads Q, K and V as strided views of the QKV projection; the chain's other nodes emit nothing.
* Softmax, LayerNorm, pooling, reductions, ArgMax -> their kernels.
* Views (Reshape, Flatten, Squeeze, Unsqueeze, Identity, Dropout) emit nothing.
"""

from __future__ import annotations

import hashlib
import math
import os
from collections.abc import Sequence
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Callable

import numpy as np

from .. import ops
from ..errors import CodegenError
from ..ir import Graph, Node, TensorType, Value, comment_text, numpy_dtype
from ..memory import ALIAS_OPS, MemoryPlan, Strategy, plan_memory
from .attention import AttentionMatch, find_attention
from .folding import FoldPlan, plan_folds
from .folding import _overlap as fold_overlap

ALIGN = 256  # arena offsets, weights chunks and the HBM block are 256-byte aligned

DTYPE_CODES = {
    "float32": 0,
    "float64": 1,
    "int64": 2,
    "int32": 3,
    "int8": 4,
    "uint8": 5,
    "bool": 6,
}
INT_DTYPES = ("int64", "int32", "int8", "uint8", "bool")

ACT_CODES = {
    "none": "MGC_ACT_NONE",
    "relu": "MGC_ACT_RELU",
    "clip": "MGC_ACT_CLIP",
    "gelu": "MGC_ACT_GELU",
    "gelu_tanh": "MGC_ACT_GELU_TANH",
    "tanh": "MGC_ACT_TANH",
    "sigmoid": "MGC_ACT_SIGMOID",
}

EW_OPCODES = {
    "Add": "MGC_EW_ADD", "Sub": "MGC_EW_SUB", "Mul": "MGC_EW_MUL", "Div": "MGC_EW_DIV",
    "Pow": "MGC_EW_POW", "Max": "MGC_EW_MAX", "Min": "MGC_EW_MIN", "Equal": "MGC_EW_EQUAL",
    "Less": "MGC_EW_LESS", "Greater": "MGC_EW_GREATER", "LessOrEqual": "MGC_EW_LESS_EQUAL",
    "GreaterOrEqual": "MGC_EW_GREATER_EQUAL", "And": "MGC_EW_AND", "Or": "MGC_EW_OR",
    "Xor": "MGC_EW_XOR", "Where": "MGC_EW_WHERE", "Relu": "MGC_EW_RELU",
    "Sigmoid": "MGC_EW_SIGMOID", "Tanh": "MGC_EW_TANH", "Erf": "MGC_EW_ERF",
    "Sqrt": "MGC_EW_SQRT", "Exp": "MGC_EW_EXP", "Log": "MGC_EW_LOG", "Neg": "MGC_EW_NEG",
    "Abs": "MGC_EW_ABS", "Reciprocal": "MGC_EW_RECIPROCAL", "Floor": "MGC_EW_FLOOR",
    "Ceil": "MGC_EW_CEIL", "Sin": "MGC_EW_SIN", "Cos": "MGC_EW_COS",
    "Softplus": "MGC_EW_SOFTPLUS", "Identity": "MGC_EW_IDENTITY", "Not": "MGC_EW_NOT",
    "LeakyRelu": "MGC_EW_LEAKY_RELU", "HardSigmoid": "MGC_EW_HARD_SIGMOID",
    "Clip": "MGC_EW_CLIP", "Cast": "MGC_EW_CAST",
}
_ANY_DTYPE = frozenset({"Equal", "Less", "Greater", "LessOrEqual", "GreaterOrEqual", "And", "Or",
                        "Xor", "Not", "Where", "Cast"})
_FLOAT32_OPS = frozenset(EW_OPCODES) | {"Gelu"}
_FLOAT64_OPS = frozenset({"Add", "Sub", "Mul", "Div", "Neg", "Identity"})
_INT_OPS = frozenset({"Add", "Sub", "Mul", "Div", "Max", "Min", "Neg", "Abs", "Relu", "Identity", "Clip"})

# Read Transposes through GEMM operand strides (codegen/folding.py); tests turn it off to compare.
FOLD_TRANSPOSES = True
# Run stride-2 convolutions over few channels on a space-to-depth copy of the input.
SPACE_TO_DEPTH = True
# Run the ResNet stem (7 x 7, stride 2, 3 -> 64 channels) as one mgc_hip_conv_stem launch that
# reads the image in place (NCHW through its strides when it reaches the stem through a
# Transpose) instead of the space-to-depth copy and a GEMM; tests turn it off to compare.
# Measured on MI355X in the ResNet-50 forward (graph replays, alternating on one box): batch 1
# 0.3873 -> 0.3855 ms, batch 32 2.7678 -> 2.7654 ms.
CONV_STEM = True
# Run a GlobalAveragePool over an NHWC activation and the FusedGemm that alone reads it (through
# a Reshape / Flatten view) as one mgc_hip_pool_fc launch when the batch is at most
# POOL_FC_MAX_BATCH (every workgroup pools its whole image, so larger batches keep the pooling
# launch and the GEMM); tests turn it off to compare. Measured on MI355X (graph replays,
# alternating on one box): MobileNetV2 b1 0.2560 -> 0.2529 ms, ResNet-50 b1 0.3839 -> 0.3825 ms.
FUSE_POOL_FC = True
POOL_FC_MAX_BATCH = 4
# Run an embedding lookup (Gather of a constant table), the Add of a same-shape or leading-
# broadcast addend that alone reads it and the LayerNormalization over the sum's rows as one
# mgc_hip_gather_layer_norm launch (which also stores the sum when later nodes read it); tests
# turn it off to compare. Measured on MI355X (graph replays, alternating on one box): BERT-base
# b1 0.7702 -> 0.7626 ms, b16 3.440 -> 3.426 ms; GPT-2 b1 0.8800 -> 0.8721 ms, b8 2.7305 ->
# 2.7212 ms.
FUSE_GATHER_LAYER_NORM = True
# Fuse recognized attention chains into mgc_hip_attention (tests turn it off to compare).
FUSE_ATTENTION = True
# Run a LayerNormalization that directly follows the FusedGemm producing its input inside that
# GEMM's split-K reduction (mgc_hip_gemm_layer_norm); tests turn it off to compare.
FUSE_GEMM_LAYER_NORM = True
# Compute a residual block's projection shortcut (a 1 x 1 convolution with no activation that
# only the block's last 1 x 1 convolution reads, as its residual) inside that convolution's GEMM
# by concatenating the two reductions along K; tests turn it off to compare.
FUSE_PROJECTION_SHORTCUT = True
# Compute a 3 x 3 depthwise convolution inside the GEMM of the 1 x 1 convolution that alone reads
# its output (mgc_hip_gemm_dw: the A tiles are the depthwise output, which is never stored), for
# GEMMs of at least DEPTHWISE_FUSE_MIN_ROWS output pixels (enough 8 x 8 pixel tiles to occupy
# every CU) or over at most DEPTHWISE_FUSE_SHALLOW_K channels (three K stages or fewer, where
# the saved launch outweighs the few tiles); tests turn it off to compare.
FUSE_DEPTHWISE_POINTWISE = True
DEPTHWISE_FUSE_MIN_ROWS = 16384
DEPTHWISE_FUSE_SHALLOW_K = 96
# Run a whole inverted-residual block (1 x 1 expansion with relu / clip -> 3 x 3 depthwise with
# relu / clip -> 1 x 1 projection, MobileNetV2's t > 1 blocks) as one mgc_hip_mbconv launch,
# for blocks of at least MBCONV_MIN_ROWS output pixels (the kernel's 8 x 8-pixel tiles then
# number at least 256, one per CU); tests turn it off to compare.
FUSE_INVERTED_RESIDUAL = True
MBCONV_MIN_ROWS = 16384
# mgc_hip_mbconv_supported: input channels, expanded channels, output channels
MBCONV_CIN = (16, 24, 32)
MBCONV_MAX_CEXP = 256
MBCONV_MAX_COUT = 32
# The same launch with a 3 x 3 convolution of a 3-channel image (with relu / clip) in place of
# the expansion (mgc_hip_mbconv_stem: MobileNetV2's stem and first block), at any size: the
# stem's output, the depthwise output and the stem's NHWC input copy are never written.
FUSE_STEM_BLOCK = True
MBCONV_STEM_MIN_ROWS = 0
# Run an inverted-residual block's 1 x 1 expansion (relu / clip) and the 3 x 3 depthwise
# convolution (relu / clip) that alone reads it as one mgc_hip_expand_dw launch (a workgroup per
# image and 32 expanded channels; the expanded tensor never goes to memory) when
# mgc_hip_expand_dw_supported accepts the shape and the images times 32-channel slices number
# at least EXPAND_DW_MIN_WORKGROUPS; tests turn it off to compare. Measured on MI355X with no
# lower bound: MobileNetV2 batch 1 0.266 -> 0.256 ms (its 14 x 14 and 7 x 7 blocks then run as
# 6 to 30 workgroups each, still ahead of two launches), batch 32 unchanged (0.5455 ms with a
# bound of 0, 32, 96 or 256).
FUSE_EXPAND_DEPTHWISE = True
EXPAND_DW_MIN_WORKGROUPS = 0
# The fused GEMMs address their image and weight operands through buffer resources with 32-bit
# byte offsets, and their launchers refuse operands of this many bytes or more (the unfused
# kernels have a generic path for them): both fusions are only taken below it.
FUSED_OPERAND_LIMIT = 0x7FFFFFFF

MAX_RANK = 6
MAX_LEAVES = 16
MAX_INSTR = 32
MAX_BATCH_RANK = 4


def _f(v: float) -> str:
    """A C float literal."""
    v = float(v)
    if math.isnan(v):
        return "NAN"
    if math.isinf(v):
        return "INFINITY" if v > 0 else "(-INFINITY)"
    return f"{float(np.float32(v))!r}f"


def _strides(shape: Sequence[int]) -> list[int]:
    out = [1] * len(shape)
    for i in range(len(shape) - 2, -1, -1):
        out[i] = out[i + 1] * int(shape[i + 1])
    return out


def _broadcast_strides(shape: Sequence[int], out_shape: Sequence[int]) -> list[int]:
    """Element strides of ``shape`` broadcast (right-aligned) to ``out_shape``."""
    src = _strides(shape)
    pad = len(out_shape) - len(shape)
    return [0 if d < pad or shape[d - pad] == 1 else src[d - pad] for d in range(len(out_shape))]


def collapse(shape: Sequence[int], stride_sets: list[list[int]]) -> tuple[list[int], list[list[int]]]:
    """Drop unit dims and merge neighbours that are contiguous for every operand
    (the dimension collapsing of the reference's loop nests, codegen/c.py:370-378)."""
    keep = [i for i, d in enumerate(shape) if d != 1]
    dims = [int(shape[i]) for i in keep]
    strides = [[s[i] for i in keep] for s in stride_sets]
    d = len(dims) - 1
    while d > 0:
        if all(s[d - 1] == s[d] * dims[d] for s in strides):
            dims[d - 1] *= dims[d]
            del dims[d]
            for s in strides:
                s[d - 1] = s[d]
                del s[d]
        d -= 1
    return dims, strides


@dataclass
class WeightsBuilder:
    """The weights blob the model uploads once: every constant the kernels read, each starting
    at a 256-byte aligned offset (the alignment of the DMA loads), and a constant added twice
    under the same key stored once. Arrays are referenced, not copied, until the blob is
    materialized."""

    pieces: list[tuple[int, np.ndarray]] = field(default_factory=list)
    end: int = 0
    offsets: dict[Any, int] = field(default_factory=dict)

    def add(self, array: np.ndarray, key: Any = None) -> int:
        """Byte offset of ``array`` in the blob."""
        if key is not None and key in self.offsets:
            return self.offsets[key]
        data = np.ascontiguousarray(array)
        at = (self.end + ALIGN - 1) // ALIGN * ALIGN
        self.pieces.append((at, data))
        self.end = at + data.nbytes
        if key is not None:
            self.offsets[key] = at
        return at

    @property
    def nbytes(self) -> int:
        return max((self.end + ALIGN - 1) // ALIGN * ALIGN, ALIGN)

    def digest(self) -> str:
        """Content hash of the blob (names the weights file in the build cache)."""
        h = hashlib.sha256(str(self.nbytes).encode())
        for at, data in self.pieces:
            h.update(np.int64(at).tobytes())
            h.update(data.reshape(-1).view(np.uint8).data)
        return h.hexdigest()[:24]

    def blob(self) -> np.ndarray:
        image = np.zeros(self.nbytes, np.uint8)
        for at, data in self.pieces:
            image[at : at + data.nbytes] = data.reshape(-1).view(np.uint8)
        return image

    def write(self, path: Path) -> None:
        """Write the blob to ``path`` atomically (a temporary file renamed into place)."""
        staging = path.with_suffix(path.suffix + f".tmp{os.getpid()}")
        self.blob().tofile(staging)
        staging.replace(path)


def _pointwise_nhwc(node: Node) -> bool:
    """A float32 NHWC convolution with a constant 1 x 1 kernel, no padding and one group."""
    if node.op not in ("Conv", "FusedConv") or ops.conv_layout(node) != "NHWC":
        return False
    w, xt = node.input(1), node.input(0).tensor_type
    if w.data is None or xt.dtype != "float32" or w.tensor_type.shape[:2] != (1, 1):
        return False
    if int(node.attrs.get("group", 1)) != 1:
        return False
    g = ops.window_geometry(node, xt.shape[1:3], (1, 1))
    return all(p == 0 for p in g.pads) and all(v is None or v.data is not None for v in node.inputs[2:3])


def _stem_conv_nhwc(node: Node) -> bool:
    """A float32 NHWC convolution mgc_hip_mbconv_stem evaluates in place of an expansion: a
    constant 3 x 3 kernel over 3 input channels, one group, strides 1 or 2, no dilation,
    constant bias (or none), no residual, relu or clip."""
    if node.op != "FusedConv" or ops.conv_layout(node) != "NHWC":
        return False
    if node.attrs.get("activation", "none") not in ("relu", "clip"):
        return False
    w, xt = node.input(1), node.input(0).tensor_type
    if w.data is None or xt.dtype != "float32" or xt.rank != 4 or w.tensor_type.shape[:3] != (3, 3, 3):
        return False
    if int(node.attrs.get("group", 1)) != 1 or node.input(0).data is not None:
        return False
    g = ops.window_geometry(node, xt.shape[1:3], (3, 3))
    if tuple(g.dilations) != (1, 1) or max(g.strides) > 2:
        return False
    b = node.optional_input(2)
    return (b is None or b.data is not None) and node.optional_input(3) is None


def _tensor_bytes(v: Value) -> int:
    t = v.tensor_type
    return int(np.prod(t.shape, dtype=np.int64)) * np.dtype(numpy_dtype(t.dtype)).itemsize


def find_projection_shortcuts(graph: Graph) -> dict[int, Node]:
    """id(c3) -> ds for every residual block whose projection shortcut ds can run inside the
    GEMM of the block's last convolution c3 (a ResNet downsample block).

    c3: pointwise NHWC FusedConv, stride 1, whose residual input is ds's output and whose
    input channels K1 are a multiple of 32 (a whole number of 32-wide K stages before the
    second source starts). ds: pointwise NHWC convolution with no activation and no residual,
    any stride, input channels a multiple of 4, whose output only c3 reads (as its residual) and
    which the schedule puts before c3; its input must be a tensor (not a constant). The fused
    launch reads c3's input, ds's input and the stacked [N][K1 + K2] weights each below
    FUSED_OPERAND_LIMIT bytes."""
    order = {id(n): i for i, n in enumerate(graph.nodes)}
    outputs = {id(v) for v in graph.outputs}
    found: dict[int, Node] = {}
    for c3 in graph.nodes:
        if c3.op != "FusedConv" or not _pointwise_nhwc(c3):
            continue
        r = c3.optional_input(3)
        ds = r.producer if r is not None else None
        if ds is None or not _pointwise_nhwc(ds) or id(r) in outputs or r.users != [c3]:
            continue
        if sum(v is r for v in c3.inputs) != 1 or order[id(ds)] > order[id(c3)]:
            continue
        if ds.op == "FusedConv" and (ds.attrs.get("activation", "none") != "none" or ds.optional_input(3) is not None):
            continue
        xt, at = ds.input(0).tensor_type, c3.input(0).tensor_type
        g3 = ops.window_geometry(c3, at.shape[1:3], (1, 1))
        gd = ops.window_geometry(ds, xt.shape[1:3], (1, 1))
        if g3.strides != (1, 1) or tuple(gd.out_hw) != tuple(at.shape[1:3]) or xt.shape[0] != at.shape[0]:
            continue
        if ds.input(0).data is not None or at.shape[3] % 32 or xt.shape[3] % 4:
            continue
        if ds.input(1).tensor_type.shape[3] != c3.input(1).tensor_type.shape[3]:
            continue
        stacked = 4 * (at.shape[3] + xt.shape[3]) * c3.input(1).tensor_type.shape[3]
        if max(_tensor_bytes(c3.input(0)), _tensor_bytes(ds.input(0)), stacked) >= FUSED_OPERAND_LIMIT:
            continue
        found[id(c3)] = ds
    return found


def _depthwise3x3_nhwc(node: Node) -> bool:
    """A float32 NHWC depthwise convolution (one channel per group) with a constant 3 x 3
    kernel, strides (1, 1) or (2, 2), no dilation, constant bias (or none), no residual and
    C % 4 == 0."""
    if node.op not in ("Conv", "FusedConv") or ops.conv_layout(node) != "NHWC":
        return False
    w, xt = node.input(1), node.input(0).tensor_type
    if w.data is None or xt.dtype != "float32" or xt.rank != 4 or not HipEmitter.depthwise(node):
        return False
    if w.tensor_type.shape[:2] != (3, 3) or xt.shape[3] % 4 or node.input(0).data is not None:
        return False
    g = ops.window_geometry(node, xt.shape[1:3], (3, 3))
    if tuple(g.dilations) != (1, 1) or tuple(g.strides) not in ((1, 1), (2, 2)):
        return False
    b = node.optional_input(2)
    return (b is None or b.data is not None) and node.optional_input(3) is None


def find_depthwise_pointwise(graph: Graph, min_rows: int | None = None) -> dict[int, Node]:
    """id(pw) -> dw for every 3 x 3 depthwise convolution dw whose output only the pointwise
    convolution pw reads (MobileNet's depthwise -> projection pair), when pw's GEMM has at least
    ``min_rows`` rows (default DEPTHWISE_FUSE_MIN_ROWS) or at most DEPTHWISE_FUSE_SHALLOW_K
    input channels: pw is a stride-1 pointwise NHWC convolution, dw a depthwise 3 x 3
    convolution (stride 1 or 2, any padding) over a tensor whose channels are a multiple of 4,
    with the depthwise input and pw's weights each below FUSED_OPERAND_LIMIT bytes."""
    if min_rows is None:
        min_rows = DEPTHWISE_FUSE_MIN_ROWS
    outputs = {id(v) for v in graph.outputs}
    found: dict[int, Node] = {}
    for pw in graph.nodes:
        if not _pointwise_nhwc(pw):
            continue
        d = pw.input(0)
        dw = d.producer
        if dw is None or not _depthwise3x3_nhwc(dw) or id(d) in outputs or d.users != [pw]:
            continue
        if sum(v is d for v in pw.inputs) != 1:
            continue
        at = d.tensor_type
        if ops.window_geometry(pw, at.shape[1:3], (1, 1)).strides != (1, 1):
            continue
        if at.shape[0] * at.shape[1] * at.shape[2] < min_rows and at.shape[3] > DEPTHWISE_FUSE_SHALLOW_K:
            continue
        if max(_tensor_bytes(dw.input(0)), _tensor_bytes(pw.input(1))) >= FUSED_OPERAND_LIMIT:
            continue
        found[id(pw)] = dw
    return found


def find_inverted_residuals(graph: Graph, min_rows: int | None = None) -> dict[int, tuple[Node, Node]]:
    """id(pw) -> (ex, dw) for every inverted-residual block that mgc_hip_mbconv can run as one
    launch: ex a pointwise NHWC FusedConv (stride 1, relu or clip, no residual) whose output only
    dw reads, dw a 3 x 3 depthwise FusedConv (stride 1 or 2, relu or clip) whose output only pw
    reads, pw a stride-1 pointwise NHWC convolution (any bias, residual and activation), with
    the kernel's channel limits (input 16, 24 or 32 channels, at most MBCONV_MAX_CEXP expanded
    and MBCONV_MAX_COUT output channels), at least ``min_rows`` output pixels (default
    MBCONV_MIN_ROWS) and the block input below FUSED_OPERAND_LIMIT bytes. With FUSE_STEM_BLOCK,
    ex may instead be a stem convolution (``_stem_conv_nhwc``: 3 x 3 over a 3-channel image,
    stride 1 or 2, any padding) ahead of a block without expansion, which mgc_hip_mbconv_stem runs as
    one launch at MBCONV_STEM_MIN_ROWS output pixels or more."""
    if min_rows is None:
        min_rows = MBCONV_MIN_ROWS
    outputs = {id(v) for v in graph.outputs}

    def clamp_act(node: Node) -> bool:
        return node.op == "FusedConv" and node.attrs.get("activation", "none") in ("relu", "clip")

    found: dict[int, tuple[Node, Node]] = {}
    for pw in graph.nodes:
        if not _pointwise_nhwc(pw):
            continue
        d = pw.input(0)
        dw = d.producer
        if dw is None or not _depthwise3x3_nhwc(dw) or not clamp_act(dw) or id(d) in outputs or d.users != [pw]:
            continue
        if sum(v is d for v in pw.inputs) != 1:
            continue
        e = dw.input(0)
        ex = e.producer
        if ex is None or id(e) in outputs or e.users != [dw] or ex.input(0).data is not None:
            continue
        stem = FUSE_STEM_BLOCK and _stem_conv_nhwc(ex)
        if not stem and (not _pointwise_nhwc(ex) or not clamp_act(ex) or ex.optional_input(3) is not None):
            continue
        xt, et, dt = ex.input(0).tensor_type, e.tensor_type, d.tensor_type
        if not stem and ops.window_geometry(ex, xt.shape[1:3], (1, 1)).strides != (1, 1):
            continue
        if ops.window_geometry(pw, dt.shape[1:3], (1, 1)).strides != (1, 1):
            continue
        cin, cexp, cout = 32 if stem else xt.shape[3], et.shape[3], pw.input(1).tensor_type.shape[3]
        if cin not in MBCONV_CIN or cexp % 4 or cexp > MBCONV_MAX_CEXP or cout > MBCONV_MAX_COUT:
            continue
        rows = min(min_rows, MBCONV_STEM_MIN_ROWS) if stem else min_rows
        if dt.shape[0] * dt.shape[1] * dt.shape[2] < rows or _tensor_bytes(ex.input(0)) >= FUSED_OPERAND_LIMIT:
            continue
        found[id(pw)] = (ex, dw)
    return found


def expand_dw_supported(h: int, w: int, cin: int, cexp: int, stride: int, oh: int, ow: int) -> bool:
    """The shapes mgc_hip_expand_dw_supported accepts: 64 or 96 input channels over at most 256
    image pixels, or 160 over at most 64; expanded channels a multiple of 32; stride 1 or 2; a
    depthwise window ((oh - 1) stride + 3) x ((ow - 1) stride + 3) of at most 256 pixels (128
    for 160 input channels)."""
    if min(h, w, oh, ow, cexp) <= 0 or cexp % 32 or stride not in (1, 2):
        return False
    window = ((oh - 1) * stride + 3) * ((ow - 1) * stride + 3)
    row_blocks_per_wave = ((h * w + 15) // 16 + 3) // 4
    if cin in (64, 96):
        return h * w <= 256 and row_blocks_per_wave <= 4 and window <= 256
    return cin == 160 and h * w <= 64 and row_blocks_per_wave <= 1 and window <= 128


def find_expand_depthwise(graph: Graph, min_workgroups: int | None = None) -> dict[int, Node]:
    """id(dw) -> ex for every 1 x 1 expansion ex whose output only the 3 x 3 depthwise
    convolution dw reads, when mgc_hip_expand_dw can run the pair as one launch: ex a pointwise
    NHWC FusedConv (stride 1, relu or clip, no residual), dw a depthwise FusedConv (relu or
    clip, stride 1 or 2, padding at most 2), the shape expand_dw_supported accepts, at least
    ``min_workgroups`` (default EXPAND_DW_MIN_WORKGROUPS) images x 32-channel slices and the
    block input below FUSED_OPERAND_LIMIT bytes."""
    if min_workgroups is None:
        min_workgroups = EXPAND_DW_MIN_WORKGROUPS
    outputs = {id(v) for v in graph.outputs}

    def clamp_act(node: Node) -> bool:
        return node.op == "FusedConv" and node.attrs.get("activation", "none") in ("relu", "clip")

    found: dict[int, Node] = {}
    for dw in graph.nodes:
        if not _depthwise3x3_nhwc(dw) or not clamp_act(dw):
            continue
        e = dw.input(0)
        ex = e.producer
        if ex is None or not _pointwise_nhwc(ex) or not clamp_act(ex) or ex.optional_input(3) is not None:
            continue
        if id(e) in outputs or e.users != [dw] or ex.input(0).data is not None:
            continue
        xt, et = ex.input(0).tensor_type, e.tensor_type
        if ops.window_geometry(ex, xt.shape[1:3], (1, 1)).strides != (1, 1):
            continue
        nb, h, w, cin = xt.shape
        cexp = et.shape[3]
        g = ops.window_geometry(dw, (h, w), (3, 3))
        oh, ow = g.out_hw
        if g.strides[0] != g.strides[1] or max(g.pads[0], g.pads[1]) > 2:
            continue
        if not expand_dw_supported(h, w, cin, cexp, g.strides[0], oh, ow):
            continue
        if nb * (cexp // 32) < min_workgroups or _tensor_bytes(ex.input(0)) >= FUSED_OPERAND_LIMIT:
            continue
        found[id(dw)] = ex
    return found


def find_gather_layer_norm(graph: Graph) -> dict[int, tuple[Node, Node, Value, int, bool]]:
    """id(LayerNormalization) -> (Gather, Add, addend, addend rows, store the sum?) for every
    embedding lookup
    that runs as one mgc_hip_gather_layer_norm launch: a Gather along axis 0 of a constant float
    table (rows of cols floats, cols a multiple of 4 and at most 1024) with int64 / int32 indices,
    whose output only an Add reads; the Add's other operand a float tensor that is the output's
    shape or repeats over its leading dimensions; and a LayerNormalization over the last axis
    that reads the sum (no Mean / InvStdDev wanted). Other readers of the sum (GPT-2's first
    residual) must come after the LayerNorm in schedule order; the launch then also stores the
    sum. None of the three outputs but the LayerNorm's may be a graph output."""
    found: dict[int, tuple[Node, Node, Value, int, bool]] = {}
    outputs = set(map(id, graph.outputs))
    order = {id(n): i for i, n in enumerate(graph.nodes)}
    for gather in graph.nodes:
        if gather.op != "Gather" or len(gather.inputs) != 2:
            continue
        table, ids = gather.input(0), gather.input(1)
        tt = table.tensor_type
        if table.data is None or tt.dtype != "float32" or tt.rank != 2:
            continue
        axis = int(gather.attrs.get("axis", 0))
        if (axis + tt.rank if axis < 0 else axis) != 0 or ids.tensor_type.dtype not in ("int64", "int32"):
            continue
        cols = tt.shape[1]
        if cols % 4 or not 4 <= cols <= 1024:
            continue
        g_out = gather.output
        if id(g_out) in outputs or len(g_out.users) != 1 or g_out.users[0].op != "Add":
            continue
        add = g_out.users[0]
        if len(add.inputs) != 2 or add.input(0) is add.input(1):
            continue
        other = add.input(1) if add.input(0) is g_out else add.input(0)
        ot, yt = other.tensor_type, add.output.tensor_type
        if ot.dtype != "float32" or yt.shape != g_out.tensor_type.shape or ot.rank > yt.rank:
            continue
        dims = (1,) * (yt.rank - ot.rank) + tuple(ot.shape)
        if dims[-1] != cols:
            continue
        lead = 0
        while lead < yt.rank - 1 and dims[lead] == 1:
            lead += 1
        if tuple(dims[lead:-1]) != tuple(yt.shape[lead:-1]):
            continue
        add_rows = int(np.prod(dims[lead:-1])) if lead < yt.rank - 1 else 1
        if id(add.output) in outputs:
            continue
        lns = [u for u in add.output.users if u.op == "LayerNormalization" and u.input(0) is add.output]
        if not lns:
            continue
        ln = min(lns, key=lambda u: order[id(u)])
        others = [u for u in add.output.users if u is not ln]
        if any(order[id(u)] <= order[id(ln)] for u in others):
            continue
        ln_axis = int(ln.attrs.get("axis", -1))
        if (ln_axis + yt.rank if ln_axis < 0 else ln_axis) != yt.rank - 1:
            continue
        if any(o.users or id(o) in outputs for o in ln.outputs[1:]):
            continue
        if ln.output.tensor_type.dtype != "float32":
            continue
        found[id(ln)] = (gather, add, other, add_rows, bool(others))
    return found


def find_pool_fc(graph: Graph) -> dict[int, Node]:
    """id(FusedGemm) -> the GlobalAveragePool it reads through one view, for the pairs that run as
    one mgc_hip_pool_fc launch: an NHWC float pooling of at most POOL_FC_MAX_BATCH images whose
    output (and the view's) nothing else reads and no graph output is, and a FusedGemm over the
    pooled vectors (K = the channel count, at most 4096 and a multiple of 4) with a constant
    right-hand side and no residual."""
    found: dict[int, Node] = {}
    outputs = set(map(id, graph.outputs))
    for gap in graph.nodes:
        if gap.op != "GlobalAveragePool" or ops.conv_layout(gap) != "NHWC":
            continue
        xt = gap.input(0).tensor_type
        if xt.dtype != "float32" or xt.rank != 4 or not 1 <= xt.shape[0] <= POOL_FC_MAX_BATCH:
            continue
        n, c = xt.shape[0], xt.shape[3]
        if c % 4 or not 4 <= c <= 4096 or xt.shape[1] * xt.shape[2] < 1:
            continue
        pooled = gap.output
        if id(pooled) in outputs or len(pooled.users) != 1:
            continue
        view = pooled.users[0]
        if view.op not in ("Reshape", "Flatten", "Squeeze") or view.input(0) is not pooled:
            continue
        if id(view.output) in outputs or len(view.output.users) != 1:
            continue
        fc = view.output.users[0]
        if fc.op != "FusedGemm" or fc.input(0) is not view.output or fc.optional_input(3) is not None:
            continue
        b = fc.input(1)
        bt = b.tensor_type
        if b.data is None or bt.rank != 2 or fc.output.tensor_type.dtype != "float32":
            continue
        k = bt.shape[1] if int(fc.attrs.get("trans_b", 0)) else bt.shape[0]
        if k != c or view.output.tensor_type.size != n * c:
            continue
        found[id(fc)] = gap
    return found


def pack_b_nk(b: np.ndarray) -> np.ndarray:
    """A constant K x N right-hand side stored as its transpose [N][K] (k contiguous), the
    layout the MFMA GEMM reads with 16-byte k-quad loads."""
    return np.ascontiguousarray(np.asarray(b, np.float32).T)


@dataclass
class GeneratedModel:
    source: str
    weights: WeightsBuilder
    arena_bytes: int
    inputs: list[tuple[str, TensorType]]
    outputs: list[tuple[str, TensorType]]
    plan: MemoryPlan
    lines: int
    kernels: dict[str, int]
    node_flops: list[int]
    # algorithmic FLOPs of the GEMM-family launches (every mgc_hip_gemm / _gemm_dw / _mbconv /
    # _gemm_layer_norm call: 2 M N K per batch element, plus the depthwise and expansion work a
    # fused call computes); attention products run in the attention kernel and are not counted
    gemm_flops: int = 0


class HipEmitter:
    """Generates the host C++ source and weights blob of one scheduled graph."""

    SUPPORTED = frozenset(
        {
            *(op for op in ops.REGISTRY if ops.is_elementwise(op)),
            "FusedElementwise", "Transpose", "Expand", "Slice", "Concat", "Split", "Pad", "Tile",
            "Gather", "Shape", "Size", "ConstantOfShape", "Range", "ReduceMean", "ReduceSum",
            "ReduceMax", "ReduceMin", "ReduceProd", "ArgMax", "Softmax", "LogSoftmax",
            "LayerNormalization", "BatchNormalization", "MatMul", "Gemm", "FusedGemm", "Conv",
            "FusedConv", "MaxPool", "AveragePool", "GlobalAveragePool", "GlobalMaxPool",
            *ALIAS_OPS,
        }
    )

    def __init__(
        self,
        graph: Graph,
        strategy: Strategy = "greedy_by_size",
        inplace: bool = True,
        profile: bool = False,
        gemm_workspace: Callable[[int, int, int, int], int] | None = None,
        gemm_ln_workspace: Callable[[int, int, int], int] | None = None,
    ) -> None:
        unsupported = sorted({n.op for n in graph.nodes} - self.SUPPORTED)
        if unsupported:
            raise CodegenError(f"the hip backend does not support: {', '.join(unsupported)}")
        for v in graph.values():
            if v.type is not None and v.type.dtype == "float16":
                raise CodegenError(f"float16 tensors are not supported ({v.name})")
        self.graph = graph
        self.profile = profile
        self._gemm_ws = gemm_workspace
        # id(last 1 x 1 conv) -> its projection shortcut, and the shortcuts' ids. The shortcut's
        # input is then read at the last conv's step, which the plan must keep it alive for.
        self._shortcut: dict[int, Node] = find_projection_shortcuts(graph) if FUSE_PROJECTION_SHORTCUT else {}
        self._shortcut_skip = {id(ds) for ds in self._shortcut.values()}
        # id(pointwise conv) -> the depthwise convolution computed in its GEMM; the depthwise
        # input is then read at the pointwise step, which the plan must keep it alive for.
        # id(projection conv) -> (expansion, depthwise) of an inverted-residual block run as one
        # launch; the block input is then read at the projection's step.
        self._mb: dict[int, tuple[Node, Node]] = find_inverted_residuals(graph) if FUSE_INVERTED_RESIDUAL else {}
        taken = set(self._shortcut) | self._shortcut_skip
        for pw_id in [i for i, (ex, dw) in self._mb.items() if {i, id(ex), id(dw)} & taken]:
            del self._mb[pw_id]
        self._mb_skip = {id(n) for pair in self._mb.values() for n in pair}
        self._dwpw: dict[int, Node] = find_depthwise_pointwise(graph) if FUSE_DEPTHWISE_POINTWISE else {}
        taken |= set(self._mb) | self._mb_skip
        for pw_id in [i for i, dw in self._dwpw.items() if id(dw) in taken or i in taken]:
            del self._dwpw[pw_id]
        self._dwpw_skip = {id(dw) for dw in self._dwpw.values()}
        # id(depthwise conv) -> the expansion computed in its launch (mgc_hip_expand_dw); the
        # expansion's input is then read at the depthwise step.
        self._xd: dict[int, Node] = find_expand_depthwise(graph) if FUSE_EXPAND_DEPTHWISE else {}
        taken |= set(self._dwpw) | self._dwpw_skip
        for dw_id in [i for i, ex in self._xd.items() if i in taken or id(ex) in taken]:
            del self._xd[dw_id]
        self._xd_skip = {id(ex) for ex in self._xd.values()}
        # id(FusedGemm) -> the global average pooling computed in its launch (mgc_hip_pool_fc);
        # the pooling's input is then read at the GEMM's step.
        self._pool_fc: dict[int, Node] = find_pool_fc(graph) if FUSE_POOL_FC else {}
        self._pool_fc_skip = {id(gap) for gap in self._pool_fc.values()}
        # id(LayerNormalization) -> (Gather, Add, addend, addend rows, store the sum?) run as
        # one launch; the indices and the addend are then read at the LayerNorm's step.
        self._gln: dict[int, tuple[Node, Node, Value, int, bool]] = (
            find_gather_layer_norm(graph) if FUSE_GATHER_LAYER_NORM else {})
        self._gln_skip = {id(n) for g, a, *_ in self._gln.values() for n in (g, a)}
        order = {id(n): i for i, n in enumerate(graph.nodes)}
        keep = {id(ds.input(0)): order[id(c3)] for c3 in graph.nodes
                if (ds := self._shortcut.get(id(c3))) is not None}
        for fc_id, gap in self._pool_fc.items():
            keep[id(gap.input(0))] = max(keep.get(id(gap.input(0)), 0), order[fc_id])
        for ln_id, (gather, _, other, *_) in self._gln.items():
            for v in (gather.input(1), other):
                keep[id(v)] = max(keep.get(id(v), 0), order[ln_id])
        for pw in graph.nodes:
            if (dw := self._dwpw.get(id(pw))) is not None:
                keep[id(dw.input(0))] = max(keep.get(id(dw.input(0)), 0), order[id(pw)])
            if (pair := self._mb.get(id(pw))) is not None:
                xin = pair[0].input(0)
                keep[id(xin)] = max(keep.get(id(xin), 0), order[id(pw)])
            if (ex := self._xd.get(id(pw))) is not None:  # pw is the depthwise node here
                xin = ex.input(0)
                keep[id(xin)] = max(keep.get(id(xin), 0), order[id(pw)])
        self.plan = plan_memory(graph, strategy=strategy, alignment=ALIGN, inplace=inplace,
                                workspace=self._workspace_bytes, extra_reads=keep)
        self.weights = WeightsBuilder()
        self.body: list[str] = []
        self.kernels: dict[str, int] = {}
        self._gemm_flops = 0
        # Constants the emitter creates itself (unfused BatchNorm scale/shift). Weights chunks are
        # keyed by id(value), so these must outlive the emission or a later temporary could reuse
        # an id and alias an earlier chunk.
        self._owned_constants: list[Value] = []
        self._attn_emit: dict[int, AttentionMatch] = {}
        self._attn_skip: dict[int, AttentionMatch] = {}
        # Scratch past the planned arena (the plan's offsets stay as they are) for fused
        # attention outputs that must not be written over their operands.
        # Layout: [grouped Q/K/V projection output | staged attention output].
        self._scratch_off = (max(self.plan.arena_bytes, ALIGN) + ALIGN - 1) // ALIGN * ALIGN
        self._scratch_bytes = 0
        qkv_bytes = out_bytes = 0
        if FUSE_ATTENTION:
            for m in find_attention(graph, self.plan):
                self._attn_emit[id(m.emit_at)] = m
                for n in m.absorbed:
                    if n is not m.emit_at:
                        self._attn_skip[id(n)] = m
                if m.staged:
                    out_bytes = max(out_bytes, m.out.tensor_type.nbytes)
                if m.qkv_gemms:
                    qkv_bytes = max(qkv_bytes, 3 * m.out.tensor_type.nbytes)
        excluded = (set(self._attn_skip) | set(self._attn_emit) | set(self._shortcut) | self._shortcut_skip
                    | set(self._dwpw) | self._dwpw_skip | set(self._mb) | self._mb_skip | set(self._xd)
                    | self._xd_skip | set(self._pool_fc) | self._pool_fc_skip | set(self._gln) | self._gln_skip)
        self._folds = plan_folds(graph, self.plan, self._workspace_bytes, excluded) if FOLD_TRANSPOSES else FoldPlan()
        self._scratch_qkv_off = self._scratch_off
        self._scratch_out_off = self._scratch_off + (qkv_bytes + ALIGN - 1) // ALIGN * ALIGN
        self._scratch_bytes = self._scratch_out_off - self._scratch_off + out_bytes
        # Stride-2 convolutions over few channels (the ResNet stem) run as stride-1
        # convolutions over a space-to-depth copy of their input, written to the scratch area
        # (scratch contents live only within one node's launches, so every use shares it).
        self._s2d: dict[int, Value | None] = {}
        self._s2d_skip: set[int] = set()
        # ResNet stems: id(conv) -> the NCHW tensor read in place, or None for the NHWC input
        self._cstem: dict[int, Value | None] = {}
        if CONV_STEM:
            order = {id(n): i for i, n in enumerate(graph.nodes)}
            for n in graph.nodes:
                if id(n) in excluded or not self._conv_stem_ok(n):
                    continue
                self._cstem[id(n)] = self._s2d_source(n, order, excluded)
                if self._cstem[id(n)] is not None:
                    self._s2d_skip.add(id(n.input(0).producer))
        if SPACE_TO_DEPTH:
            order = {id(n): i for i, n in enumerate(graph.nodes)}
            for n in graph.nodes:
                if id(n) in excluded or id(n) in self._cstem or self._s2d_geometry(n) is None:
                    continue
                self._s2d[id(n)] = self._s2d_source(n, order, excluded)
                if self._s2d[id(n)] is not None:
                    self._s2d_skip.add(id(n.input(0).producer))
                self._scratch_bytes = max(self._scratch_bytes, n.input(0).tensor_type.nbytes)
        # Stem blocks read their image in place when it reaches the stem through an NCHW -> NHWC
        # Transpose: id(projection) -> the NCHW tensor.
        self._stem_src: dict[int, Value] = {}
        order = {id(n): i for i, n in enumerate(graph.nodes)}
        for pw in graph.nodes:
            pair = self._mb.get(id(pw))
            if pair is None or not _stem_conv_nhwc(pair[0]):
                continue
            src = self._s2d_source(pair[0], order, excluded - self._mb_skip, reader=pw)
            if src is not None:
                self._stem_src[id(pw)] = src
                self._s2d_skip.add(id(pair[0].input(0).producer))
        # FusedGemm -> LayerNormalization of its rows, scheduled back to back: the LayerNorm runs
        # in the GEMM's split-K reduction. id(gemm) -> (LayerNorm, partials in scratch?)
        self._gemm_ln: dict[int, tuple[Node, bool]] = {}
        self._ln_skip: dict[int, Node] = {}
        if FUSE_GEMM_LAYER_NORM and gemm_ln_workspace is not None:
            taken = excluded | set(self._folds.skipped) | self._s2d_skip | set(self._s2d) | set(self._cstem)
            for node, ln in zip(graph.nodes, graph.nodes[1:]):
                shape = self._gemm_ln_shape(node, ln, taken)
                if shape is None:
                    continue
                need = 4 * int(gemm_ln_workspace(*shape))
                if need <= 0:
                    continue
                off = self.plan.workspaces.get(id(node))
                in_scratch = not (off is not None and self._workspace_bytes(node) >= need
                                  and not (self.plan.location(ln.output).kind == "arena"
                                           and self._region_overlap(ln.output, off, need)))
                if in_scratch:
                    self._scratch_bytes = max(self._scratch_bytes, need)
                self._gemm_ln[id(node)] = (ln, in_scratch)
                self._ln_skip[id(ln)] = node

    def _gemm_ln_shape(self, node: Node, ln: Node, taken: set[int]) -> tuple[int, int, int] | None:
        """(M, N, K) when the LayerNorm ``ln`` can run in ``node``'s split-K reduction: a float
        FusedGemm whose output ``ln`` normalizes over exactly the N output columns, constant
        LayerNorm parameters, and an ``ln`` output that does not overlap the residual the
        reduction reads (an exact alias is fine: each row is read before it is written)."""
        if node.op != "FusedGemm" or ln.op != "LayerNormalization" or ln.input(0) is not node.output:
            return None
        if id(node) in taken or id(ln) in taken:
            return None
        if any(o.users or o in self.graph.outputs for o in ln.outputs[1:]):  # Mean / InvStdDev wanted
            return None
        at, bt, ot = node.input(0).tensor_type, node.input(1).tensor_type, node.output.tensor_type
        if ot.dtype != "float32" or ln.output.tensor_type.dtype != "float32" or ot.rank < 1:
            return None
        trans = int(node.attrs.get("trans_b", 0))
        k, n = (bt.shape[1], bt.shape[0]) if trans else bt.shape
        axis = int(ln.attrs.get("axis", -1))
        axis = axis + ot.rank if axis < 0 else axis
        if axis != ot.rank - 1 or ot.shape[-1] != n or n % 4:
            return None
        if any(v is not None and v.data is None for v in ln.inputs[1:3]):
            return None
        res = node.optional_input(3)
        if res is not None and self._overlap(res, ln.output) and not self._same_storage(res, ln.output):
            return None
        return at.size // max(k, 1), n, k

    def _overlap(self, a: Value, b: Value) -> bool:
        la, lb = self.plan.location(a), self.plan.location(b)
        if la.kind != lb.kind or la.kind == "const":
            return False
        if la.kind in ("input", "output"):
            return la.index == lb.index
        return la.index < lb.index + b.tensor_type.nbytes and lb.index < la.index + a.tensor_type.nbytes

    def _same_storage(self, a: Value, b: Value) -> bool:
        la, lb = self.plan.location(a), self.plan.location(b)
        return la.kind == lb.kind and la.index == lb.index and a.tensor_type.nbytes == b.tensor_type.nbytes

    def _region_overlap(self, v: Value, off: int, nbytes: int) -> bool:
        loc = self.plan.location(v)
        return loc.index < off + nbytes and off < loc.index + v.tensor_type.nbytes

    # -- workspace hook ------------------------------------------------------------------------
    def _gemm_shape(self, node: Node) -> tuple[int, int, int, int] | None:
        if node.op == "FusedGemm":
            a, b = node.input(0).tensor_type, node.input(1).tensor_type
            k, n = (b.shape[1], b.shape[0]) if int(node.attrs.get("trans_b", 0)) else b.shape
            return a.size // max(k, 1), n, k, 1
        if node.op == "Gemm":
            out = node.output.tensor_type
            a = node.input(0).tensor_type
            k = a.shape[0] if int(node.attrs.get("transA", 0)) else a.shape[1]
            return out.shape[0], out.shape[1], k, 1
        if node.op in ("Conv", "FusedConv") and ops.conv_layout(node) == "NHWC" and not self.depthwise(node):
            # the implicit GEMM of one group (groups run one after another on the same workspace)
            out, w = node.output.tensor_type, node.input(1).tensor_type
            kh, kw, cg, kout = w.shape
            group = int(node.attrs.get("group", 1))
            return out.shape[0] * out.shape[1] * out.shape[2], kout // group, kh * kw * cg, 1
        return None

    def _workspace_bytes(self, node: Node) -> int:
        if self._gemm_ws is None:
            return 0
        shape = self._gemm_shape(node)
        if shape is None:
            return 0
        need = 4 * int(self._gemm_ws(*shape))
        ds = self._shortcut.get(id(node))
        if ds is not None:  # the GEMM over both reductions
            m, n, k, batch = shape
            need = max(need, 4 * int(self._gemm_ws(m, n, k + ds.input(0).tensor_type.shape[3], batch)))
        return need

    # -- pointers ------------------------------------------------------------------------------
    def _root(self, value: Value) -> Value:
        while value.data is None and value.producer is not None and value.producer.op in ALIAS_OPS:
            value = value.producer.input(0)
        return value

    def const_offset(self, value: Value) -> int:
        assert value.data is not None
        return self.weights.add(value.data, key=("raw", id(value)))

    def ptr(self, value: Value) -> str:
        """Byte-pointer expression (unsigned char *) of a value's storage."""
        loc = self.plan.location(value)
        if loc.kind == "const":
            root = self._root(value)
            if root.data is None:
                raise CodegenError(f"constant {value.name!r} has no data")
            return f"(W + {self.const_offset(root)})"
        if loc.kind == "input":
            return f"((const unsigned char *)in[{loc.index}])"
        if loc.kind == "output":
            return f"((unsigned char *)out[{loc.index}])"
        return f"(A + {loc.index})"

    def fptr(self, value: Value) -> str:
        return f"((float *){self.ptr(value)})"

    def ws_ptr(self, node: Node) -> str:
        off = self.plan.workspaces.get(id(node))
        return "NULL" if off is None else f"((float *)(A + {off}))"

    def emit(self, line: str) -> None:
        self.body.append(line)

    def count(self, kernel: str) -> None:
        self.kernels[kernel] = self.kernels.get(kernel, 0) + 1

    # -- nodes ---------------------------------------------------------------------------------
    def node(self, node: Node, index: int) -> None:
        types = ", ".join(str(o.type) for o in node.outputs)
        self.emit(f"/* {node.op} {comment_text(node.name)} -> {types} */")
        if self.profile:
            self.emit(f"mgc_hip_node_begin(x, {index});")
        self._lower(node)
        if self.profile:
            self.emit(f"mgc_hip_node_end(x, {index});")

    def _lower(self, node: Node) -> None:
        if id(node) in self._attn_skip:
            m = self._attn_skip[id(node)]
            self.emit(f"/* part of the fused attention at {comment_text(m.emit_at.name)} */")
            return
        if id(node) in self._attn_emit:
            self._attention(self._attn_emit[id(node)])
            return
        if id(node) in self._folds.skipped:
            self.emit(f"/* {self._folds.skipped[id(node)]} */")
            self.count("folded")
            return
        if id(node) in self._s2d_skip:
            self.emit("/* read in NCHW by the launch of the convolution it feeds (space-to-depth copy or stem block) */")
            self.count("folded")
            return
        if id(node) in self._shortcut_skip:
            self.emit("/* projection shortcut: computed in the GEMM of the convolution that adds it */")
            self.count("folded")
            return
        if id(node) in self._dwpw_skip:
            self.emit("/* depthwise convolution: computed in the GEMM of the pointwise convolution that reads it */")
            self.count("folded")
            return
        if id(node) in self._mb_skip:
            self.emit("/* inverted-residual block: computed in the launch of its projection convolution */")
            self.count("folded")
            return
        if id(node) in self._xd_skip:
            self.emit("/* expansion: computed in the launch of the depthwise convolution that reads it */")
            self.count("folded")
            return
        if id(node) in self._ln_skip:
            self.emit(f"/* computed in the split-K reduction of {comment_text(self._ln_skip[id(node)].name)} */")
            return
        if id(node) in self._gln_skip:
            self.emit("/* computed in the launch of the LayerNormalization that reads it (gather + add + LayerNorm) */")
            self.count("folded")
            return
        if id(node) in self._pool_fc_skip:
            self.emit("/* global average pooling: computed in the launch of the fully connected layer that reads it */")
            self.count("folded")
            return
        if node.op in ALIAS_OPS:
            if node.op == "Dropout" and len(node.outputs) > 1:
                mask = node.outputs[1]
                if mask.users or mask in self.graph.outputs:
                    self.emit(f"mgc_hip_fill(x, {self.ptr(mask)}, {mask.tensor_type.size}L, 1, 1ULL);")
            self.count("view")
            return
        if node.op == "FusedElementwise":
            program = [(str(op), dict(a), [int(v) for v in args]) for op, a, args in node.attrs["program"]]
            self.elementwise(node.output, program, list(node.inputs))
            return
        if ops.is_elementwise(node.op):
            args = [i if node.inputs[i] is not None else -1 for i in range(len(node.inputs))]
            self.elementwise(node.output, [(node.op, dict(node.attrs), args)], list(node.inputs))
            return
        getattr(self, f"op_{node.op}")(node)

    # -- elementwise programs ------------------------------------------------------------------
    def _instr_fields(self, op: str, attrs: dict[str, Any], in_dtype: str, out_dtype: str, n_args: int) -> tuple[str, float, float]:
        if op in _ANY_DTYPE:
            return EW_OPCODES[op], 0.0, 0.0
        ok = (
            (in_dtype == "float32" and op in _FLOAT32_OPS)
            or (in_dtype == "float64" and op in _FLOAT64_OPS)
            or (in_dtype in INT_DTYPES and op in _INT_OPS)
        )
        if not ok:
            raise CodegenError(f"elementwise {op} on {in_dtype} is not supported by the hip backend")
        if op == "Gelu":
            tanh = attrs.get("approximate", "none") == "tanh"
            return ("MGC_EW_GELU_TANH" if tanh else "MGC_EW_GELU"), 0.0, 0.0
        if op == "LeakyRelu":
            return EW_OPCODES[op], float(attrs.get("alpha", 0.01)), 0.0
        if op == "HardSigmoid":
            return EW_OPCODES[op], float(attrs.get("alpha", 0.2)), float(attrs.get("beta", 0.5))
        if op == "Clip":
            return EW_OPCODES[op], float(attrs.get("min", -np.inf)), float(attrs.get("max", np.inf))
        return EW_OPCODES[op], 0.0, 0.0

    @staticmethod
    def _cast_pow_exponents(program: list[tuple[str, dict[str, Any], list[int]]],
                            leaves: list[Value | None]) -> list[tuple[str, dict[str, Any], list[int]]]:
        """Pow raises to the exponent converted to the base's dtype (reference ops.py:164-167:
        ``np.power(a, b.astype(a.dtype))``); the kernel evaluates an instruction in one dtype,
        so an exponent of another dtype gets a Cast instruction in front of the Pow."""
        n_leaves = len(leaves)
        types: list[TensorType | None] = [None if v is None else v.type for v in leaves]
        out: list[tuple[str, dict[str, Any], list[int]]] = []
        moved: dict[int, int] = {}  # register of an instruction result -> its register after insertions

        def infer(op: str, attrs: dict[str, Any], args: list[int]) -> TensorType:
            sub = Node(op, [], [Value("_")], dict(attrs))
            return ops.spec(op).infer(sub, [types[a] if a >= 0 else None for a in args], [None] * len(args))[0]

        for k, (op, attrs, args) in enumerate(program):
            args = [moved.get(a, a) if a >= 0 else a for a in args]
            if op == "Pow" and len(args) == 2 and min(args) >= 0 and types[args[0]].dtype != types[args[1]].dtype:
                cast = ("Cast", {"to": types[args[0]].dtype}, [args[1]])
                out.append(cast)
                types.append(infer(*cast))
                args = [args[0], n_leaves + len(out) - 1]
            out.append((op, attrs, args))
            types.append(infer(op, attrs, args))
            moved[n_leaves + k] = n_leaves + len(out) - 1
        return out

    def elementwise(self, out_value: Value, program: list[tuple[str, dict[str, Any], list[int]]], leaves: list[Value | None]) -> None:
        shape = out_value.tensor_type.shape
        program = self._cast_pow_exponents(program, leaves)
        n_leaves = len(leaves)
        if n_leaves > MAX_LEAVES or len(program) > MAX_INSTR:
            raise CodegenError(f"elementwise program too large ({n_leaves} leaves, {len(program)} ops)")
        present = [(i, v) for i, v in enumerate(leaves) if v is not None]
        stride_sets = [_strides(shape)] + [_broadcast_strides(v.tensor_type.shape, shape) for _, v in present]
        dims, coll = collapse(shape, stride_sets)
        if len(dims) > MAX_RANK:
            raise CodegenError(f"elementwise over {len(dims)} non-collapsible dims is not supported")
        total = int(np.prod(dims)) if dims else 1
        if total == 0 or out_value.tensor_type.size == 0:
            self.count("elementwise")
            return
        lines = ["mgc_hip_ew_args e; memset(&e, 0, sizeof e);", f"e.rank = {len(dims)};"]
        for d, n in enumerate(dims):
            lines.append(f"e.dims[{d}] = {n}L; e.out_strides[{d}] = {coll[0][d]}L;")
        lines.append(f"e.n_leaves = {n_leaves}; e.n_instr = {len(program)};")
        for k, (i, v) in enumerate(present):
            st = coll[k + 1]
            lines.append(
                f"e.leaf[{i}].p = {self.ptr(v)}; e.leaf[{i}].dtype = {DTYPE_CODES[v.tensor_type.dtype]};"
                + "".join(f" e.leaf[{i}].strides[{d}] = {s}L;" for d, s in enumerate(st) if s)
            )
        types_all: list[TensorType | None] = [None if v is None else v.type for v in leaves]
        consts: list[np.ndarray | None] = [None if v is None else v.data for v in leaves]
        for k, (op, attrs, args) in enumerate(program):
            sub = Node(op, [], [Value("_")], dict(attrs))
            out_t = ops.spec(op).infer(sub, [types_all[a] if a >= 0 else None for a in args],
                                       [consts[a] if a >= 0 else None for a in args])[0]
            first = next((types_all[a] for a in args if a >= 0), None)
            in_dtype = first.dtype if first is not None else out_t.dtype
            opcode, fa, fb = self._instr_fields(op, attrs, in_dtype, out_t.dtype, len(args))
            regs = [(-1 if a < 0 else (a if a < n_leaves else MAX_LEAVES + a - n_leaves)) for a in args]
            regs = (regs + [-1, -1, -1])[:3]
            lines.append(
                f"e.instr[{k}].op = {opcode}; e.instr[{k}].in_dtype = {DTYPE_CODES[in_dtype]}; "
                f"e.instr[{k}].out_dtype = {DTYPE_CODES[out_t.dtype]}; "
                f"e.instr[{k}].args[0] = {regs[0]}; e.instr[{k}].args[1] = {regs[1]}; "
                f"e.instr[{k}].args[2] = {regs[2]}; e.instr[{k}].fa = {_f(fa)}; e.instr[{k}].fb = {_f(fb)};"
            )
            types_all.append(out_t)
            consts.append(None)
        lines.append(f"e.out = (void *){self.ptr(out_value)}; e.out_dtype = {DTYPE_CODES[out_value.tensor_type.dtype]};")
        lines.append("mgc_hip_elementwise(x, &e);")
        self.emit("{ " + " ".join(lines) + " }")
        self.count("elementwise")

    # -- copies --------------------------------------------------------------------------------
    def copy(self, shape: Sequence[int], out_ptr: str, out_strides: list[int], out_base: int,
             in_ptr: str, in_strides: list[int], in_base: int, elem_bytes: int,
             in_mod: list[int] | None = None) -> None:
        total = int(np.prod(shape)) if len(shape) else 1
        if total == 0:
            return
        if in_mod is None:
            dims, (ost, ist) = collapse(shape, [list(out_strides), list(in_strides)])
            mods = [0] * len(dims)
        else:
            dims, ost, ist, mods = [int(d) for d in shape], list(out_strides), list(in_strides), list(in_mod)
        if len(dims) > MAX_RANK:
            raise CodegenError(f"copy over {len(dims)} non-collapsible dims is not supported")
        parts = ["mgc_hip_copy_args c; memset(&c, 0, sizeof c);", f"c.rank = {len(dims)};"]
        for d, n in enumerate(dims):
            parts.append(
                f"c.dims[{d}] = {n}L; c.out_strides[{d}] = {ost[d]}L; c.in_strides[{d}] = {ist[d]}L; c.in_mod[{d}] = {mods[d]}L;"
            )
        parts.append(f"c.in_base = {in_base}L; c.out_base = {out_base}L; c.in = {in_ptr}; c.out = {out_ptr};")
        parts.append(f"c.elem_bytes = {elem_bytes}; mgc_hip_copy(x, &c);")
        self.emit("{ " + " ".join(parts) + " }")

    def op_Transpose(self, node: Node) -> None:
        xv = node.input(0)
        perm = ops.transpose_perm(node, xv.tensor_type.rank)
        src = _strides(xv.tensor_type.shape)
        out_t = node.output.tensor_type
        self.copy(out_t.shape, self.ptr(node.output), _strides(out_t.shape), 0, self.ptr(xv),
                  [src[p] for p in perm], 0, out_t.itemsize)
        self.count("transpose")

    def op_Expand(self, node: Node) -> None:
        out_t = node.output.tensor_type
        xv = node.input(0)
        self.copy(out_t.shape, self.ptr(node.output), _strides(out_t.shape), 0, self.ptr(xv),
                  _broadcast_strides(xv.tensor_type.shape, out_t.shape), 0, out_t.itemsize)
        self.count("copy")

    def op_Tile(self, node: Node) -> None:
        xv = node.input(0)
        xs, os_ = xv.tensor_type.shape, node.output.tensor_type.shape
        self.copy(os_, self.ptr(node.output), _strides(os_), 0, self.ptr(xv), _strides(xs), 0,
                  xv.tensor_type.itemsize, in_mod=[int(d) for d in xs])
        self.count("copy")

    def op_Slice(self, node: Node) -> None:
        xv = node.input(0)
        xs = xv.tensor_type.shape
        sl = ops.slice_params(node, xs, [None if v is None else v.data for v in node.inputs])
        src = _strides(xs)
        base = sum(int(s.start or 0) * st for s, st in zip(sl, src))
        strides = [int(s.step or 1) * st for s, st in zip(sl, src)]
        out_t = node.output.tensor_type
        self.copy(out_t.shape, self.ptr(node.output), _strides(out_t.shape), 0, self.ptr(xv), strides, base, out_t.itemsize)
        self.count("copy")

    def op_Concat(self, node: Node) -> None:
        out_t = node.output.tensor_type
        axis = int(node.attrs.get("axis", 0))
        axis = axis + out_t.rank if axis < 0 else axis
        ost = _strides(out_t.shape)
        offset = 0
        for v in node.inputs:
            if v is None:
                continue
            t = v.tensor_type
            if t.size:
                self.copy(t.shape, self.ptr(node.output), ost, offset * ost[axis], self.ptr(v),
                          _strides(t.shape), 0, t.itemsize)
            offset += t.shape[axis]
        self.count("copy")

    def op_Split(self, node: Node) -> None:
        xv = node.input(0)
        xt = xv.tensor_type
        axis = int(node.attrs.get("axis", 0))
        axis = axis + xt.rank if axis < 0 else axis
        src = _strides(xt.shape)
        offset = 0
        for out_v in node.outputs:
            t = out_v.tensor_type
            if out_v.users or out_v in self.graph.outputs:
                self.copy(t.shape, self.ptr(out_v), _strides(t.shape), 0, self.ptr(xv), src,
                          offset * src[axis], t.itemsize)
            offset += t.shape[axis]
        self.count("copy")

    def op_Pad(self, node: Node) -> None:
        mode = node.attrs.get("mode", "constant")
        if mode != "constant":
            raise CodegenError(f"Pad mode {mode!r} is not supported by the hip backend")
        xv = node.input(0)
        xt, ot = xv.tensor_type, node.output.tensor_type
        pads = ops.pad_amounts(node, xt.rank, [None if v is None else v.data for v in node.inputs])
        if any(p < 0 for p in pads):
            raise CodegenError("negative Pad amounts are not supported by the hip backend")
        fill_v = node.optional_input(2)
        fill = 0.0
        if fill_v is not None:
            if fill_v.data is None:
                raise CodegenError("Pad value must be a constant")
            fill = fill_v.data.reshape(()).item()
        self._fill(node.output, np.asarray(fill, dtype=numpy_dtype(ot.dtype)))
        ost = _strides(ot.shape)
        base = sum(p * s for p, s in zip(pads[: xt.rank], ost))
        self.copy(xt.shape, self.ptr(node.output), ost, base, self.ptr(xv), _strides(xt.shape), 0, xt.itemsize)
        self.count("copy")

    def _fill(self, value: Value, scalar: np.ndarray) -> None:
        t = value.tensor_type
        if t.size == 0:
            return
        raw = np.zeros(8, np.uint8)
        b = np.asarray(scalar, dtype=numpy_dtype(t.dtype)).reshape(1).view(np.uint8)
        raw[: b.size] = b
        bits = int(raw.view(np.uint64)[0])
        self.emit(f"mgc_hip_fill(x, {self.ptr(value)}, {t.size}L, {t.itemsize}, {bits}ULL);")

    def _write_constant(self, value: Value, array: np.ndarray) -> None:
        t = value.tensor_type
        flat = np.asarray(array, dtype=numpy_dtype(t.dtype)).reshape(-1)
        if flat.size and np.all(flat == flat[0]):
            self._fill(value, flat[0])
            return
        off = self.weights.add(flat)
        self.copy((flat.size,), self.ptr(value), [1], 0, f"(W + {off})", [1], 0, t.itemsize)

    # -- gather and constants ------------------------------------------------------------------
    def op_Gather(self, node: Node) -> None:
        xv, idx = node.input(0), node.input(1)
        xt, it = xv.tensor_type, idx.tensor_type
        axis = int(node.attrs.get("axis", 0))
        axis = axis + xt.rank if axis < 0 else axis
        outer = int(np.prod(xt.shape[:axis])) if axis else 1
        inner = int(np.prod(xt.shape[axis + 1 :])) if axis + 1 < xt.rank else 1
        if it.dtype not in ("int64", "int32"):
            raise CodegenError(f"Gather indices of type {it.dtype} are not supported by the hip backend")
        self.emit(
            f"mgc_hip_gather(x, {self.ptr(xv)}, {self.ptr(idx)}, {DTYPE_CODES[it.dtype]}, {outer}L, "
            f"{xt.shape[axis]}L, {it.size}L, {inner * xt.itemsize}L, {self.ptr(node.output)});"
        )
        self.count("gather")

    def op_Shape(self, node: Node) -> None:
        self._write_constant(node.output, ops.shape_value(node, node.input(0).tensor_type.shape))
        self.count("constant")

    def op_Size(self, node: Node) -> None:
        self._write_constant(node.output, np.asarray([node.input(0).tensor_type.size], np.int64))
        self.count("constant")

    def op_ConstantOfShape(self, node: Node) -> None:
        value = node.attrs.get("value")
        fill = np.asarray(value).reshape(-1)[0].item() if value is not None else 0.0
        self._fill(node.output, np.asarray(fill, dtype=numpy_dtype(node.output.tensor_type.dtype)))
        self.count("constant")

    def op_Range(self, node: Node) -> None:
        t = node.output.tensor_type
        if t.dtype not in ("float32", "float64", "int64", "int32"):
            raise CodegenError(f"Range of {t.dtype} is not supported by the hip backend")
        self.emit(
            f"mgc_hip_range(x, {DTYPE_CODES[t.dtype]}, {self.ptr(node.input(0))}, {self.ptr(node.input(2))}, "
            f"{t.size}L, {self.ptr(node.output)});"
        )
        self.count("constant")

    # -- reductions and normalization ------------------------------------------------------------
    def _reduce(self, node: Node, kind: str) -> None:
        xv = node.input(0)
        xt = xv.tensor_type
        axes = ops.reduce_axes(node, xt.rank, [None if v is None else v.data for v in node.inputs])
        out = node.output
        if not axes:
            self.copy((xt.size,), self.ptr(out), [1], 0, self.ptr(xv), [1], 0, xt.itemsize)
            self.count("reduce")
            return
        if list(axes) != list(range(axes[0], axes[-1] + 1)):
            raise CodegenError(f"{node.op} over non-adjacent axes {axes} is not supported")
        outer = int(np.prod(xt.shape[: axes[0]])) if axes[0] else 1
        n = int(np.prod([xt.shape[a] for a in axes]))
        inner = int(np.prod(xt.shape[axes[-1] + 1 :])) if axes[-1] + 1 < xt.rank else 1
        if kind in ("mean", "max") and xt.dtype == "float32":
            self.emit(f"mgc_hip_reduce_mid(x, {int(kind == 'max')}, {outer}L, {n}L, {inner}L, {self.fptr(xv)}, {self.fptr(out)});")
        else:
            if xt.dtype not in ("float32", "float64", "int64", "int32"):
                raise CodegenError(f"{node.op} on {xt.dtype} is not supported by the hip backend")
            code = {"sum": 0, "mean": 1, "max": 2, "min": 3, "prod": 4}[kind]
            self.emit(f"mgc_hip_reduce(x, {code}, {DTYPE_CODES[xt.dtype]}, {outer}L, {n}L, {inner}L, {self.ptr(xv)}, {self.ptr(out)});")
        self.count("reduce")

    def op_ReduceMean(self, node: Node) -> None:
        self._reduce(node, "mean")

    def op_ReduceSum(self, node: Node) -> None:
        self._reduce(node, "sum")

    def op_ReduceMax(self, node: Node) -> None:
        self._reduce(node, "max")

    def op_ReduceMin(self, node: Node) -> None:
        self._reduce(node, "min")

    def op_ReduceProd(self, node: Node) -> None:
        self._reduce(node, "prod")

    def op_ArgMax(self, node: Node) -> None:
        xv = node.input(0)
        xt = xv.tensor_type
        if xt.dtype not in ("float32", "float64", "int64", "int32"):
            raise CodegenError(f"ArgMax on {xt.dtype} is not supported by the hip backend")
        axis = int(node.attrs.get("axis", 0))
        axis = axis + xt.rank if axis < 0 else axis
        outer = int(np.prod(xt.shape[:axis])) if axis else 1
        inner = int(np.prod(xt.shape[axis + 1 :])) if axis + 1 < xt.rank else 1
        self.emit(f"mgc_hip_argmax(x, {DTYPE_CODES[xt.dtype]}, {outer}L, {xt.shape[axis]}L, {inner}L, {self.ptr(xv)}, (int64_t *){self.ptr(node.output)});")
        self.count("reduce")

    def _require_f32(self, node: Node, t: TensorType) -> None:
        if t.dtype != "float32":
            raise CodegenError(f"{node.op} on {t.dtype} is not supported by the hip backend")

    def _softmax(self, node: Node, log: int) -> None:
        xv = node.input(0)
        xt = xv.tensor_type
        self._require_f32(node, xt)
        axis = int(node.attrs.get("axis", -1))
        axis = axis + xt.rank if axis < 0 else axis
        outer = int(np.prod(xt.shape[:axis])) if axis else 1
        inner = int(np.prod(xt.shape[axis + 1 :])) if axis + 1 < xt.rank else 1
        self.emit(f"mgc_hip_softmax(x, {outer}L, {xt.shape[axis]}L, {inner}L, {self.fptr(xv)}, {self.fptr(node.output)}, {log});")
        self.count("softmax")

    def op_Softmax(self, node: Node) -> None:
        self._softmax(node, 0)

    def op_LogSoftmax(self, node: Node) -> None:
        self._softmax(node, 1)

    def _vector_ptr(self, value: Value | None, n: int, what: str) -> str:
        if value is None:
            return "NULL"
        if value.tensor_type.size != n:
            raise CodegenError(f"{what} must have {n} elements, got {value.tensor_type.shape}")
        if value.tensor_type.dtype != "float32":
            raise CodegenError(f"{what} must be float32")
        return self.fptr(value)

    def op_LayerNormalization(self, node: Node) -> None:
        if id(node) in self._gln:
            self._gather_layer_norm(node, *self._gln[id(node)])
            return
        xv = node.input(0)
        xt = xv.tensor_type
        self._require_f32(node, xt)
        axis = int(node.attrs.get("axis", -1))
        axis = axis + xt.rank if axis < 0 else axis
        cols = int(np.prod(xt.shape[axis:]))
        rows = xt.size // max(cols, 1)
        scale = self._vector_ptr(node.optional_input(1), cols, "LayerNormalization scale")
        bias = self._vector_ptr(node.optional_input(2), cols, "LayerNormalization bias")
        eps = _f(float(node.attrs.get("epsilon", 1e-5)))
        self.emit(f"mgc_hip_layer_norm(x, {rows}L, {cols}L, {self.fptr(xv)}, {scale}, {bias}, {eps}, {self.fptr(node.output)});")
        self.count("layer_norm")

    def _gather_layer_norm(self, ln: Node, gather: Node, add: Node, other: Value, add_rows: int,
                           store_sum: bool) -> None:
        """Gather -> Add -> LayerNormalization as one mgc_hip_gather_layer_norm launch (the
        reference's op_Gather, codegen/c.py:662-688, the Add's loop nest, c.py:360-529, and
        mgc_layer_norm); the sum is stored too when later nodes read it."""
        table, ids = gather.input(0), gather.input(1)
        dim, cols = table.tensor_type.shape
        rows = ids.tensor_type.size
        scale = self._vector_ptr(ln.optional_input(1), cols, "LayerNormalization scale")
        bias = self._vector_ptr(ln.optional_input(2), cols, "LayerNormalization bias")
        eps = _f(float(ln.attrs.get("epsilon", 1e-5)))
        self.emit(
            f"{{ mgc_hip_gather_ln_args gl; gl.table = {self.fptr(table)}; gl.dim = {dim}L; "
            f"gl.idx = {self.ptr(ids)}; gl.idx_dtype = {DTYPE_CODES[ids.tensor_type.dtype]}; "
            f"gl.addend = {self.fptr(other)}; gl.add_rows = {add_rows}L; gl.scale = {scale}; gl.bias = {bias}; "
            f"gl.eps = {eps}; gl.out = {self.fptr(ln.output)}; gl.rows = {rows}L; gl.cols = {cols}; "
            f"gl.sum = {self.fptr(add.output) if store_sum else 'NULL'}; mgc_hip_gather_layer_norm(x, &gl); }}"
        )
        self.count("gather_layer_norm")

    def op_BatchNormalization(self, node: Node) -> None:
        xv = node.input(0)
        xt = xv.tensor_type
        self._require_f32(node, xt)
        params = [None if v is None else v.data for v in node.inputs[1:5]]
        if any(p is None for p in params):
            raise CodegenError("BatchNormalization parameters must be constants")
        scale, bias, mean, var = (np.asarray(p, np.float64) for p in params)
        inv = scale / np.sqrt(var + float(node.attrs.get("epsilon", 1e-5)))
        shift = bias - mean * inv
        c = inv.size
        nhwc = node.attrs.get("layout") == "NHWC"
        bshape = (c,) if nhwc else (c,) + (1,) * (xt.rank - 2)
        g = Graph("bn")
        mul = g.constant(inv.astype(np.float32).reshape(bshape), "bn_mul")
        add = g.constant(shift.astype(np.float32).reshape(bshape), "bn_add")
        self._owned_constants += [mul, add]
        self.elementwise(node.output, [("Mul", {}, [0, 1]), ("Add", {}, [3, 2])], [xv, mul, add])

    # -- GEMM family ---------------------------------------------------------------------------
    def _gemm_call(self, m: int, n: int, k: int, a: list[str], b: list[str], c: str, ldc: int, *,
                   batch: Sequence[tuple[int, int, int, int, int]] = (), alpha: float = 1.0,
                   bias: str = "NULL", bias_mode: int = 0, res: str = "NULL", ldr: int = 0,
                   beta: float = 1.0, act: str = "none", lo: float = 0.0, hi: float = 6.0,
                   workspace: str = "NULL", workspace_floats: int = 0,
                   layer_norm: tuple[str, str, str, str] | None = None, extra: Sequence[str] = (),
                   depthwise: str | None = None, mbconv: str | None = None, stem: str | None = None,
                   extra_flops: int = 0) -> None:
        """One mgc_hip_gemm call; ``layer_norm`` = (scale, bias, eps, out) makes it an
        mgc_hip_gemm_layer_norm call whose split-K reduction also normalizes the rows; ``mbconv``
        declares and fills an mgc_hip_mbconv_args ``mb`` and makes it an mgc_hip_mbconv call (with
        ``stem``, which declares and fills an mgc_hip_stem_args ``st``, mgc_hip_mbconv_stem); ``extra``
        are further field assignments (the concatenated-K operand); ``depthwise`` declares and
        fills an mgc_hip_dw_args ``d`` and makes it an mgc_hip_gemm_dw call."""
        if len(batch) > MAX_BATCH_RANK:
            raise CodegenError(f"GEMM with {len(batch)} batch dimensions is not supported")
        parts = ["mgc_hip_gemm_args g; memset(&g, 0, sizeof g);", f"g.M = {m}; g.N = {n}; g.K = {k};"]
        parts += a + b
        parts.append(f"g.c = (float *){c}; g.ldc = {ldc}L;")
        parts.append(f"g.alpha = {_f(alpha)}; g.beta = {_f(beta)}; g.bias = {bias}; g.bias_mode = {bias_mode};")
        parts.append(f"g.res = {res}; g.ldr = {ldr}L; g.act = {ACT_CODES[act]}; g.lo = {_f(lo)}; g.hi = {_f(hi)};")
        if batch:
            parts.append(f"g.batch_rank = {len(batch)};")
            for d, (dim, abs_, bbs, cbs, rbs) in enumerate(batch):
                parts.append(f"g.batch_dims[{d}] = {dim}; g.a_bs[{d}] = {abs_}L; g.b_bs[{d}] = {bbs}L; g.c_bs[{d}] = {cbs}L; g.r_bs[{d}] = {rbs}L;")
        parts.append(f"g.workspace = {workspace}; g.workspace_floats = {workspace_floats}L;")
        parts += extra
        if layer_norm is not None:
            scale, lbias, eps, out = layer_norm
            parts.append(f"mgc_hip_gemm_layer_norm(x, &g, {scale}, {lbias}, {eps}, {out});")
        elif depthwise is not None:
            parts += [depthwise, "mgc_hip_gemm_dw(x, &g, &d);"]
        elif mbconv is not None and stem is not None:
            parts += [mbconv, stem, "mgc_hip_mbconv_stem(x, &g, &mb, &st);"]
        elif mbconv is not None:
            parts += [mbconv, "mgc_hip_mbconv(x, &g, &mb);"]
        else:
            parts.append("mgc_hip_gemm(x, &g);")
        self.emit("{ " + " ".join(parts) + " }")
        self.count("gemm")
        self._gemm_flops += 2 * m * n * k * math.prod(d for d, *_ in batch) + extra_flops
        if layer_norm is not None:
            self.count("gemm_layer_norm")

    @staticmethod
    def _strided(field_: str, p: str, rs: int, cs: int) -> list[str]:
        return [f"g.{field_}.kind = MGC_OP_STRIDED; g.{field_}.p = (const float *){p}; g.{field_}.rs = {rs}L; g.{field_}.cs = {cs}L;"]

    def _packed_b(self, matrix: np.ndarray, key: Any) -> list[str]:
        """Constant K x N right-hand side stored [N][K]: element (k, n) at n * K + k."""
        k = matrix.shape[0]
        off = self.weights.add(pack_b_nk(matrix), key=key)
        return self._strided("b", f"(W + {off})", 1, k)

    def _act(self, node: Node) -> tuple[str, float, float]:
        return (str(node.attrs.get("activation", "none")), float(node.attrs.get("clip_min", 0.0)),
                float(node.attrs.get("clip_max", 6.0)))

    def _workspace(self, node: Node) -> tuple[str, int]:
        ptr = self.ws_ptr(node)
        if ptr == "NULL":
            return "NULL", 0
        return ptr, self._workspace_bytes(node) // 4

    def op_FusedGemm(self, node: Node) -> None:
        if id(node) in self._pool_fc:
            self._pool_fc_call(node, self._pool_fc[id(node)])
            return
        a, b = node.input(0), node.input(1)
        at, bt = a.tensor_type, b.tensor_type
        self._require_f32(node, at)
        trans = int(node.attrs.get("trans_b", 0))
        k, n = (bt.shape[1], bt.shape[0]) if trans else bt.shape
        m = at.size // max(k, 1)
        if b.data is not None:
            bspec = self._packed_b(b.data.T if trans else b.data, ("packed", id(b), trans))
        else:
            bspec = self._strided("b", self.ptr(b), 1 if trans else n, k if trans else 1)
        bias_v, res_v = node.optional_input(2), node.optional_input(3)
        act, lo, hi = self._act(node)
        ws, ws_floats = self._workspace(node)
        out, layer_norm = self.ptr(node.output), None
        if id(node) in self._gemm_ln:
            ln, in_scratch = self._gemm_ln[id(node)]
            if in_scratch:
                ws, ws_floats = f"(float *)(A + {self._scratch_off})", self._scratch_bytes // 4
            y = node.output
            if not (y in self.graph.outputs or len(y.users) > 1):
                out = "NULL"  # only the LayerNorm reads the GEMM output
            layer_norm = (self._vector_ptr(ln.optional_input(1), n, "LayerNormalization scale"),
                          self._vector_ptr(ln.optional_input(2), n, "LayerNormalization bias"),
                          _f(float(ln.attrs.get("epsilon", 1e-5))), self.fptr(ln.output))
        self._gemm_call(
            m, n, k, self._strided("a", self.ptr(a), k, 1), bspec, out, n,
            bias=self._vector_ptr(bias_v, n, "FusedGemm bias") if bias_v is not None else "NULL",
            bias_mode=1 if bias_v is not None else 0,
            res=self.fptr(res_v) if res_v is not None else "NULL", ldr=n, act=act, lo=lo, hi=hi,
            workspace=ws, workspace_floats=ws_floats, layer_norm=layer_norm,
        )

    def _pool_fc_call(self, node: Node, gap: Node) -> None:
        """GlobalAveragePool (NHWC) -> view -> FusedGemm as one mgc_hip_pool_fc launch: the
        reference's mgc_reduce_mid mean (codegen/c.py:1255-1270) and the GEMM over the pooled
        vectors (c.py:974-1003)."""
        xt = gap.input(0).tensor_type
        nb, h, w, c = xt.shape
        b = node.input(1)
        trans = int(node.attrs.get("trans_b", 0))
        matrix = b.data.T if trans else b.data  # K x N
        f = matrix.shape[1]
        woff = self.weights.add(pack_b_nk(matrix), key=("packed", id(b), trans))
        bias_v = node.optional_input(2)
        act, lo, hi = self._act(node)
        bias = self._vector_ptr(bias_v, f, "FusedGemm bias") if bias_v is not None else "NULL"
        self.emit(
            f"{{ mgc_hip_pool_fc_args pf; pf.x = {self.fptr(gap.input(0))}; pf.w = (const float *)(W + {woff}); "
            f"pf.bias = {bias}; pf.out = {self.fptr(node.output)}; pf.ldo = {f}L; pf.N = {nb}; pf.P = {h * w}; "
            f"pf.C = {c}; pf.F = {f}; pf.act = {ACT_CODES[act]}; pf.lo = {_f(lo)}; pf.hi = {_f(hi)}; "
            f"mgc_hip_pool_fc(x, &pf); }}"
        )
        self.count("pool_fc")

    def op_Gemm(self, node: Node) -> None:
        a, b, c = node.input(0), node.input(1), node.optional_input(2)
        at, bt = a.tensor_type, b.tensor_type
        self._require_f32(node, at)
        ta, tb = int(node.attrs.get("transA", 0)), int(node.attrs.get("transB", 0))
        m, k = (at.shape[1], at.shape[0]) if ta else at.shape
        n = bt.shape[0] if tb else bt.shape[1]
        alpha = float(node.attrs.get("alpha", 1.0))
        beta = float(node.attrs.get("beta", 1.0))
        aspec = self._strided("a", self.ptr(a), 1 if ta else k, m if ta else 1)
        if b.data is not None:
            bspec = self._packed_b(b.data.T if tb else b.data, ("packed", id(b), tb))
        else:
            bspec = self._strided("b", self.ptr(b), 1 if tb else n, k if tb else 1)
        bias, mode, res, ldr = "NULL", 0, "NULL", 0
        if c is not None:
            ct = c.tensor_type
            full = np.broadcast_shapes(ct.shape, (m, n))
            if c.data is not None and ct.size in (1, n) and (ct.rank < 2 or ct.shape[0] == 1):
                vec = np.broadcast_to(c.data.reshape(-1) * beta, (n,)).astype(np.float32)
                bias, mode = f"((const float *)(W + {self.weights.add(vec)}))", 1
            elif c.data is not None and ct.rank == 2 and ct.shape == (m, 1):
                vec = (c.data.reshape(-1) * beta).astype(np.float32)
                bias, mode = f"((const float *)(W + {self.weights.add(vec)}))", 2
            elif tuple(ct.shape) == (m, n) and full == (m, n):
                res, ldr = self.fptr(c), n
            else:
                raise CodegenError(f"Gemm bias of shape {ct.shape} is not supported")
        ws, ws_floats = self._workspace(node)
        self._gemm_call(m, n, k, aspec, bspec, self.ptr(node.output), n, alpha=alpha, bias=bias,
                        bias_mode=mode, res=res, ldr=ldr, beta=beta, workspace=ws, workspace_floats=ws_floats)

    def _operand_view(self, v: Value) -> tuple[str, list[int]]:
        """Pointer and per-dimension element strides a GEMM reads ``v`` through: a folded
        Transpose's output is its input read with permuted strides."""
        t = self._folds.inputs.get(id(v))
        if t is None:
            return self.ptr(v), _strides(v.tensor_type.shape)
        x = t.input(0)
        src = _strides(x.tensor_type.shape)
        return self.ptr(x), [src[p] for p in ops.transpose_perm(t, x.tensor_type.rank)]

    def op_MatMul(self, node: Node) -> None:
        a, b = node.input(0), node.input(1)
        at, bt = a.tensor_type, b.tensor_type
        self._require_f32(node, at)
        ap, ast = self._operand_view(a)
        bp, bst = self._operand_view(b)
        ashape, bshape = tuple(at.shape), tuple(bt.shape)
        if at.rank == 1:  # a row vector [1, k]
            ashape, ast = (1, *ashape), [at.shape[0], *ast]
        if bt.rank == 1:  # a column vector [k, 1]
            bshape, bst = (*bshape, 1), [*bst, 1]
        m, k = ashape[-2], ashape[-1]
        n = bshape[-1]
        batch_shape = tuple(int(d) for d in np.broadcast_shapes(ashape[:-2], bshape[:-2]))
        nb = len(batch_shape)

        def batch_strides(shape: tuple[int, ...], strides: list[int]) -> list[int]:
            pad = nb - (len(shape) - 2)
            return [0 if d < pad or shape[d - pad] == 1 else strides[d - pad] for d in range(nb)]

        a_bs, b_bs = batch_strides(ashape, ast), batch_strides(bshape, bst)
        t = self._folds.outputs.get(id(node))
        if t is not None:
            # write the Transpose's output: MatMul dim i is output dim j where perm[j] = i
            zt = t.output.tensor_type
            perm = ops.transpose_perm(t, zt.rank)
            zs = _strides(zt.shape)
            cst = [zs[perm.index(i)] for i in range(zt.rank)]
            cptr, ldc, c_bs = self.ptr(t.output), cst[-2], cst[:-2]
        else:
            cptr, ldc, c_bs = self.ptr(node.output), n, [s * m * n for s in _strides(batch_shape)]
        dims, (a_c, b_c, c_c) = collapse(batch_shape, [a_bs, b_bs, c_bs])
        batch = [(d, sa, sb, sc, 0) for d, sa, sb, sc in zip(dims, a_c, b_c, c_c)]
        if b.data is not None and not any(b_c) and id(b) not in self._folds.inputs:
            bspec = self._packed_b(b.data.reshape(k, n), ("packed", id(b), 0))
        else:
            bspec = self._strided("b", bp, bst[-2], bst[-1])
        self._gemm_call(m, n, k, self._strided("a", ap, ast[-2], ast[-1]), bspec, cptr, ldc, batch=batch)

    def _attention(self, m: AttentionMatch) -> None:
        HD = m.H * m.D
        if m.qkv_gemms:
            # Q, K and V as one GEMM with the three weight matrices side by side, into scratch
            g0 = m.qkv_gemms[0]
            a = g0.input(0)
            trans = int(g0.attrs.get("trans_b", 0))
            mats = [gm.input(1).data.T if trans else gm.input(1).data for gm in m.qkv_gemms]
            weights = np.ascontiguousarray(np.concatenate(mats, axis=1), np.float32)
            k = weights.shape[0]
            bias, mode = "NULL", 0
            if g0.optional_input(2) is not None:
                vec = np.concatenate([gm.input(2).data.reshape(-1) for gm in m.qkv_gemms]).astype(np.float32)
                bias, mode = f"((const float *)(W + {self.weights.add(vec)}))", 1
            act, lo, hi = self._act(g0)
            qkv = f"(A + {self._scratch_qkv_off})"
            self._gemm_call(m.B * m.S, 3 * HD, k, self._strided("a", self.ptr(a), k, 1),
                            self._packed_b(weights, ("qkv", *(id(gm.input(1)) for gm in m.qkv_gemms), trans)),
                            qkv, 3 * HD, bias=bias, bias_mode=mode, act=act, lo=lo, hi=hi)
            views = [f"((const float *){qkv} + {j * HD})" for j in range(3)]
            strides = [(m.S * 3 * HD, 3 * HD)] * 3
        else:
            views = [f"((const float *){self.ptr(op.value)} + {op.col})" for op in (m.q, m.k, m.v)]
            strides = [(op.batch_stride, op.row_stride) for op in (m.q, m.k, m.v)]

        out = f"((float *)(A + {self._scratch_out_off}))" if m.staged else self.fptr(m.out)
        (qb, qs), (kb, ks), (vb, vs) = strides
        fields = [
            f"t.B = {m.B}; t.H = {m.H}; t.S = {m.S}; t.Skv = {m.Skv}; t.D = {m.D};",
            f"t.q = {views[0]}; t.q_b = {qb}L; t.q_s = {qs}L; t.q_h = {m.D}L;",
            f"t.k = {views[1]}; t.k_b = {kb}L; t.k_s = {ks}L; t.k_h = {m.D}L;",
            f"t.v = {views[2]}; t.v_b = {vb}L; t.v_s = {vs}L; t.v_h = {m.D}L;",
            f"t.o = {out}; t.o_b = {m.S * m.H * m.D}L; t.o_s = {m.H * m.D}L; t.o_h = {m.D}L;",
            f"t.scale = {_f(m.ops.scale)}; t.scale_div = {int(m.ops.divide)};",
        ]
        if m.ops.bias is not None:
            sb, sh, sq, sk = self._score_strides(m.ops.bias)
            fields.append(f"t.bias = {self.fptr(m.ops.bias)}; t.bias_b = {sb}L; t.bias_h = {sh}L; "
                          f"t.bias_s = {sq}L; t.bias_j = {sk}L;")
        if m.ops.causal:
            fields.append(f"t.causal = 1; t.fill = {_f(m.ops.fill)};")
        elif m.ops.mask is not None:
            sb, sh, sq, sk = self._score_strides(m.ops.mask)
            fields.append(f"t.mask = (const unsigned char *){self.ptr(m.ops.mask)}; t.mask_b = {sb}L; "
                          f"t.mask_h = {sh}L; t.mask_s = {sq}L; t.mask_j = {sk}L; "
                          f"t.mask_keep = {int(m.ops.mask_keep)}; t.fill = {_f(m.ops.fill)};")
        self.emit("{ mgc_hip_attention_args t; memset(&t, 0, sizeof t);")
        for f_ in fields:
            self.emit("  " + f_)
        self.emit("  mgc_hip_attention(x, &t); }")
        self.count("attention")
        if m.staged:
            nbytes = m.out.tensor_type.nbytes
            self.copy((nbytes,), self.ptr(m.out), [1], 0, f"(A + {self._scratch_out_off})", [1], 0, 1)

    @staticmethod
    def _score_strides(value: Value) -> list[int]:
        """Element strides over (batch, head, query, key) of a tensor that broadcasts over the
        attention scores [B, H, S, Skv]: 0 for a broadcast dimension."""
        shape = (1,) * (4 - value.tensor_type.rank) + tuple(value.tensor_type.shape)
        strides = _strides(shape)
        return [0 if d == 1 else st for d, st in zip(shape, strides)]

    # -- convolution and pooling ---------------------------------------------------------------
    @staticmethod
    def depthwise(node: Node) -> bool:
        if node.op not in ("Conv", "FusedConv"):
            return False
        group = int(node.attrs.get("group", 1))
        w = node.input(1).tensor_type
        nhwc = node.attrs.get("layout") == "NHWC"
        cg, k = (w.shape[2], w.shape[3]) if nhwc else (w.shape[1], w.shape[0])
        return group > 1 and cg == 1 and k == group

    def op_Conv(self, node: Node) -> None:
        self.op_FusedConv(node)

    def op_FusedConv(self, node: Node) -> None:
        xv, wv = node.input(0), node.input(1)
        xt, wt = xv.tensor_type, wv.tensor_type
        self._require_f32(node, xt)
        nhwc = ops.conv_layout(node) == "NHWC"
        group = int(node.attrs.get("group", 1))
        if nhwc:
            nb, h, wd, c = xt.shape
            kh, kw, cg, kout = wt.shape
        else:
            nb, c, h, wd = xt.shape
            kout, cg, kh, kw = wt.shape
        g = ops.window_geometry(node, (h, wd), (kh, kw))
        oh, ow = g.out_hw
        pt, pl = g.pads[0], g.pads[1]
        bias_v, res_v = node.optional_input(2), node.optional_input(3)
        act, lo, hi = self._act(node) if node.op == "FusedConv" else ("none", 0.0, 6.0)
        bias = self._vector_ptr(bias_v, kout, "Conv bias") if bias_v is not None else "NULL"
        res = self.fptr(res_v) if res_v is not None else "NULL"
        if wv.data is None:
            raise CodegenError("convolution weights must be constant for the hip backend")
        out_ptr = self.ptr(node.output)
        if id(node) in self._xd:
            self._expand_depthwise(node, self._xd[id(node)])
            return
        if self.depthwise(node):
            wflat = wv.data.reshape(kh * kw, c) if nhwc else wv.data.reshape(c, kh * kw)
            woff = self.weights.add(np.ascontiguousarray(wflat, np.float32), key=("dw", id(wv)))
            self.emit(
                f"mgc_hip_depthwise(x, {int(nhwc)}, {nb}, {h}, {wd}, {c}, {kh}, {kw}, {g.strides[0]}, {g.strides[1]}, "
                f"{g.dilations[0]}, {g.dilations[1]}, {pt}, {pl}, {oh}, {ow}, {self.fptr(xv)}, "
                f"(const float *)(W + {woff}), {bias}, {res}, {ACT_CODES[act]}, {_f(lo)}, {_f(hi)}, (float *){out_ptr});"
            )
            self.count("depthwise")
            return
        if id(node) in self._cstem:
            self._conv_stem(node, bias, act, lo, hi)
            return
        if id(node) in self._s2d:
            self._conv_space_to_depth(node, bias, res, act, lo, hi)
            return
        if id(node) in self._shortcut:
            self._conv_with_shortcut(node, self._shortcut[id(node)])
            return
        if id(node) in self._dwpw:
            self._conv_with_depthwise(node, self._dwpw[id(node)])
            return
        if id(node) in self._mb:
            self._inverted_residual(node, *self._mb[id(node)])
            return
        kg = kout // group
        geo = (f"g.{{f}}.H = {h}; g.{{f}}.W = {wd}; g.{{f}}.C = {c}; g.{{f}}.KH = {kh}; g.{{f}}.KW = {kw}; "
               f"g.{{f}}.SH = {g.strides[0]}; g.{{f}}.SW = {g.strides[1]}; g.{{f}}.DH = {g.dilations[0]}; "
               f"g.{{f}}.DW = {g.dilations[1]}; g.{{f}}.PT = {pt}; g.{{f}}.PL = {pl}; g.{{f}}.OH = {oh}; "
               f"g.{{f}}.OW = {ow}; g.{{f}}.cg = {cg};")
        for gi in range(group):
            gbias = f"({bias} + {gi * kg})" if bias != "NULL" else "NULL"
            if nhwc:
                wmat = wv.data[:, :, :, gi * kg : (gi + 1) * kg].reshape(kh * kw * cg, kg)
                bspec = self._packed_b(wmat, ("conv", id(wv), gi))
                pointwise = kh == kw == 1 and g.strides == (1, 1) and g.pads == (0, 0, 0, 0)
                xp = f"({self.fptr(xv)} + {gi * cg})"
                if pointwise:
                    aspec = self._strided("a", xp, c, 1)
                else:
                    aspec = [f"g.a.kind = MGC_OP_CONV_NHWC; g.a.p = {xp}; " + geo.format(f="a")]
                ws, ws_floats = self._workspace(node)
                self._gemm_call(
                    nb * oh * ow, kg, kh * kw * cg, aspec, bspec, f"({self.fptr(node.output)} + {gi * kg})", kout,
                    bias=gbias, bias_mode=1 if bias != "NULL" else 0,
                    res=f"({res} + {gi * kg})" if res != "NULL" else "NULL", ldr=kout, act=act, lo=lo, hi=hi,
                    workspace=ws, workspace_floats=ws_floats,
                )
            else:
                wmat = np.ascontiguousarray(wv.data[gi * kg : (gi + 1) * kg].reshape(kg, cg * kh * kw), np.float32)
                woff = self.weights.add(wmat, key=("convA", id(wv), gi))
                aspec = self._strided("a", f"(W + {woff})", cg * kh * kw, 1)
                bspec = [f"g.b.kind = MGC_OP_CONV_NCHW; g.b.p = ({self.fptr(xv)} + {gi * cg * h * wd}); " + geo.format(f="b")]
                plane = oh * ow
                batch = [(nb, 0, c * h * wd, kout * plane, kout * plane if res != "NULL" else 0)]
                self._gemm_call(
                    kg, plane, cg * kh * kw, aspec, bspec, f"({self.fptr(node.output)} + {gi * kg * plane})", plane,
                    batch=batch, bias=gbias, bias_mode=2 if bias != "NULL" else 0,
                    res=f"({res} + {gi * kg * plane})" if res != "NULL" else "NULL", ldr=plane, act=act, lo=lo, hi=hi,
                )

    def _conv_with_shortcut(self, node: Node, ds: Node) -> None:
        """act(a W3 + x_s Wd + b3 + bd) as one GEMM over K = K1 + C2: a is the pointwise
        convolution's NHWC input (K1 channels), x_s the shortcut's input x sampled at its
        stride (C2 channels), B the two weight matrices stacked along K and the bias their sum.
        The shortcut's output is never written. When a or x is a caller buffer (a graph input or
        output) the generated code checks its 16-byte alignment and otherwise runs the two
        convolutions apart."""
        a, xv = node.input(0), ds.input(0)
        nb, oh, ow, k1 = a.tensor_type.shape
        _, h2, w2, c2 = xv.tensor_type.shape
        w3, wd = node.input(1).data, ds.input(1).data
        n = w3.shape[3]
        stacked = np.concatenate([w3.reshape(k1, n), wd.reshape(c2, n)], axis=0).astype(np.float32)
        bspec = self._packed_b(stacked, ("shortcut", id(node.input(1)), id(ds.input(1))))
        biases = [v.data for v in (node.optional_input(2), ds.optional_input(2)) if v is not None]
        bias = "NULL"
        if biases:  # summed in double, rounded once
            total = sum(np.asarray(b, np.float64).reshape(n) for b in biases)
            bias = f"(const float *)(W + {self.weights.add(total.astype(np.float32), key=('shortcut_bias', id(node)))})"
        sh, sw = ops.window_geometry(ds, (h2, w2), (1, 1)).strides
        act, lo, hi = self._act(node)
        ws, ws_floats = self._workspace(node)
        a2 = (f"g.a2.kind = MGC_OP_CONV_NHWC; g.a2.p = {self.fptr(xv)}; g.a2.H = {h2}; g.a2.W = {w2}; "
              f"g.a2.C = {c2}; g.a2.KH = 1; g.a2.KW = 1; g.a2.SH = {sh}; g.a2.SW = {sw}; g.a2.DH = 1; "
              f"g.a2.DW = 1; g.a2.PT = 0; g.a2.PL = 0; g.a2.OH = {oh}; g.a2.OW = {ow}; g.a2.cg = {c2}; "
              f"g.k1 = {k1};")
        external = [v for v in (a, xv) if self.plan.location(v).kind in ("input", "output")]
        if external:
            cond = " && ".join(f"(((uintptr_t){self.ptr(v)} & 15) == 0)" for v in external)
            self.emit(f"if ({cond}) {{")
        self._gemm_call(nb * oh * ow, n, k1 + c2, self._strided("a", self.fptr(a), k1, 1), bspec,
                        self.fptr(node.output), n, bias=bias, bias_mode=1 if bias != "NULL" else 0,
                        act=act, lo=lo, hi=hi, workspace=ws, workspace_floats=ws_floats, extra=[a2])
        self.count("gemm_shortcut")
        if external:
            self.emit("} else {")
            counted = self._gemm_flops  # the fallback's launches run instead of the fused one
            saved = self._shortcut.pop(id(node))
            try:
                self.op_FusedConv(ds)
                self.op_FusedConv(node)
            finally:
                self._gemm_flops = counted
                self._shortcut[id(node)] = saved
            self.emit("}")

    def _conv_with_depthwise(self, node: Node, dw: Node) -> None:
        """pw(act_d(dw(x))) as one GEMM whose A tiles are the depthwise output, computed from x
        while each tile is staged (mgc_hip_gemm_dw); the depthwise output is never written. When
        x is a caller buffer (a graph input or output) the generated code checks its 16-byte
        alignment and otherwise runs the two convolutions apart."""
        xv = dw.input(0)
        nb, h, wd, c = xv.tensor_type.shape
        g = ops.window_geometry(dw, (h, wd), (3, 3))
        oh, ow = g.out_hw
        wdw = np.ascontiguousarray(dw.input(1).data.reshape(9, c), np.float32)
        dwoff = self.weights.add(wdw, key=("dw", id(dw.input(1))))
        dbias_v = dw.optional_input(2)
        dbias = self._vector_ptr(dbias_v, c, "Conv bias") if dbias_v is not None else "NULL"
        dact, dlo, dhi = self._act(dw) if dw.op == "FusedConv" else ("none", 0.0, 6.0)
        n = node.input(1).tensor_type.shape[3]
        bspec = self._packed_b(node.input(1).data.reshape(c, n), ("conv", id(node.input(1)), 0))
        bias_v, res_v = node.optional_input(2), node.optional_input(3)
        bias = self._vector_ptr(bias_v, n, "Conv bias") if bias_v is not None else "NULL"
        res = self.fptr(res_v) if res_v is not None else "NULL"
        act, lo, hi = self._act(node) if node.op == "FusedConv" else ("none", 0.0, 6.0)
        dws = (f"mgc_hip_dw_args d; memset(&d, 0, sizeof d); d.x = {self.fptr(xv)}; "
               f"d.w = (const float *)(W + {dwoff}); d.bias = {dbias}; d.H = {h}; d.W = {wd}; d.C = {c}; "
               f"d.SH = {g.strides[0]}; d.SW = {g.strides[1]}; d.PT = {g.pads[0]}; d.PL = {g.pads[1]}; "
               f"d.OH = {oh}; d.OW = {ow}; d.act = {ACT_CODES[dact]}; d.lo = {_f(dlo)}; d.hi = {_f(dhi)};")
        external = self.plan.location(xv).kind in ("input", "output")
        if external:
            self.emit(f"if ((((uintptr_t){self.ptr(xv)}) & 15) == 0) {{")
        self._gemm_call(nb * oh * ow, n, c, [], bspec, self.fptr(node.output), n, bias=bias,
                        bias_mode=1 if bias != "NULL" else 0, res=res, ldr=n, act=act, lo=lo, hi=hi,
                        depthwise=dws, extra_flops=ops.flops(dw))
        self.count("gemm_depthwise")
        if external:
            self.emit("} else {")
            counted = self._gemm_flops  # the fallback's launches run instead of the fused one
            saved = self._dwpw.pop(id(node))
            try:
                self.op_FusedConv(dw)
                self.op_FusedConv(node)
            finally:
                self._gemm_flops = counted
                self._dwpw[id(node)] = saved
            self.emit("}")

    def _inverted_residual(self, node: Node, ex: Node, dw: Node) -> None:
        """pw(act_d(dw(act_e(ex(x))))) as one mgc_hip_mbconv launch: the projection GEMM whose
        A operand is the depthwise output of the expansion of x, both evaluated per tile; neither
        intermediate is written. When x is a caller buffer (a graph input or output) the
        generated code checks its 16-byte alignment and otherwise runs the three convolutions
        apart. A stem block (ex a 3 x 3 convolution of a 3-channel image) is one
        mgc_hip_mbconv_stem launch reading the image through its strides (NCHW in place when
        it reaches the stem through a Transpose); its four-byte loads need no alignment check."""
        if _stem_conv_nhwc(ex):
            self._stem_block(node, ex, dw)
            return
        xv = ex.input(0)
        nb, h, wd, cin = xv.tensor_type.shape
        cexp = ex.input(1).tensor_type.shape[3]
        g = ops.window_geometry(dw, (h, wd), (3, 3))
        oh, ow = g.out_hw
        we = self._packed_b(ex.input(1).data.reshape(cin, cexp), ("conv", id(ex.input(1)), 0))[0]
        we_ptr = we.split("g.b.p = ")[1].split(";")[0]
        ebias_v = ex.optional_input(2)
        ebias = self._vector_ptr(ebias_v, cexp, "Conv bias") if ebias_v is not None else "NULL"
        wdw = np.ascontiguousarray(dw.input(1).data.reshape(9, cexp), np.float32)
        dwoff = self.weights.add(wdw, key=("dw", id(dw.input(1))))
        dbias_v = dw.optional_input(2)
        dbias = self._vector_ptr(dbias_v, cexp, "Conv bias") if dbias_v is not None else "NULL"
        eact, elo, ehi = self._act(ex)
        dact, dlo, dhi = self._act(dw)
        n = node.input(1).tensor_type.shape[3]
        bspec = self._packed_b(node.input(1).data.reshape(cexp, n), ("conv", id(node.input(1)), 0))
        bias_v, res_v = node.optional_input(2), node.optional_input(3)
        bias = self._vector_ptr(bias_v, n, "Conv bias") if bias_v is not None else "NULL"
        res = self.fptr(res_v) if res_v is not None else "NULL"
        act, lo, hi = self._act(node) if node.op == "FusedConv" else ("none", 0.0, 6.0)
        mbs = (f"mgc_hip_mbconv_args mb; memset(&mb, 0, sizeof mb); mb.x = {self.fptr(xv)}; "
               f"mb.we = (const float *){we_ptr}; mb.be = {ebias}; mb.wd = (const float *)(W + {dwoff}); "
               f"mb.bd = {dbias}; mb.H = {h}; mb.W = {wd}; mb.Cin = {cin}; mb.Cexp = {cexp}; "
               f"mb.SH = {g.strides[0]}; mb.SW = {g.strides[1]}; mb.PT = {g.pads[0]}; mb.PL = {g.pads[1]}; "
               f"mb.OH = {oh}; mb.OW = {ow}; mb.act_e = {ACT_CODES[eact]}; mb.lo_e = {_f(elo)}; "
               f"mb.hi_e = {_f(ehi)}; mb.act_d = {ACT_CODES[dact]}; mb.lo_d = {_f(dlo)}; mb.hi_d = {_f(dhi)};")
        external = self.plan.location(xv).kind in ("input", "output")
        if external:
            self.emit(f"if ((((uintptr_t){self.ptr(xv)}) & 15) == 0) {{")
        self._gemm_call(nb * oh * ow, n, cexp, [], bspec, self.fptr(node.output), n, bias=bias,
                        bias_mode=1 if bias != "NULL" else 0, res=res, ldr=n, act=act, lo=lo, hi=hi, mbconv=mbs,
                        extra_flops=ops.flops(ex) + ops.flops(dw))
        self.count("gemm_mbconv")
        if external:
            self.emit("} else {")
            saved = self._mb.pop(id(node))
            skipped = {id(ex), id(dw)}
            self._mb_skip -= skipped
            counted = self._gemm_flops  # the fallback's launches run instead of the fused one
            try:
                self.op_FusedConv(ex)
                self.op_FusedConv(dw)
                self.op_FusedConv(node)
            finally:
                self._gemm_flops = counted
                self._mb[id(node)] = saved
                self._mb_skip |= skipped
            self.emit("}")

    def _stem_block(self, node: Node, stem: Node, dw: Node) -> None:
        """pw(act_d(dw(act_s(stem(img))))) as one mgc_hip_mbconv_stem launch: the stem's output
        and the depthwise output are evaluated per 8 x 8-pixel tile and never written; the image
        is read in place through its strides."""
        xv = stem.input(0)
        nb, h0, w0, c0 = xv.tensor_type.shape
        et = dw.input(0).tensor_type
        h, wd, cexp = et.shape[1], et.shape[2], et.shape[3]
        sg = ops.window_geometry(stem, (h0, w0), (3, 3))
        g = ops.window_geometry(dw, (h, wd), (3, 3))
        oh, ow = g.out_hw
        # stem weights [3][3][3][Cexp] -> k = (3 ty + tx) 3 + c, padded to 32 window values
        wmat = np.zeros((32, cexp), np.float32)
        wmat[:27] = stem.input(1).data.reshape(27, cexp)
        we = self._packed_b(wmat, ("stem", id(stem.input(1))))[0]
        we_ptr = we.split("g.b.p = ")[1].split(";")[0]
        ebias_v = stem.optional_input(2)
        ebias = self._vector_ptr(ebias_v, cexp, "Conv bias") if ebias_v is not None else "NULL"
        wdw = np.ascontiguousarray(dw.input(1).data.reshape(9, cexp), np.float32)
        dwoff = self.weights.add(wdw, key=("dw", id(dw.input(1))))
        dbias_v = dw.optional_input(2)
        dbias = self._vector_ptr(dbias_v, cexp, "Conv bias") if dbias_v is not None else "NULL"
        eact, elo, ehi = self._act(stem)
        dact, dlo, dhi = self._act(dw)
        n = node.input(1).tensor_type.shape[3]
        bspec = self._packed_b(node.input(1).data.reshape(cexp, n), ("conv", id(node.input(1)), 0))
        bias_v, res_v = node.optional_input(2), node.optional_input(3)
        bias = self._vector_ptr(bias_v, n, "Conv bias") if bias_v is not None else "NULL"
        res = self.fptr(res_v) if res_v is not None else "NULL"
        act, lo, hi = self._act(node) if node.op == "FusedConv" else ("none", 0.0, 6.0)
        src = self._stem_src.get(id(node))
        if src is not None:  # NCHW [n][c][y][x], read in place
            img, strides = f"(const float *){self.ptr(src)}", (c0 * h0 * w0, h0 * w0, w0, 1)
        else:  # NHWC [n][y][x][c]
            img, strides = self.fptr(xv), (h0 * w0 * c0, 1, w0 * c0, c0)
        mbs = (f"mgc_hip_mbconv_args mb; memset(&mb, 0, sizeof mb); mb.x = NULL; "
               f"mb.we = (const float *){we_ptr}; mb.be = {ebias}; mb.wd = (const float *)(W + {dwoff}); "
               f"mb.bd = {dbias}; mb.H = {h}; mb.W = {wd}; mb.Cin = 32; mb.Cexp = {cexp}; "
               f"mb.SH = {g.strides[0]}; mb.SW = {g.strides[1]}; mb.PT = {g.pads[0]}; mb.PL = {g.pads[1]}; "
               f"mb.OH = {oh}; mb.OW = {ow}; mb.act_e = {ACT_CODES[eact]}; mb.lo_e = {_f(elo)}; "
               f"mb.hi_e = {_f(ehi)}; mb.act_d = {ACT_CODES[dact]}; mb.lo_d = {_f(dlo)}; mb.hi_d = {_f(dhi)};")
        sts = (f"mgc_hip_stem_args st; memset(&st, 0, sizeof st); st.img = {img}; st.C = {c0}; st.H = {h0}; "
               f"st.W = {w0}; st.sn = {strides[0]}L; st.sc = {strides[1]}L; st.sh = {strides[2]}L; "
               f"st.sw = {strides[3]}L; st.KH = 3; st.KW = 3; st.SH = {sg.strides[0]}; st.SW = {sg.strides[1]}; "
               f"st.PT = {sg.pads[0]}; st.PL = {sg.pads[1]};")
        self._gemm_call(nb * oh * ow, n, cexp, [], bspec, self.fptr(node.output), n, bias=bias,
                        bias_mode=1 if bias != "NULL" else 0, res=res, ldr=n, act=act, lo=lo, hi=hi, mbconv=mbs,
                        stem=sts, extra_flops=ops.flops(stem) + ops.flops(dw))
        self.count("gemm_mbconv")
        self.count("mbconv_stem")

    def _expand_depthwise(self, node: Node, ex: Node) -> None:
        """act_d(dw(act_e(ex(x)))) as one mgc_hip_expand_dw launch writing the depthwise node's
        output; the expanded tensor is not written. When x or that output is a caller buffer
        (a graph input or output) the generated code checks its 16-byte alignment and otherwise
        runs the two convolutions apart."""
        xv = ex.input(0)
        nb, h, wd, cin = xv.tensor_type.shape
        cexp = ex.input(1).tensor_type.shape[3]
        g = ops.window_geometry(node, (h, wd), (3, 3))
        oh, ow = g.out_hw
        we = self._packed_b(ex.input(1).data.reshape(cin, cexp), ("conv", id(ex.input(1)), 0))[0]
        we_ptr = we.split("g.b.p = ")[1].split(";")[0]
        ebias_v = ex.optional_input(2)
        ebias = self._vector_ptr(ebias_v, cexp, "Conv bias") if ebias_v is not None else "NULL"
        wdw = np.ascontiguousarray(node.input(1).data.reshape(9, cexp), np.float32)
        dwoff = self.weights.add(wdw, key=("dw", id(node.input(1))))
        dbias_v = node.optional_input(2)
        dbias = self._vector_ptr(dbias_v, cexp, "Conv bias") if dbias_v is not None else "NULL"
        eact, elo, ehi = self._act(ex)
        dact, dlo, dhi = self._act(node)
        args = (f"mgc_hip_expand_dw_args xd; memset(&xd, 0, sizeof xd); xd.x = {self.fptr(xv)}; "
                f"xd.we = (const float *){we_ptr}; xd.be = {ebias}; xd.wd = (const float *)(W + {dwoff}); "
                f"xd.bd = {dbias}; xd.out = {self.fptr(node.output)}; xd.N = {nb}; xd.H = {h}; xd.W = {wd}; "
                f"xd.Cin = {cin}; xd.Cexp = {cexp}; xd.SH = {g.strides[0]}; xd.SW = {g.strides[1]}; "
                f"xd.PT = {g.pads[0]}; xd.PL = {g.pads[1]}; xd.OH = {oh}; xd.OW = {ow}; "
                f"xd.act_e = {ACT_CODES[eact]}; xd.lo_e = {_f(elo)}; xd.hi_e = {_f(ehi)}; "
                f"xd.act_d = {ACT_CODES[dact]}; xd.lo_d = {_f(dlo)}; xd.hi_d = {_f(dhi)};")
        external = [v for v in (xv, node.output) if self.plan.location(v).kind in ("input", "output")]
        if external:
            cond = " && ".join(f"(((uintptr_t){self.ptr(v)} & 15) == 0)" for v in external)
            self.emit(f"if ({cond}) {{")
        self.emit("{ " + args + " mgc_hip_expand_dw(x, &xd); }")
        self.count("expand_depthwise")
        self._gemm_flops += ops.flops(ex) + ops.flops(node)
        if external:
            self.emit("} else {")
            saved = self._xd.pop(id(node))
            self._xd_skip.discard(id(ex))
            counted = self._gemm_flops  # the fallback's launches run instead of the fused one
            try:
                self.op_FusedConv(ex)
                self.op_FusedConv(node)
            finally:
                self._gemm_flops = counted
                self._xd[id(node)] = saved
                self._xd_skip.add(id(ex))
            self.emit("}")

    # -- space-to-depth convolution -------------------------------------------------------------
    @staticmethod
    def _s2d_geometry(node: Node) -> dict[str, int] | None:
        """A stride-2 NHWC convolution whose channel count rules out the 16-byte operand path
        (C % 4 != 0, e.g. an RGB stem) as a stride-1 convolution over the space-to-depth input
        x2[b, i, j, (dy, dx, c)] = x[b, 2i + dy, 2j + dx, c]: tap (t, u) of the new kernel with
        sub-pixel (dy, dx) is tap (2t + dy - 2P + pt, 2u + dx - 2Q + pl) of the original, where
        P = ceil(pt / 2), Q = ceil(pl / 2) are the new top/left pads (zero where that tap is
        outside the original kernel)."""
        if node.op not in ("Conv", "FusedConv") or ops.conv_layout(node) != "NHWC":
            return None
        if int(node.attrs.get("group", 1)) != 1 or node.input(1).data is None:
            return None
        xt, wt = node.input(0).tensor_type, node.input(1).tensor_type
        if xt.dtype != "float32" or xt.rank != 4:
            return None
        nb, h, wd, c = xt.shape
        kh, kw, cg, kout = wt.shape
        g = ops.window_geometry(node, (h, wd), (kh, kw))
        if tuple(g.strides) != (2, 2) or tuple(g.dilations) != (1, 1) or c % 4 == 0 or h % 2 or wd % 2:
            return None
        pt, pl = g.pads[0], g.pads[1]
        P, Q = (pt + 1) // 2, (pl + 1) // 2
        return dict(nb=nb, h=h, w=wd, c=c, kh=kh, kw=kw, kout=kout, pt=pt, pl=pl, P=P, Q=Q,
                    KH=-(-(kh + 2 * P - pt) // 2), KW=-(-(kw + 2 * Q - pl) // 2),
                    oh=g.out_hw[0], ow=g.out_hw[1])

    def _conv_stem_ok(self, node: Node) -> bool:
        """A ResNet stem mgc_hip_conv_stem computes: a float32 NHWC 7 x 7 convolution of a
        3-channel image into 64 channels at stride 2, constant weights, no residual, its output
        in the arena (a caller's output buffer may be misaligned) and the image below the
        launch's 2 GiB offset limit."""
        if node.op not in ("Conv", "FusedConv") or ops.conv_layout(node) != "NHWC":
            return False
        if int(node.attrs.get("group", 1)) != 1 or node.input(1).data is None:
            return False
        if node.optional_input(3) is not None or node.output in self.graph.outputs:
            return False
        xt, wt = node.input(0).tensor_type, node.input(1).tensor_type
        if xt.dtype != "float32" or xt.rank != 4 or xt.shape[3] != 3 or tuple(wt.shape) != (7, 7, 3, 64):
            return False
        g = ops.window_geometry(node, (xt.shape[1], xt.shape[2]), (7, 7))
        if tuple(g.strides) != (2, 2) or tuple(g.dilations) != (1, 1) or min(g.pads) < 0:
            return False
        return xt.nbytes < FUSED_OPERAND_LIMIT

    def _conv_stem(self, node: Node, bias: str, act: str, lo: float, hi: float) -> None:
        """The ResNet stem as one mgc_hip_conv_stem launch: its image window per output tile is
        read in place (NCHW through the strides when a Transpose brought it to NHWC) and the
        weights are packed into the kernel's step order, k pair (c, i, tap columns 2 q, 2 q + 1)
        with the seventh column padded to eight."""
        xv = node.input(0)
        nb, h, wd, c = xv.tensor_type.shape
        g = ops.window_geometry(node, (h, wd), (7, 7))
        oh, ow = g.out_hw
        w = node.input(1).data  # [7][7][3][64]
        wpad = np.zeros((7, 8, 3, 64), np.float32)
        wpad[:, :7] = w
        # [i][q][h][c][b][l] -> [c][i][q][l][h][b]: step e = (c 7 + i) 4 + q, lane (l, h), n block b
        packed = np.ascontiguousarray(wpad.reshape(7, 4, 2, 3, 2, 32).transpose(3, 0, 1, 5, 2, 4), np.float32)
        woff = self.weights.add(packed.reshape(-1), key=("stem7", id(node.input(1))))
        src = self._cstem[id(node)]
        if src is not None:  # NCHW [n][c][y][x], read in place
            img, strides = f"(const float *){self.ptr(src)}", (c * h * wd, h * wd, wd, 1)
        else:  # NHWC [n][y][x][c]
            img, strides = self.fptr(xv), (h * wd * c, 1, wd * c, c)
        self.emit(
            f"{{ mgc_hip_stem_args st; memset(&st, 0, sizeof st); st.img = {img}; st.C = {c}; st.H = {h}; "
            f"st.W = {wd}; st.sn = {strides[0]}L; st.sc = {strides[1]}L; st.sh = {strides[2]}L; "
            f"st.sw = {strides[3]}L; st.KH = 7; st.KW = 7; st.SH = 2; st.SW = 2; st.PT = {g.pads[0]}; "
            f"st.PL = {g.pads[1]}; mgc_hip_conv_stem_args cs; memset(&cs, 0, sizeof cs); "
            f"cs.w = (const float *)(W + {woff}); cs.bias = {bias}; cs.out = {self.fptr(node.output)}; "
            f"cs.ldc = 64; cs.N = {nb}; cs.OH = {oh}; cs.OW = {ow}; cs.act = {ACT_CODES[act]}; "
            f"cs.lo = {_f(lo)}; cs.hi = {_f(hi)}; mgc_hip_conv_stem(x, &st, &cs); }}"
        )
        self.count("gemm_stem")
        self._gemm_flops += ops.flops(node)

    def _s2d_source(self, conv: Node, order: dict[int, int], excluded: set[int], reader: Node | None = None) -> Value | None:
        """The NCHW tensor the space-to-depth copy (or, for a stem block, the launch of
        ``reader``) can read directly when the convolution's input is an NCHW -> NHWC Transpose
        used by nothing else (the Transpose then emits nothing), provided nothing between the
        Transpose and the reading node overwrites that tensor."""
        x = conv.input(0)
        t = x.producer
        if t is None or t.op != "Transpose" or id(t) in excluded or id(t) in self._folds.skipped:
            return None
        if x in self.graph.outputs or x.users != [conv] or ops.transpose_perm(t, 4) != [0, 2, 3, 1]:
            return None
        src = t.input(0)
        for n in self.graph.nodes[order[id(t)] + 1 : order[id(reader or conv)]]:
            if any(fold_overlap(self.plan, o, src) for o in n.outputs):
                return None
            if id(n) in self.plan.workspaces:
                return None
        return src

    def _conv_space_to_depth(self, node: Node, bias: str, res: str, act: str, lo: float, hi: float) -> None:
        s2 = self._s2d_geometry(node)
        assert s2 is not None
        nb, h, wd, c, kout = s2["nb"], s2["h"], s2["w"], s2["c"], s2["kout"]
        h2, w2, c4 = h // 2, wd // 2, 4 * c
        dst = f"(A + {self._scratch_off})"
        src = self._s2d[id(node)]
        out_st = _strides([nb, h2, w2, 2, 2, c])  # x2[b, i, j, dy, dx, c]
        if src is not None and c <= 8:
            # NCHW source [b, c, 2i + dy, 2j + dx]: a thread per output pixel, paired reads
            self.emit(f"mgc_hip_space_to_depth(x, {nb}, {c}, {h}, {wd}, (const float *){self.ptr(src)}, (float *){dst});")
        elif src is not None:
            # walked as (b, i, c, dy, j, dx) so that neighbouring threads read neighbouring
            # source elements
            order = [0, 1, 5, 3, 2, 4]
            in_st = [c * h * wd, 2 * wd, 2, wd, 1, h * wd]
            self.copy([[nb, h2, w2, 2, 2, c][d] for d in order], dst, [out_st[d] for d in order], 0,
                      self.ptr(src), [in_st[d] for d in order], 0, 4)
        else:  # NHWC source [b, 2i + dy, 2j + dx, c]
            in_st = [h * wd * c, 2 * wd * c, 2 * c, wd * c, c, 1]
            self.copy([nb, h2, w2, 2, 2, c], dst, out_st, 0, self.ptr(node.input(0)), in_st, 0, 4)
        self.count("space_to_depth")
        w = node.input(1).data
        KH, KW = s2["KH"], s2["KW"]
        w2m = np.zeros((KH, KW, 2, 2, c, kout), np.float32)
        for t in range(KH):
            for dy in range(2):
                r = 2 * t + dy - 2 * s2["P"] + s2["pt"]
                if not 0 <= r < s2["kh"]:
                    continue
                for u in range(KW):
                    for dx in range(2):
                        q = 2 * u + dx - 2 * s2["Q"] + s2["pl"]
                        if 0 <= q < s2["kw"]:
                            w2m[t, u, dy, dx] = w[r, q]
        kdim = KH * KW * c4
        # the rearranged weights depend on the pads too, so those are part of the blob key
        bspec = self._packed_b(w2m.reshape(kdim, kout), ("s2d", id(node.input(1)), s2["pt"], s2["pl"]))
        oh, ow = s2["oh"], s2["ow"]
        geo = (f"g.a.H = {h2}; g.a.W = {w2}; g.a.C = {c4}; g.a.KH = {KH}; g.a.KW = {KW}; g.a.SH = 1; "
               f"g.a.SW = 1; g.a.DH = 1; g.a.DW = 1; g.a.PT = {s2['P']}; g.a.PL = {s2['Q']}; "
               f"g.a.OH = {oh}; g.a.OW = {ow}; g.a.cg = {c4};")
        aspec = [f"g.a.kind = MGC_OP_CONV_NHWC; g.a.p = (const float *){dst}; " + geo]
        # algorithmic work is the original convolution's (the zero taps of the rearranged kernel
        # are padding the matrix cores execute)
        self._gemm_call(nb * oh * ow, kout, kdim, aspec, bspec, self.ptr(node.output), kout,
                        bias=bias, bias_mode=1 if bias != "NULL" else 0, res=res, ldr=kout,
                        act=act, lo=lo, hi=hi, extra_flops=ops.flops(node) - 2 * nb * oh * ow * kout * kdim)

    def _pool(self, node: Node, is_max: int) -> None:
        xv = node.input(0)
        xt = xv.tensor_type
        self._require_f32(node, xt)
        nhwc = ops.conv_layout(node) == "NHWC"
        nb, h, wd, c = xt.shape if nhwc else (xt.shape[0], xt.shape[2], xt.shape[3], xt.shape[1])
        kernel = [int(k) for k in node.attrs["kernel_shape"]]
        g = ops.window_geometry(node, (h, wd), (kernel[0], kernel[1]), bool(node.attrs.get("ceil_mode", 0)))
        pt, pl, pb, pr = g.pads
        oh, ow = g.out_hw
        include = int(node.attrs.get("count_include_pad", 0))
        self.emit(
            f"mgc_hip_pool(x, {int(nhwc)}, {is_max}, {nb}, {h}, {wd}, {c}, {kernel[0]}, {kernel[1]}, "
            f"{g.strides[0]}, {g.strides[1]}, {g.dilations[0]}, {g.dilations[1]}, {pt}, {pl}, {pb}, {pr}, "
            f"{oh}, {ow}, {include}, {self.fptr(xv)}, {self.fptr(node.output)});"
        )
        self.count("pool")

    def op_MaxPool(self, node: Node) -> None:
        self._pool(node, 1)

    def op_AveragePool(self, node: Node) -> None:
        self._pool(node, 0)

    def _global_pool(self, node: Node, is_max: int) -> None:
        xv = node.input(0)
        xt = xv.tensor_type
        self._require_f32(node, xt)
        if ops.conv_layout(node) == "NHWC":
            outer, n, inner = xt.shape[0], int(np.prod(xt.shape[1:-1])), xt.shape[-1]
        else:
            outer, n, inner = xt.shape[0] * xt.shape[1], int(np.prod(xt.shape[2:])), 1
        self.emit(f"mgc_hip_reduce_mid(x, {is_max}, {outer}L, {n}L, {inner}L, {self.fptr(xv)}, {self.fptr(node.output)});")
        self.count("reduce")

    def op_GlobalAveragePool(self, node: Node) -> None:
        self._global_pool(node, 0)

    def op_GlobalMaxPool(self, node: Node) -> None:
        self._global_pool(node, 1)

    # -- whole program -------------------------------------------------------------------------
    def generate(self) -> GeneratedModel:
        for k, node in enumerate(self.graph.nodes):
            self.node(node, k)
        for value, j in self.plan.copies:
            t = value.tensor_type
            self.copy((t.nbytes,), f"((unsigned char *)out[{j}])", [1], 0, self.ptr(value), [1], 0, 1)
        arena = max(self.plan.arena_bytes, ALIGN)
        if self._scratch_bytes:
            arena = self._scratch_off + (self._scratch_bytes + ALIGN - 1) // ALIGN * ALIGN
        weights = self.weights
        n_in, n_out = len(self.graph.inputs), len(self.graph.named_outputs())
        in_bytes = ", ".join(f"{v.tensor_type.nbytes}UL" for v in self.graph.inputs) or "0UL"
        out_bytes = ", ".join(f"{v.tensor_type.nbytes}UL" for _, v in self.graph.named_outputs()) or "0UL"
        n_prof = len(self.graph.nodes) if self.profile else 0
        head = [
            "/* Generated by ml-graph-compiler (hip backend, gfx950). Host code only: every node is",
            " * one launcher call into libmgc_hip.so with constant offsets. */",
            "#include <stdint.h>",
            "#include <string.h>",
            "#include <math.h>",
            '#include "mgc_hip.h"',
            "",
            f"/* graph {comment_text(self.graph.name)}: {len(self.graph.nodes)} nodes, arena {arena} bytes, "
            f"weights {weights.nbytes} bytes */",
            "",
            "static void mgc_forward(mgc_hip_exec *x, const void *const *in, void *const *out, unsigned char *A,",
            "                        const unsigned char *W) {",
            "    (void)in; (void)out; (void)A; (void)W; (void)x;",
        ]
        tail = [
            "}",
            "",
            f"static const size_t mgc_in_bytes[] = {{{in_bytes}}};",
            f"static const size_t mgc_out_bytes[] = {{{out_bytes}}};",
            f"static mgc_hip_model MODEL = {{{arena}UL, {weights.nbytes}UL, {n_in}, {n_out}, mgc_in_bytes, "
            f"mgc_out_bytes, {n_prof}, mgc_forward, NULL}};",
            "",
            'extern "C" {',
            f"size_t mgc_arena_bytes(void) {{ return {arena}UL; }}",
            f"size_t mgc_weights_bytes(void) {{ return {weights.nbytes}UL; }}",
            "int mgc_hip_init(const unsigned char *w, unsigned char **A, unsigned char **W) {",
            "    return mgc_hip_model_init(&MODEL, w, A, W);",
            "}",
            "int mgc_run(const void *const *inputs, void *const *outputs, unsigned char *A, const unsigned char *W) {",
            "    return mgc_hip_model_run(&MODEL, inputs, outputs, A, W);",
            "}",
            "int mgc_run_device(const void *const *inputs, void *const *outputs, unsigned char *A,",
            "                   const unsigned char *W) {",
            "    return mgc_hip_model_run_device(&MODEL, inputs, outputs, A, W);",
            "}",
            "int mgc_hip_upload(const void *const *inputs) { return mgc_hip_model_upload(&MODEL, inputs); }",
            "int mgc_hip_launch(int replays) { return mgc_hip_model_launch(&MODEL, replays); }",
            "int mgc_hip_sync(void) { return mgc_hip_model_sync(&MODEL); }",
            "int mgc_hip_download(void *const *outputs) { return mgc_hip_model_download(&MODEL, outputs); }",
            "double mgc_hip_time_graph(int replays) { return mgc_hip_model_time_graph(&MODEL, replays); }",
            "void mgc_hip_release(void) { mgc_hip_model_release(&MODEL); }",
            "void mgc_set_num_threads(int n) { (void)n; }",
            "int mgc_get_max_threads(void) { return 1; }",
            "int mgc_has_openmp(void) { return 0; }",
            "int mgc_has_neon(void) { return 0; }",
            "void mgc_set_blocking(int mc, int kc, int npb) { (void)mc; (void)kc; (void)npb; }",
        ]
        if self.profile:
            tail += [
                f"int mgc_profile_size(void) {{ return {n_prof}; }}",
                "const double *mgc_profile_data(void) { return mgc_hip_model_profile_data(&MODEL); }",
                "int mgc_hip_profile_run(int replays) { return mgc_hip_model_profile_run(&MODEL, replays); }",
                "void mgc_hip_profile_reset(void) { mgc_hip_model_profile_reset(&MODEL); }",
            ]
        tail += ["}", ""]
        body = ["    " + line for line in self.body]
        source = "\n".join(head + body + tail)
        return GeneratedModel(
            source=source,
            weights=weights,
            arena_bytes=arena,
            inputs=[(v.name, v.tensor_type) for v in self.graph.inputs],
            outputs=[(name, v.tensor_type) for name, v in self.graph.named_outputs()],
            plan=self.plan,
            lines=source.count("\n"),
            kernels=dict(sorted(self.kernels.items())),
            node_flops=self._node_flops(),
            gemm_flops=self._gemm_flops,
        )

    def _node_flops(self) -> list[int]:
        """FLOPs per node, with the nodes a fused attention call absorbs (among them a QKV
        projection GEMM) counted at the node that emits the call, and a projection shortcut or a
        depthwise convolution at the convolution whose GEMM computes it, and a global average
        pooling at the fully connected layer whose launch computes it: the launches of that
        node do the work."""
        index = {id(n): i for i, n in enumerate(self.graph.nodes)}
        flops = [ops.flops(n) for n in self.graph.nodes]
        for nid, m in self._attn_skip.items():
            i = index[nid]
            flops[index[id(m.emit_at)]] += flops[i]
            flops[i] = 0
        for c3_id, ds in self._shortcut.items():
            i = index[id(ds)]
            flops[index[c3_id]] += flops[i]
            flops[i] = 0
        for pw_id, dw in self._dwpw.items():
            i = index[id(dw)]
            flops[index[pw_id]] += flops[i]
            flops[i] = 0
        for pw_id, pair in self._mb.items():
            for n in pair:
                i = index[id(n)]
                flops[index[pw_id]] += flops[i]
                flops[i] = 0
        for fc_id, gap in self._pool_fc.items():
            i = index[id(gap)]
            flops[index[fc_id]] += flops[i]
            flops[i] = 0
        for dw_id, ex in self._xd.items():
            i = index[id(ex)]
            flops[index[dw_id]] += flops[i]
            flops[i] = 0
        return flops


def generate_hip(
    graph: Graph,
    strategy: Strategy = "greedy_by_size",
    inplace: bool = True,
    profile: bool = False,
    gemm_workspace: Callable[[int, int, int, int], int] | None = None,
    gemm_ln_workspace: Callable[[int, int, int], int] | None = None,
) -> GeneratedModel:
    """Generate the host source and weights blob of a scheduled graph for the hip backend.
    ``gemm_workspace`` / ``gemm_ln_workspace`` ask the kernel library for split-K workspace
    sizes (without the second, no LayerNorm is fused into a GEMM)."""
    return HipEmitter(graph, strategy, inplace, profile, gemm_workspace, gemm_ln_workspace).generate()
