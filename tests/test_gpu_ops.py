"""Every hip lowering, one operator at a time, against the oracle.

The operator list and shapes follow the reference's backend tests
(tests/test_codegen.py:94-396): unary and binary elementwise with broadcasting, comparisons,
integer math, parameterized activations, data movement, reductions, normalization, MatMul and
Gemm variants, convolution (strides, pads, dilations, groups, depthwise, auto_pad) at O0 and O3,
pooling (pads, ceil mode, count_include_pad, dilations) and global pooling. The oracle is the
numpy restatement of the reference interpreter; integer and index results must match exactly.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import pytest

from helpers import check_hip, f32, op_graph, pos, rng

pytestmark = pytest.mark.gpu

UNARY = ["Relu", "Sigmoid", "Tanh", "Erf", "Exp", "Neg", "Abs", "Floor", "Ceil", "Sin", "Cos", "Softplus", "Identity"]


@pytest.mark.parametrize("op", UNARY)
def test_unary(op, hip_cache):
    g, feeds = op_graph(op, [f32(3, 70) * 3])
    check_hip(g, feeds, hip_cache, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("op", ["Sqrt", "Log", "Reciprocal"])
def test_unary_positive(op, hip_cache):
    g, feeds = op_graph(op, [pos(4, 33)])
    check_hip(g, feeds, hip_cache)


@pytest.mark.parametrize("op", ["Add", "Sub", "Mul", "Div", "Max", "Min", "Pow"])
# ((3, 8), ()) and ((2, 1, 4), (3, 1)): a broadcast leaf on the 4-wide path, whose 16-byte load
# reaches past the leaf's last element (those bytes must read as zero, not fault or spill over)
@pytest.mark.parametrize("shapes", [((2, 3, 4), (4,)), ((2, 1, 4), (3, 1)), ((5,), (5,)), ((), (2, 2)),
                                    ((3, 8), ())])
def test_binary_broadcast(op, shapes, hip_cache):
    a = pos(*shapes[0]) if op == "Pow" else f32(*shapes[0])
    g, feeds = op_graph(op, [a, pos(*shapes[1])])
    check_hip(g, feeds, hip_cache)


@pytest.mark.parametrize(
    "op, shapes",
    [
        ("Add", ((3, 1000, 3001), (3, 1000, 3001))),  # one element per item, 9M items
        ("Add", ((4, 2048, 2560), (2560,))),           # four per item: 5.2M items, a bias row
        ("Gelu", ((3, 1024, 3000),)),
    ],
)
def test_elementwise_several_items_per_thread(op, shapes, hip_cache):
    """Launches of more work items than the grid has threads (the grid-stride loop runs
    several trips, the last one partial)."""
    g, feeds = op_graph(op, [f32(*s) for s in shapes])
    check_hip(g, feeds, hip_cache)


@pytest.mark.parametrize("op", ["Equal", "Less", "Greater", "LessOrEqual", "GreaterOrEqual"])
def test_compare(op, hip_cache):
    a = rng.integers(0, 3, (3, 4)).astype(np.float32)
    g, feeds = op_graph(op, [a, rng.integers(0, 3, (4,)).astype(np.float32)])
    check_hip(g, feeds, hip_cache)


@pytest.mark.parametrize("op", ["And", "Or", "Xor"])
def test_logical(op, hip_cache):
    g, feeds = op_graph(op, [rng.random((3, 4)) > 0.5, rng.random((4,)) > 0.5])
    check_hip(g, feeds, hip_cache)


def test_not_where_cast_and_integer_math(hip_cache):
    check_hip(*op_graph("Not", [rng.random((5,)) > 0.5]), hip_cache)
    check_hip(*op_graph("Where", [rng.random((3, 1)) > 0.5, f32(3, 4), f32(4)]), hip_cache)
    for to, src in [(7, f32(6) * 5), (1, np.arange(6, dtype=np.int64)), (9, np.asarray([0, 1, 2, 0], np.float32))]:
        check_hip(*op_graph("Cast", [src], attrs={"to": to}), hip_cache)
    ints = np.asarray([7, -7, 9, 4], np.int64)
    for op in ("Add", "Sub", "Mul", "Div", "Max", "Min"):
        check_hip(*op_graph(op, [ints, np.asarray([2, 2, -4, 3], np.int64)]), hip_cache)


@pytest.mark.parametrize(
    "op, attrs, inputs, const",
    [
        ("Clip", {}, [f32(3, 5), np.asarray(-0.5, np.float32), np.asarray(0.5, np.float32)], {1, 2}),
        ("Clip", {}, [f32(3, 5), None, np.asarray(0.2, np.float32)], {2}),
        ("LeakyRelu", {"alpha": 0.2}, [f32(3, 5)], set()),
        ("HardSigmoid", {}, [f32(3, 5)], set()),
        ("Gelu", {}, [f32(3, 5)], set()),
        ("Gelu", {"approximate": "tanh"}, [f32(3, 5)], set()),
    ],
)
def test_parameterized_elementwise(op, attrs, inputs, const, hip_cache):
    g, feeds = op_graph(op, inputs, const=const, attrs=attrs)
    check_hip(g, feeds, hip_cache, rtol=1e-5, atol=1e-6)


def test_integer_clip(hip_cache):
    g, feeds = op_graph("Clip", [np.arange(-5, 5, dtype=np.int64), np.asarray(-2, np.int64), np.asarray(3, np.int64)], const={1, 2})
    check_hip(g, feeds, hip_cache)


@pytest.mark.parametrize(
    "op, inputs, const, attrs",
    [
        ("Transpose", [f32(2, 3, 4, 5)], set(), {"perm": [0, 2, 3, 1]}),
        ("Transpose", [f32(3, 4)], set(), {}),
        # the LDS-tiled transpose (the contiguous dim moves; both dims >= 32): ragged tiles,
        # one and two batch dims, 8-byte elements
        ("Transpose", [f32(70, 90)], set(), {"perm": [1, 0]}),
        ("Transpose", [f32(4, 64, 33)], set(), {"perm": [0, 2, 1]}),
        ("Transpose", [f32(2, 3, 40, 48)], set(), {"perm": [1, 0, 3, 2]}),
        ("Transpose", [np.arange(40 * 50, dtype=np.int64).reshape(40, 50)], set(), {"perm": [1, 0]}),
        # ... with 16-byte accesses (extents, strides and bases multiples of 16 bytes), ragged tiles
        ("Transpose", [f32(2, 3, 100, 72)], set(), {"perm": [0, 1, 3, 2]}),
        ("Transpose", [f32(36, 5, 68)], set(), {"perm": [2, 1, 0]}),
        ("Transpose", [np.arange(66 * 98, dtype=np.int64).reshape(66, 98)], set(), {"perm": [1, 0]}),
        ("Expand", [f32(3, 1), np.asarray([2, 3, 4], np.int64)], {1}, {}),
        ("Tile", [f32(2, 3), np.asarray([2, 2], np.int64)], {1}, {}),
        ("Slice", [f32(6, 8), np.asarray([1, -6], np.int64), np.asarray([5, 100], np.int64),
                   np.asarray([0, 1], np.int64), np.asarray([2, 3], np.int64)], {1, 2, 3, 4}, {}),
        ("Slice", [f32(6, 8), np.asarray([4], np.int64), np.asarray([0], np.int64),
                   np.asarray([1], np.int64), np.asarray([-2], np.int64)], {1, 2, 3, 4}, {}),
        ("Concat", [f32(2, 3), f32(2, 5), f32(2, 1)], set(), {"axis": 1}),
        ("Concat", [f32(1, 3), f32(2, 3)], {0}, {"axis": 0}),
        ("Pad", [f32(2, 3), np.asarray([1, 0, 2, 3], np.int64), np.asarray(1.5, np.float32)], {1, 2}, {}),
        ("Gather", [f32(10, 4), np.asarray([[1, -1], [3, 0]], np.int64)], set(), {"axis": 0}),
        ("Gather", [f32(3, 10, 2), np.asarray([4, 2], np.int64)], {1}, {"axis": 1}),
        ("Shape", [f32(2, 3, 4)], set(), {}),
        ("Size", [f32(2, 3, 4)], set(), {}),
        ("ConstantOfShape", [np.asarray([2, 3], np.int64)], {0}, {"value": np.asarray([7], np.int64)}),
        ("Range", [np.asarray(1.0, np.float32), np.asarray(9.0, np.float32), np.asarray(1.5, np.float32)], {0, 1, 2}, {}),
        ("ReduceMean", [f32(2, 3, 4)], set(), {"axes": [1, 2], "keepdims": 1}),
        ("ReduceMean", [f32(2, 3, 4)], set(), {"axes": [-1], "keepdims": 0}),
        ("ReduceSum", [f32(2, 3, 4), np.asarray([0, 1], np.int64)], {1}, {"keepdims": 0}),
        ("ReduceMax", [f32(2, 3, 4)], set(), {"axes": [1]}),
        ("ReduceMin", [f32(2, 3, 4)], set(), {"axes": [2]}),
        ("ReduceProd", [pos(2, 3)], set(), {"axes": [1]}),
        ("ArgMax", [f32(3, 7)], set(), {"axis": 1, "keepdims": 0}),
        ("Softmax", [f32(2, 3, 9)], set(), {"axis": -1}),
        ("Softmax", [f32(2, 7, 3)], set(), {"axis": 1}),
        ("LogSoftmax", [f32(4, 9)], set(), {"axis": -1}),
        ("Flatten", [f32(2, 3, 4)], set(), {"axis": 2}),
        ("Unsqueeze", [f32(2, 3), np.asarray([0, 3], np.int64)], {1}, {}),
        ("Squeeze", [f32(2, 1, 3), np.asarray([1], np.int64)], {1}, {}),
        ("Identity", [f32(4)], set(), {}),
    ],
)
def test_data_movement_and_reductions(op, inputs, const, attrs, hip_cache):
    g, feeds = op_graph(op, inputs, const=const, attrs=attrs)
    check_hip(g, feeds, hip_cache, exact=op in COPY_OPS)


# operators that only move data: their outputs must equal the oracle's bit for bit
COPY_OPS = {"Transpose", "Expand", "Tile", "Slice", "Concat", "Pad", "Gather", "Shape", "Size", "ConstantOfShape",
            "Flatten", "Unsqueeze", "Squeeze", "Identity", "ReduceMax", "ReduceMin", "ArgMax"}


@pytest.mark.parametrize(
    "table, indices, axis, const_table",
    [
        # the embedding lookup of BERT-base: a [30522, 768] table and [2, 128] int64 ids with
        # negative ids counting from the end (reference ops.py:596-603 wraps them)
        ("f32", (30522, 768), 0, True),
        ("f32", (10, 4), 0, False),
        ("f32", (6, 1100), 0, False),    # rows of 4400 bytes: more than 256 16-byte chunks
        ("f32", (3, 10, 2), 1, True),
        ("f32", (2, 3, 11), 2, False),
        ("f32", (2, 3, 11), -1, False),
        ("i64", (50, 6), 0, True),       # an int64 table, gathered rows of 48 bytes
        ("i64", (4, 50), 1, False),
        ("i32", (7, 9, 3), 1, False),
        ("f32", (9, 5), 0, False),       # a scalar index: the axis disappears
    ],
)
@pytest.mark.parametrize("index_dtype", [np.int64, np.int32])
def test_gather_bit_exact(table, indices, axis, const_table, index_dtype, hip_cache):
    """Gather is a pure copy: every output bit equals the oracle's (np.take), for float32,
    int64 and int32 tables, int64 and int32 indices, negative indices, every axis."""
    shape = indices
    if table == "f32":
        data = (rng.standard_normal(shape) * 1e3).astype(np.float32)
        data.flat[:: max(1, data.size // 7)] = np.float32(np.nan)   # NaN payloads copy unchanged
    elif table == "i64":
        data = rng.integers(-(2**62), 2**62, shape, dtype=np.int64)
    else:
        data = rng.integers(-(2**31), 2**31 - 1, shape, dtype=np.int64).astype(np.int32)
    dim = shape[axis]
    if shape == (9, 5):
        idx = np.asarray(-3, index_dtype)
    elif shape == (30522, 768):
        idx = rng.integers(-dim, dim, (2, 128)).astype(index_dtype)
    else:
        idx = rng.integers(-dim, dim, (3, 4)).astype(index_dtype)
    g, feeds = op_graph("Gather", [data, idx], const={0} if const_table else set(), attrs={"axis": axis})
    got = check_hip(g, feeds, hip_cache, exact=True)
    want = np.take(data, np.where(idx < 0, idx + dim, idx), axis=axis)
    assert got["out0"].tobytes() == want.tobytes()


def test_split_and_dropout(hip_cache):
    g, feeds = op_graph("Split", [f32(4, 9), np.asarray([2, 3, 4], np.int64)], const={1}, attrs={"axis": 1}, n_outputs=3)
    check_hip(g, feeds, hip_cache)
    g, feeds = op_graph("Dropout", [f32(3, 4)], n_outputs=2)
    check_hip(g, feeds, hip_cache)


def test_layer_and_batch_norm(hip_cache):
    check_hip(*op_graph("LayerNormalization", [f32(2, 5, 16), pos(16), f32(16)], const={1, 2},
                        attrs={"axis": -1, "epsilon": 1e-5}), hip_cache)
    check_hip(*op_graph("LayerNormalization", [f32(2, 3, 4), pos(3, 4)], attrs={"axis": 1}), hip_cache)
    # rows of 768 and 1000 (several float4 per lane, the last partly filled), 1024 (the widest
    # row held in registers), 1028 and 10 (the scalar kernel), and a row without bias
    for cols in (768, 1000, 1024, 1028, 10):
        check_hip(*op_graph("LayerNormalization", [f32(37, cols) * 3 + 1, pos(cols), f32(cols)], const={1, 2},
                            attrs={"axis": -1, "epsilon": 1e-5}), hip_cache)
    check_hip(*op_graph("LayerNormalization", [f32(5, 768), np.ones(768, np.float32)], const={1}), hip_cache)
    check_hip(*op_graph("BatchNormalization", [f32(2, 3, 4, 5), pos(3), f32(3), f32(3), pos(3)], const={1, 2, 3, 4}),
              hip_cache)


@pytest.mark.parametrize(
    "a_shape, b_shape, const_b",
    [
        ((5, 7), (7, 3), False),
        ((5, 7), (7, 30), True),
        ((2, 3, 5, 7), (7, 9), True),
        ((2, 3, 5, 7), (2, 3, 7, 4), False),
        ((2, 1, 5, 7), (3, 7, 4), False),
        ((7,), (7, 5), False),
        ((4, 7), (7,), False),
        ((1, 1), (1, 1), False),
        ((33, 65), (65, 29), True),
        ((200, 136), (136, 264), True),
        ((3, 130, 68), (3, 68, 132), False),
        # narrow outputs take 128 x 32 tiles (N = 24, 96, 160, 16); N = 40 pads the same either way
        ((300, 64), (64, 24), True),
        ((257, 96), (96, 96), True),
        ((129, 128), (128, 160), True),
        ((64, 16), (16, 16), True),
        ((130, 32), (32, 40), True),
    ],
)
def test_matmul(a_shape, b_shape, const_b, hip_cache):
    g, feeds = op_graph("MatMul", [f32(*a_shape), f32(*b_shape)], const={1} if const_b else set())
    check_hip(g, feeds, hip_cache)


@pytest.mark.parametrize(
    "attrs, c_shape",
    [
        ({}, None),
        ({"transA": 1}, (3,)),
        ({"transB": 1, "alpha": 0.5, "beta": 2.0}, (1, 3)),
        ({"beta": 0.5}, (4, 3)),
        ({}, (4, 1)),
        ({}, ()),
    ],
)
def test_gemm(attrs, c_shape, hip_cache):
    a = f32(5, 4) if attrs.get("transA") else f32(4, 5)
    b = f32(3, 5) if attrs.get("transB") else f32(5, 3)
    inputs = [a, b] + ([f32(*c_shape)] if c_shape is not None else [])
    check_hip(*op_graph("Gemm", inputs, const={1, 2}, attrs=attrs), hip_cache)
    if c_shape in ((4, 3), None):
        check_hip(*op_graph("Gemm", inputs, attrs=attrs), hip_cache)


CONV_CASES = [
    ({"kernel_shape": [3, 3], "pads": [1, 1, 1, 1]}, (1, 4, 9, 8), (6, 4, 3, 3)),
    ({"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 0, 1, 2]}, (2, 3, 11, 9), (5, 3, 3, 3)),
    ({"kernel_shape": [2, 3], "dilations": [2, 1]}, (1, 2, 9, 9), (4, 2, 2, 3)),
    ({"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 2}, (1, 4, 6, 6), (6, 2, 3, 3)),
    ({"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 4}, (1, 4, 7, 7), (4, 1, 3, 3)),
    ({"kernel_shape": [3, 3], "group": 4, "strides": [2, 2]}, (2, 4, 9, 9), (8, 1, 3, 3)),
    ({"kernel_shape": [1, 1]}, (1, 16, 5, 5), (24, 16, 1, 1)),
    ({"kernel_shape": [3, 3], "auto_pad": "SAME_UPPER", "strides": [2, 2]}, (1, 3, 8, 8), (4, 3, 3, 3)),
    ({"kernel_shape": [3, 3], "pads": [1, 1, 1, 1]}, (2, 64, 10, 12), (96, 64, 3, 3)),
    ({"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 32}, (2, 32, 9, 9), (32, 1, 3, 3)),
    # depthwise over NHWC at O3 (C % 4 == 0): the 3x3 kernel with four output pixels per thread
    # (output widths that are not a multiple of four, strides 1 and 2 on either axis, asymmetric
    # pads) and the general kernel (dilation, 5x5)
    ({"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 16}, (2, 16, 7, 13), (16, 1, 3, 3)),
    ({"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 16, "strides": [2, 2]}, (2, 16, 15, 15), (16, 1, 3, 3)),
    ({"kernel_shape": [3, 3], "pads": [0, 1, 2, 0], "group": 8, "strides": [2, 2]}, (1, 8, 10, 10), (8, 1, 3, 3)),
    ({"kernel_shape": [3, 3], "pads": [2, 0, 0, 2], "group": 8, "strides": [1, 2]}, (1, 8, 6, 11), (8, 1, 3, 3)),
    ({"kernel_shape": [3, 3], "group": 12, "strides": [2, 1]}, (1, 12, 9, 6), (12, 1, 3, 3)),
    ({"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 8}, (1, 8, 5, 30), (8, 1, 3, 3)),   # four per thread
    ({"kernel_shape": [3, 3], "pads": [1, 0, 1, 1], "group": 8, "strides": [2, 2]}, (1, 8, 9, 62), (8, 1, 3, 3)),
    ({"kernel_shape": [3, 3], "pads": [2, 2, 2, 2], "group": 8, "dilations": [2, 2]}, (1, 8, 9, 9), (8, 1, 3, 3)),
    ({"kernel_shape": [5, 5], "pads": [2, 2, 2, 2], "group": 8}, (1, 8, 9, 9), (8, 1, 5, 5)),
    # narrow output channels (128 x 32 tiles at O3): pointwise and 3x3
    ({"kernel_shape": [1, 1]}, (2, 32, 9, 9), (24, 32, 1, 1)),
    ({"kernel_shape": [3, 3], "pads": [1, 1, 1, 1]}, (1, 16, 12, 12), (96, 16, 3, 3)),
]


@pytest.mark.parametrize("attrs, x_shape, w_shape", CONV_CASES)
@pytest.mark.parametrize("opt", ["O0", "O3"])
def test_conv(attrs, x_shape, w_shape, opt, hip_cache):
    g, feeds = op_graph("Conv", [f32(*x_shape), f32(*w_shape) * 0.3, f32(w_shape[0])], const={1, 2}, attrs=attrs)
    check_hip(g, feeds, hip_cache, opt=opt)


def test_depthwise_with_residual_and_clip(hip_cache):
    """Depthwise 3x3 with the residual Add and the ReLU6 Clip fused into its epilogue (O3)."""
    from ml_graph_compiler.ir import Graph, TensorType
    from ml_graph_compiler.shape_inference import infer_shapes

    for stride, hw in ((1, 10), (1, 7)):
        g = Graph("dw_res")
        x = g.add_input("x", TensorType("float32", (2, 16, hw, hw)))
        w = g.constant(f32(16, 1, 3, 3) * 0.3, "w")
        b = g.constant(f32(16), "b")
        y = g.add_node("Conv", [x, w, b], 1, {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 16,
                                               "strides": [stride, stride]}, name="dw").output
        y = g.add_node("Add", [y, x], 1, {}, name="res").output
        lo = g.constant(np.asarray(0.0, np.float32), "lo")
        hi = g.constant(np.asarray(6.0, np.float32), "hi")
        y = g.add_node("Clip", [y, lo, hi], 1, {}, name="clip").output
        g.add_output(y, "y")
        infer_shapes(g)
        check_hip(g, {"x": f32(2, 16, hw, hw) * 3}, hip_cache, opt="O3")


@pytest.mark.parametrize(
    "x_shape, stride",
    [
        ((1, 32, 30, 30), 1),     # at most 2^18 output quads: the LDS-tiled kernel
        ((1, 48, 61, 61), 2),
        ((2, 64, 60, 60), 1),
        ((2, 64, 112, 112), 1),   # more, wide rows: the preloading kernel, two outputs per thread
        ((2, 64, 240, 240), 2),   # ... stride 2
        ((64, 64, 20, 20), 1),    # narrow rows: the row-streaming kernel, one 64-column strip
                                  # (16 quads) per image, 20 of its columns used
        ((1, 1024, 130, 130), 1), # wide rows over 64 MB of input: the row-streaming kernel, four
                                  # slices of 64 quads, strips of 16 columns (130 = 8 x 16 + 2)
        ((12, 272, 26, 26), 1),   # narrow rows, two slices of 34 quads, one 28-column strip
                                  # (26 used), runs of 4 rows
        ((48, 144, 26, 26), 1),   # 144 channels in one 36-quad slice
    ],
)
def test_depthwise_kernels_by_launch_size(x_shape, stride, hip_cache):
    c = x_shape[1]
    attrs = {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": c, "strides": [stride, stride]}
    g, feeds = op_graph("Conv", [f32(*x_shape), f32(c, 1, 3, 3) * 0.3, f32(c)], const={1, 2}, attrs=attrs)
    check_hip(g, feeds, hip_cache, opt="O3")


@pytest.mark.parametrize("pads", [[1, 1, 1, 1], [0, 0, 0, 0], [0, 1, 1, 0]])
def test_row_streaming_depthwise_residual_clip(pads, hip_cache):
    """The row-streaming stride-1 kernel (narrow rows, more than 2^18 output quads) with the
    residual Add and ReLU6 in its epilogue, at the three paddings it takes (top and left 0 or
    1; the output rows then start at input row 0 or -1)."""
    from ml_graph_compiler.ir import Graph, TensorType
    from ml_graph_compiler.shape_inference import infer_shapes

    n, c, hw = 40, 96, 22
    oh = hw + pads[0] + pads[2] - 2
    g = Graph("dw_rows")
    x = g.add_input("x", TensorType("float32", (n, c, hw, hw)))
    r = g.add_input("r", TensorType("float32", (n, c, oh, hw + pads[1] + pads[3] - 2)))
    w = g.constant(f32(c, 1, 3, 3) * 0.3, "w")
    b = g.constant(f32(c), "b")
    y = g.add_node("Conv", [x, w, b], 1, {"kernel_shape": [3, 3], "pads": pads, "group": c}, name="dw").output
    y = g.add_node("Add", [y, r], 1, {}, name="res").output
    lo = g.constant(np.asarray(0.0, np.float32), "lo")
    hi = g.constant(np.asarray(6.0, np.float32), "hi")
    y = g.add_node("Clip", [y, lo, hi], 1, {}, name="clip").output
    g.add_output(y, "y")
    infer_shapes(g)
    ow = hw + pads[1] + pads[3] - 2
    check_hip(g, {"x": f32(n, c, hw, hw) * 3, "r": f32(n, c, oh, ow)}, hip_cache, opt="O3")


def test_narrow_pointwise_with_residual(hip_cache):
    """A 24-channel pointwise convolution (128 x 32 tiles) with the residual Add and ReLU in its
    epilogue (O3), over an image whose pixel count is not a multiple of the tile height."""
    from ml_graph_compiler.ir import Graph, TensorType
    from ml_graph_compiler.shape_inference import infer_shapes

    g = Graph("pw_res")
    x = g.add_input("x", TensorType("float32", (3, 24, 10, 9)))
    w = g.constant(f32(24, 24, 1, 1) * 0.3, "w")
    b = g.constant(f32(24), "b")
    y = g.add_node("Conv", [x, w, b], 1, {"kernel_shape": [1, 1]}, name="pw").output
    y = g.add_node("Add", [y, x], 1, {}, name="res").output
    y = g.add_node("Relu", [y], 1, {}, name="relu").output
    g.add_output(y, "y")
    infer_shapes(g)
    check_hip(g, {"x": f32(3, 24, 10, 9)}, hip_cache, opt="O3")


POOL_CASES = [
    {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]},
    {"kernel_shape": [2, 2], "strides": [2, 2]},
    {"kernel_shape": [3, 3], "strides": [2, 2], "ceil_mode": 1},
    {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "count_include_pad": 1},
    {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1], "ceil_mode": 1},
    {"kernel_shape": [2, 2], "dilations": [2, 2]},
]


@pytest.mark.parametrize("attrs", POOL_CASES)
@pytest.mark.parametrize("op", ["MaxPool", "AveragePool"])
@pytest.mark.parametrize("opt", ["O0", "O3"])
def test_pooling(op, attrs, opt, hip_cache):
    if op == "MaxPool":
        attrs = {k: v for k, v in attrs.items() if k != "count_include_pad"}
    g, feeds = op_graph(op, [f32(2, 3, 9, 10)], attrs=attrs)
    check_hip(g, feeds, hip_cache, opt=opt)
    # eight channels: at O3 the NHWC 16-byte kernel (3x3 windows unrolled, other windows generic)
    g, feeds = op_graph(op, [f32(2, 8, 9, 10)], attrs=attrs)
    check_hip(g, feeds, hip_cache, opt=opt)


@pytest.mark.parametrize("op", ["GlobalAveragePool", "GlobalMaxPool"])
@pytest.mark.parametrize("opt", ["O0", "O3"])
def test_global_pooling(op, opt, hip_cache):
    g, feeds = op_graph(op, [f32(2, 5, 4, 3)])
    check_hip(g, feeds, hip_cache, opt=opt)


# Mean and max over the middle axes of an NHWC-shaped tensor (what global pooling becomes at
# O3): channels divisible by four take the 16-byte kernel, with 16 column quads and 16 row parts
# per workgroup for windows of 32 or more pixels (7 x 7, 6 x 6: tails of both the column blocks
# and the row parts) and 64 column quads and 4 row parts below that.
@pytest.mark.parametrize("op", ["ReduceMean", "ReduceMax"])
@pytest.mark.parametrize("shape", [(2, 7, 7, 8), (2, 6, 6, 72), (3, 4, 4, 264), (1, 3, 5, 12)])
def test_reduce_middle_axes_vec4(op, shape, hip_cache):
    g, feeds = op_graph(op, [f32(*shape)], attrs={"axes": [1, 2], "keepdims": 1})
    check_hip(g, feeds, hip_cache, opt="O3")
