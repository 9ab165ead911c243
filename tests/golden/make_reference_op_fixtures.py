"""Writes tests/golden/reference_ops.npz + reference_ops.json: input/output vectors of every
operator the oracle implements, computed by the reference implementation itself.

Run in the build container only (it imports /root/reference/src; the GPU box has no copy):

    python tests/golden/make_reference_op_fixtures.py

The reference's operator semantics live in the ``run`` functions of its ops module
(src/ml_graph_compiler/ops.py:122-1202), which need only numpy. This script builds one
reference ``Node`` per case, calls the reference's ``ops.run`` on seeded inputs and stores the
inputs, attributes and outputs. The fixture holds only data; nothing of the reference's source
is kept. tests/test_reference_op_vectors.py then checks the oracle (oracle/interpreter.py)
against every vector, and tests/test_gpu_reference_vectors.py the hip backend.

Each case lists which inputs a compiled graph must see as constants (shape operands, axes,
pads, clip bounds): the reference needs them at compile time too.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REFERENCE_SRC = Path("/root/reference/src")

rng = np.random.default_rng(20261202)


def f32(*shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def pos(*shape):
    return (rng.random(shape) + 0.5).astype(np.float32)


def i64(*shape, lo=-9, hi=10):
    return rng.integers(lo, hi, shape).astype(np.int64)


def i32(*shape, lo=-9, hi=10):
    return rng.integers(lo, hi, shape).astype(np.int32)


def nonzero(a):
    """``a`` with every zero replaced by 3 (integer divisors)."""
    return np.where(a == 0, 3, a).astype(a.dtype)


def boolean(*shape):
    return rng.random(shape) > 0.5


def c64(*values):
    return np.asarray(values, np.int64)


def scalar(v, dtype=np.float32):
    return np.asarray(v, dtype)


def cases():
    """(name, op, inputs, const input indices, attrs, number of outputs)."""
    out = []

    def add(name, op, inputs, const=(), attrs=None, n_out=1):
        out.append((name, op, inputs, sorted(const), attrs or {}, n_out))

    # binary arithmetic with broadcasting, float and integer (integer Div truncates)
    for op in ("Add", "Sub", "Mul", "Div", "Max", "Min"):
        add(f"{op}_f32_bcast", op, [f32(2, 3, 4), pos(4)])
        add(f"{op}_f32_outer", op, [f32(3, 1), f32(1, 5)])
        add(f"{op}_i64", op, [i64(4, 5), nonzero(i64(5))])
        add(f"{op}_i32", op, [i32(6), nonzero(i32(6))])
    add("Div_i64_signs", "Div", [c64(7, -7, 9, -9, 0), c64(2, 2, -4, -4, 5)])
    add("Pow_f32", "Pow", [pos(3, 4), f32(4)])
    add("Pow_f32_int_exponent", "Pow", [f32(5), np.asarray([2, 3, 0, 1, 2], np.int64)])
    # comparisons and logic
    for op in ("Equal", "Less", "Greater", "LessOrEqual", "GreaterOrEqual"):
        add(f"{op}_f32", op, [rng.integers(0, 3, (3, 4)).astype(np.float32), rng.integers(0, 3, (4,)).astype(np.float32)])
        add(f"{op}_i64", op, [i64(5, lo=0, hi=3), i64(1, lo=0, hi=3)])
    for op in ("And", "Or", "Xor"):
        add(op, op, [boolean(3, 4), boolean(4)])
    add("Not", "Not", [boolean(7)])
    add("Where_f32", "Where", [boolean(3, 1), f32(3, 4), f32(4)])
    add("Where_i64", "Where", [boolean(5), i64(5), i64(1)])
    # unary
    for op in ("Relu", "Sigmoid", "Tanh", "Erf", "Exp", "Neg", "Abs", "Floor", "Ceil", "Sin", "Cos", "Softplus",
               "Identity"):
        add(f"{op}_f32", op, [f32(4, 25, scale=3.0)])
    for op in ("Sqrt", "Log", "Reciprocal"):
        add(f"{op}_f32", op, [pos(4, 25)])
    add("Neg_i64", "Neg", [i64(6)])
    add("Abs_i64", "Abs", [i64(6)])
    add("Relu_i64", "Relu", [i64(6)])
    add("Gelu_erf", "Gelu", [f32(50, scale=3.0)])
    add("Gelu_tanh", "Gelu", [f32(50, scale=3.0)], attrs={"approximate": "tanh"})
    add("LeakyRelu_default", "LeakyRelu", [f32(40, scale=2.0)])
    add("LeakyRelu_alpha", "LeakyRelu", [f32(40, scale=2.0)], attrs={"alpha": 0.3})
    add("HardSigmoid_default", "HardSigmoid", [f32(40, scale=4.0)])
    add("HardSigmoid_attrs", "HardSigmoid", [f32(40, scale=4.0)], attrs={"alpha": 0.5, "beta": 0.25})
    add("Clip_inputs", "Clip", [f32(3, 5), scalar(-0.5), scalar(0.5)], const={1, 2})
    add("Clip_max_only", "Clip", [f32(3, 5), None, scalar(0.2)], const={2})
    add("Clip_attrs", "Clip", [f32(3, 5)], attrs={"min": -0.1, "max": 0.3})
    add("Clip_i64", "Clip", [np.arange(-5, 5, dtype=np.int64), scalar(-2, np.int64), scalar(3, np.int64)], const={1, 2})
    add("Clip_i32", "Clip", [i32(8), scalar(-3, np.int32), scalar(4, np.int32)], const={1, 2})
    for to, src in ((7, f32(6, scale=5.0)), (6, f32(6, scale=5.0)), (1, i64(6)), (9, np.asarray([0, 1, 2, 0], np.float32)),
                    (11, f32(4)), (1, boolean(5)), (7, boolean(5))):
        add(f"Cast_to{to}_{src.dtype}", "Cast", [src], attrs={"to": to})
    add("Dropout_two_outputs", "Dropout", [f32(3, 4)], n_out=2)
    add("Dropout_one_output", "Dropout", [f32(3, 4)])
    # shape manipulation
    add("Reshape_infer", "Reshape", [f32(2, 3, 4), c64(4, -1)], const={1})
    add("Reshape_zero", "Reshape", [f32(2, 3, 4), c64(0, 12)], const={1})
    add("Flatten_axis2", "Flatten", [f32(2, 3, 4)], attrs={"axis": 2})
    add("Flatten_axis0", "Flatten", [f32(2, 3)], attrs={"axis": 0})
    add("Transpose_perm", "Transpose", [f32(2, 3, 4, 5)], attrs={"perm": [0, 2, 3, 1]})
    add("Transpose_default", "Transpose", [f32(3, 4)])
    add("Transpose_i64", "Transpose", [i64(3, 5)], attrs={"perm": [1, 0]})
    add("Squeeze_axes", "Squeeze", [f32(2, 1, 3, 1), c64(1)], const={1})
    add("Squeeze_all", "Squeeze", [f32(2, 1, 3, 1)])
    add("Unsqueeze_axes", "Unsqueeze", [f32(2, 3), c64(0, 3)], const={1})
    add("Unsqueeze_negative", "Unsqueeze", [f32(2, 3), c64(-1)], const={1})
    add("Concat_axis1", "Concat", [f32(2, 3), f32(2, 5), f32(2, 1)], attrs={"axis": 1})
    add("Concat_axis_neg", "Concat", [i64(2, 3), i64(2, 2)], attrs={"axis": -1})
    add("Split_sizes", "Split", [f32(4, 9), c64(2, 3, 4)], const={1}, attrs={"axis": 1}, n_out=3)
    add("Split_even", "Split", [f32(6, 4)], attrs={"axis": 0}, n_out=3)
    add("Split_num_outputs", "Split", [f32(2, 7)], attrs={"axis": 1, "num_outputs": 3}, n_out=3)
    add("Slice_steps", "Slice", [f32(6, 8), c64(1, -6), c64(5, 100), c64(0, 1), c64(2, 3)], const={1, 2, 3, 4})
    add("Slice_negative_step", "Slice", [f32(6, 8), c64(4), c64(0), c64(1), c64(-2)], const={1, 2, 3, 4})
    add("Slice_default_axes", "Slice", [f32(5, 6), c64(1, 2), c64(4, -1)], const={1, 2})
    add("Gather_axis0", "Gather", [f32(10, 4), np.asarray([[1, -1], [3, 0]], np.int64)], attrs={"axis": 0})
    add("Gather_axis1", "Gather", [f32(3, 10, 2), np.asarray([4, 2, -3], np.int64)], attrs={"axis": 1})
    add("Gather_i64_table", "Gather", [i64(9, 3, lo=-1000, hi=1000), np.asarray([8, 0, -9], np.int64)])
    add("Gather_i32_indices", "Gather", [f32(6, 5), np.asarray([[5, 1, 2]], np.int32)], attrs={"axis": 0})
    add("Shape", "Shape", [f32(2, 3, 4)])
    add("Shape_start_end", "Shape", [f32(2, 3, 4, 5)], attrs={"start": 1, "end": -1})
    add("Size", "Size", [f32(2, 3, 4)])
    add("ConstantOfShape_i64", "ConstantOfShape", [c64(2, 3)], const={0}, attrs={"value": np.asarray([7], np.int64)})
    add("ConstantOfShape_f32", "ConstantOfShape", [c64(4)], const={0}, attrs={"value": np.asarray([1.5], np.float32)})
    add("ConstantOfShape_default", "ConstantOfShape", [c64(3, 2)], const={0})
    add("Expand", "Expand", [f32(3, 1), c64(2, 3, 4)], const={1})
    add("Expand_smaller_target", "Expand", [f32(2, 3), c64(3)], const={1})
    add("Tile", "Tile", [f32(2, 3), c64(2, 2)], const={1})
    add("Tile_i64", "Tile", [i64(3), c64(3)], const={1})
    add("Range_f32", "Range", [scalar(1.0), scalar(9.0), scalar(1.5)], const={0, 1, 2})
    add("Range_i64", "Range", [scalar(10, np.int64), scalar(-3, np.int64), scalar(-4, np.int64)], const={0, 1, 2})
    add("Range_empty", "Range", [scalar(5.0), scalar(1.0), scalar(1.0)], const={0, 1, 2})
    add("Trilu_upper", "Trilu", [f32(4, 5)])
    add("Trilu_lower_k", "Trilu", [f32(2, 4, 5), scalar(1, np.int64)], const={1}, attrs={"upper": 0})
    add("Trilu_upper_negk", "Trilu", [f32(5, 4), scalar(-1, np.int64)], const={1})
    add("Pad_value", "Pad", [f32(2, 3), c64(1, 0, 2, 3), scalar(1.5)], const={1, 2})
    add("Pad_zero", "Pad", [f32(2, 3, 2), c64(0, 1, 0, 1, 0, 2)], const={1})
    add("Pad_axes", "Pad", [f32(2, 3, 2), c64(1, 2), None, c64(-1)], const={1, 3})
    # reductions and normalization
    for op in ("ReduceMean", "ReduceSum", "ReduceMax", "ReduceMin", "ReduceProd"):
        src = pos(2, 3, 4) if op == "ReduceProd" else f32(2, 3, 4)
        add(f"{op}_axes_keep", op, [src], attrs={"axes": [1, 2], "keepdims": 1})
        add(f"{op}_axis_drop", op, [src], attrs={"axes": [-1], "keepdims": 0})
        add(f"{op}_all", op, [src])
        add(f"{op}_axes_input", op, [src, c64(0)], const={1}, attrs={"keepdims": 0})
    add("ReduceSum_i64", "ReduceSum", [i64(3, 4)], attrs={"axes": [0]})
    add("ReduceMax_i64", "ReduceMax", [i64(3, 4)], attrs={"axes": [1], "keepdims": 0})
    add("ReduceSum_noop", "ReduceSum", [f32(2, 3)], attrs={"noop_with_empty_axes": 1})
    ties = np.asarray([[1, 3, 3, 0], [2, 2, 1, 2], [0, 0, 0, 0]], np.float32)
    add("ArgMax_ties_first", "ArgMax", [ties], attrs={"axis": 1, "keepdims": 0})
    add("ArgMax_keep", "ArgMax", [f32(3, 7)], attrs={"axis": 0})
    add("ArgMax_i64", "ArgMax", [i64(4, 6)], attrs={"axis": -1, "keepdims": 1})
    add("Softmax_last", "Softmax", [f32(2, 3, 9, scale=3.0)], attrs={"axis": -1})
    add("Softmax_mid", "Softmax", [f32(2, 7, 3, scale=3.0)], attrs={"axis": 1})
    add("Softmax_default", "Softmax", [f32(4, 6)])
    add("LogSoftmax_last", "LogSoftmax", [f32(4, 9, scale=3.0)], attrs={"axis": -1})
    add("LogSoftmax_first", "LogSoftmax", [f32(5, 3, scale=3.0)], attrs={"axis": 0})
    add("LayerNorm_last", "LayerNormalization", [f32(2, 5, 16), pos(16), f32(16)], const={1, 2},
        attrs={"axis": -1, "epsilon": 1e-5})
    add("LayerNorm_axis1", "LayerNormalization", [f32(2, 3, 4), pos(3, 4)], const={1}, attrs={"axis": 1})
    add("LayerNorm_eps", "LayerNormalization", [f32(3, 8, scale=1e-3), pos(8), f32(8)], const={1, 2},
        attrs={"epsilon": 1e-12})
    add("BatchNorm", "BatchNormalization", [f32(2, 3, 4, 5), pos(3), f32(3), f32(3), pos(3)], const={1, 2, 3, 4})
    add("BatchNorm_eps", "BatchNormalization", [f32(1, 2, 3, 3), pos(2), f32(2), f32(2), pos(2)], const={1, 2, 3, 4},
        attrs={"epsilon": 0.1})
    # contractions
    add("MatMul_2d", "MatMul", [f32(5, 7), f32(7, 3)])
    add("MatMul_batched_bcast", "MatMul", [f32(2, 1, 5, 7), f32(3, 7, 4)])
    add("MatMul_vec_left", "MatMul", [f32(7), f32(7, 5)])
    add("MatMul_vec_right", "MatMul", [f32(4, 7), f32(7)])
    add("MatMul_i64", "MatMul", [i64(3, 4), i64(4, 2)])
    add("Gemm_plain", "Gemm", [f32(4, 5), f32(5, 3)], const={1})
    add("Gemm_transA_bias", "Gemm", [f32(5, 4), f32(5, 3), f32(3)], const={1, 2}, attrs={"transA": 1})
    add("Gemm_transB_alpha_beta", "Gemm", [f32(4, 5), f32(3, 5), f32(1, 3)], const={1, 2},
        attrs={"transB": 1, "alpha": 0.5, "beta": 2.0})
    add("Gemm_full_c", "Gemm", [f32(4, 5), f32(5, 3), f32(4, 3)], const={1, 2}, attrs={"beta": 0.5})
    add("Gemm_column_c", "Gemm", [f32(4, 5), f32(5, 3), f32(4, 1)], const={1, 2})
    add("Gemm_scalar_c", "Gemm", [f32(4, 5), f32(5, 3), f32()], const={1, 2})
    for act in ("none", "relu", "clip", "gelu", "gelu_tanh", "tanh", "sigmoid"):
        add(f"FusedGemm_{act}", "FusedGemm", [f32(2, 3, 4), f32(4, 5), f32(5), f32(2, 3, 5)], const={1, 2},
            attrs={"activation": act, "clip_min": -0.5, "clip_max": 0.5})
    add("FusedGemm_trans_b", "FusedGemm", [f32(3, 4), f32(5, 4), f32(5)], const={1, 2},
        attrs={"activation": "relu", "trans_b": 1})
    conv_cases = [
        ("pad1", {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1]}, (1, 4, 9, 8), (6, 4, 3, 3)),
        ("stride2_asym", {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 0, 1, 2]}, (2, 3, 11, 9), (5, 3, 3, 3)),
        ("dilated", {"kernel_shape": [2, 3], "dilations": [2, 1]}, (1, 2, 9, 9), (4, 2, 2, 3)),
        ("group2", {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 2}, (1, 4, 6, 6), (6, 2, 3, 3)),
        ("depthwise", {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 4}, (1, 4, 7, 7), (4, 1, 3, 3)),
        ("same_upper", {"auto_pad": "SAME_UPPER", "strides": [2, 2]}, (1, 3, 8, 8), (4, 3, 3, 3)),
        ("valid", {"auto_pad": "VALID"}, (1, 2, 6, 5), (3, 2, 2, 2)),
        ("pointwise", {"kernel_shape": [1, 1]}, (1, 16, 5, 5), (24, 16, 1, 1)),
    ]
    for name, attrs, xs, ws in conv_cases:
        add(f"Conv_{name}", "Conv", [f32(*xs), f32(*ws, scale=0.3), f32(ws[0])], const={1, 2}, attrs=attrs)
    add("Conv_no_bias", "Conv", [f32(1, 3, 6, 6), f32(4, 3, 3, 3, scale=0.3)], const={1}, attrs={"pads": [1, 1, 1, 1]})
    for act in ("relu", "clip", "sigmoid"):
        add(f"FusedConv_nchw_{act}", "FusedConv", [f32(1, 3, 7, 7), f32(4, 3, 3, 3, scale=0.3), f32(4), f32(1, 4, 7, 7)],
            const={1, 2}, attrs={"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "activation": act, "clip_min": 0.0,
                                 "clip_max": 0.5})
    add("FusedConv_nhwc", "FusedConv", [f32(2, 7, 6, 3), f32(3, 3, 3, 5, scale=0.3), f32(5)], const={1, 2},
        attrs={"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "strides": [2, 1], "layout": "NHWC", "activation": "relu"})
    add("FusedConv_nhwc_depthwise", "FusedConv", [f32(1, 6, 6, 4), f32(3, 3, 1, 4, scale=0.3), f32(4), f32(1, 6, 6, 4)],
        const={1, 2}, attrs={"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "group": 4, "layout": "NHWC",
                             "activation": "clip", "clip_min": 0.0, "clip_max": 6.0})
    pool_cases = [
        ("s2_pad", {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]}),
        ("2x2", {"kernel_shape": [2, 2], "strides": [2, 2]}),
        ("ceil", {"kernel_shape": [3, 3], "strides": [2, 2], "ceil_mode": 1}),
        ("dilated", {"kernel_shape": [2, 2], "dilations": [2, 2]}),
        ("same_lower", {"kernel_shape": [3, 3], "auto_pad": "SAME_LOWER", "strides": [2, 2]}),
    ]
    for name, attrs in pool_cases:
        add(f"MaxPool_{name}", "MaxPool", [f32(2, 3, 9, 10)], attrs=attrs)
        add(f"AveragePool_{name}", "AveragePool", [f32(2, 3, 9, 10)], attrs=attrs)
    add("AveragePool_count_pad", "AveragePool", [f32(1, 2, 7, 6)],
        attrs={"kernel_shape": [3, 3], "pads": [1, 1, 1, 1], "count_include_pad": 1})
    add("AveragePool_ceil_pad", "AveragePool", [f32(1, 2, 9, 9)],
        attrs={"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1], "ceil_mode": 1})
    add("MaxPool_nhwc", "MaxPool", [f32(2, 9, 10, 3)],
        attrs={"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1], "layout": "NHWC"})
    for op in ("GlobalAveragePool", "GlobalMaxPool"):
        add(f"{op}_nchw", op, [f32(2, 5, 4, 3)])
        add(f"{op}_nhwc", op, [f32(2, 4, 3, 5)], attrs={"layout": "NHWC"})
    # FusedElementwise programs (passes/loopfuse.py:30-94): leaves, then instructions that
    # reference earlier leaves/results by index
    add("FusedElementwise_chain", "FusedElementwise", [f32(3, 4), f32(4), scalar(0.125)],
        attrs={"program": [["Add", {}, [0, 1]], ["Mul", {}, [3, 2]], ["Tanh", {}, [4]]]})
    add("FusedElementwise_clip_gelu", "FusedElementwise", [f32(2, 5, scale=3.0)],
        attrs={"program": [["Gelu", {"approximate": "tanh"}, [0]], ["Clip", {"min": -0.5, "max": 1.0}, [1]]]})
    return out


def _reference_ops():
    sys.path.insert(0, str(REFERENCE_SRC))
    import ml_graph_compiler  # the reference package

    if not str(Path(ml_graph_compiler.__file__)).startswith(str(REFERENCE_SRC)):
        raise SystemExit("imported the wrong ml_graph_compiler")
    from ml_graph_compiler import ops
    from ml_graph_compiler.ir import Node

    return ops, Node


def _jsonable(attrs):
    out = {}
    for k, v in attrs.items():
        if isinstance(v, np.ndarray):
            out[k] = {"__array__": v.tolist(), "dtype": str(v.dtype)}
        else:
            out[k] = v
    return out


def main() -> None:
    ops, Node = _reference_ops()
    arrays, manifest = {}, []
    for name, op, inputs, const, attrs, n_out in cases():
        node = Node(op, [None] * len(inputs), [None] * n_out, attrs, name=name)
        results = ops.run(node, [None if a is None else a.copy() for a in inputs])
        assert len(results) == n_out, (name, len(results))
        for i, a in enumerate(inputs):
            if a is not None:
                arrays[f"{name}/in{i}"] = a
        for j, r in enumerate(results):
            arrays[f"{name}/out{j}"] = np.asarray(r)
        manifest.append({"name": name, "op": op, "inputs": [a is not None for a in inputs], "const": const,
                         "attrs": _jsonable(attrs), "outputs": n_out})
        print(name, [np.asarray(r).dtype.name + str(list(np.shape(r))) for r in results], flush=True)
    np.savez_compressed(HERE / "reference_ops.npz", **arrays)
    (HERE / "reference_ops.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print(f"{len(manifest)} cases", flush=True)


if __name__ == "__main__":
    main()
