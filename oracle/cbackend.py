"""CPU baseline and second oracle: the reference's generated-C + OpenMP backend.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
may use this module. The compiler never imports it.

The compute kernels are the reference's own C (codegen/runtime/mgc_kernels.c), compiled from
/root/reference by oracle/Makefile into oracle/_ref/mgc_kernels.o. This module restates the part
of the reference's emitter (codegen/c.py) that the benchmark graphs need at -O3 and emits one
``mgc_run`` C function per model, calling those kernels with the same arguments the reference
would pass:

* FusedConv NHWC -> mgc_gemm with an MGC_CONV_NHWC A operand (pointwise: strided A) and
  12-wide packed B panels, batch offsets per image (c.py:1102-1226); depthwise ->
  mgc_depthwise_nhwc (c.py:1126-1136)
* FusedGemm / MatMul -> mgc_gemm, packed constant B, batched offsets (c.py:906-1086)
* MaxPool / AveragePool NHWC -> mgc_pool_nhwc; GlobalAveragePool -> mgc_reduce_mid (c.py:1228-1273)
* Softmax -> mgc_softmax, LayerNormalization -> mgc_layer_norm (c.py:823-869)
* elementwise and FusedElementwise (float32), Transpose, Split, Concat -> loop nests
  (c.py:360-529, 558-660); Gather -> row memcpy with the out-of-range check (c.py:662-688)
* views emit nothing; output copies are memcpy (c.py:1283-1285)

Memory planning is the product's planner at the reference's C-backend alignment (64). Per-model
libraries are built in this container (the reference header is only here); bench.py on the GPU
box loads the prebuilt libraries from oracle/_ref/ and regenerates the weights blob, whose
digest must match the one recorded at build time.
"""

from __future__ import annotations

import ctypes
import hashlib
import json
import math
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
REF_OUT = ORACLE_DIR / "_ref"
REF_RUNTIME = Path("/root/reference/src/ml_graph_compiler/codegen/runtime")
sys.path.insert(0, str(ORACLE_DIR.parent / "ml-graph-compiler_amd"))

from ml_graph_compiler import ops  # noqa: E402
from ml_graph_compiler.ir import Graph, Value  # noqa: E402
from ml_graph_compiler.memory import ALIAS_OPS, plan_memory  # noqa: E402

MR, NR, ALIGN = 8, 12, 64
CTYPES = {"float32": "float", "float64": "double", "int64": "int64_t", "int32": "int32_t",
          "int8": "int8_t", "uint8": "uint8_t", "bool": "uint8_t"}
ACT = {"none": "MGC_ACT_NONE", "relu": "MGC_ACT_RELU", "clip": "MGC_ACT_CLIP", "gelu": "MGC_ACT_GELU",
       "gelu_tanh": "MGC_ACT_GELU_TANH", "tanh": "MGC_ACT_TANH", "sigmoid": "MGC_ACT_SIGMOID"}
EXPR = {"Add": "({0} + {1})", "Sub": "({0} - {1})", "Mul": "({0} * {1})", "Div": "({0} / {1})",
        "Max": "fmaxf({0}, {1})", "Min": "fminf({0}, {1})", "Relu": "({0} > 0.0f ? {0} : 0.0f)",
        "Sigmoid": "mgc_sigmoidf({0})", "Tanh": "mgc_tanhf({0})", "Erf": "mgc_erff({0})",
        "Sqrt": "sqrtf({0})", "Exp": "mgc_expf({0})", "Neg": "(-{0})", "Identity": "{0}",
        "Pow": "powf({0}, {1})", "Abs": "fabsf({0})", "Reciprocal": "(1.0f / {0})"}

# workload -> the batches a library is prebuilt for: batch 1 and the GPU batch of each BASELINE
# config (the single GEMM is one call of 128 rows)
BASELINES = {"resnet50": (1, 32), "bottleneck": (1, 32), "mobilenet_v2": (1, 32), "bert_base": (1, 16),
             "gpt2": (1, 8), "single_gemm": (1,)}


class CBackendError(Exception):
    pass


def _lit(v: float) -> str:
    v = float(v)
    if math.isinf(v):
        return "INFINITY" if v > 0 else "(-INFINITY)"
    return f"{float(np.float32(v))!r}f"


def _strides(shape):
    out = [1] * len(shape)
    for i in range(len(shape) - 2, -1, -1):
        out[i] = out[i + 1] * int(shape[i + 1])
    return out


def _bstrides(shape, out_shape):
    src = _strides(shape)
    pad = len(out_shape) - len(shape)
    return [0 if d < pad or shape[d - pad] == 1 else src[d - pad] for d in range(len(out_shape))]


def pack_b_panels(b: np.ndarray) -> np.ndarray:
    """K x N -> [ceil(N/12), K, 12] zero-padded panels (codegen/c.py:222-233)."""
    b = np.asarray(b, np.float32)
    k, n = b.shape
    panels = -(-n // NR)
    out = np.zeros((panels, k, NR), np.float32)
    for p in range(panels):
        cols = b[:, p * NR : min(n, (p + 1) * NR)]
        out[p, :, : cols.shape[1]] = cols
    return out


class Blob:
    """Constants at 64-byte aligned offsets, deduplicated by key (codegen/c.py:166-219)."""

    def __init__(self) -> None:
        self.chunks: list[tuple[int, np.ndarray]] = []
        self.size = 0
        self.keys: dict = {}

    def add(self, array, key=None) -> int:
        if key is not None and key in self.keys:
            return self.keys[key]
        data = np.ascontiguousarray(array)
        off = self.size
        self.chunks.append((off, data))
        self.size = off + data.nbytes
        self.size += (-self.size) % ALIGN
        if key is not None:
            self.keys[key] = off
        return off

    @property
    def nbytes(self) -> int:
        return max(self.size, ALIGN)

    def bytes(self) -> np.ndarray:
        out = np.zeros(self.nbytes, np.uint8)
        for off, data in self.chunks:
            out[off : off + data.nbytes] = data.reshape(-1).view(np.uint8)
        return out


class CEmitter:
    """Restated C emitter for the operators of the benchmark graphs at -O3."""

    def __init__(self, graph: Graph) -> None:
        self.g = graph
        self.plan = plan_memory(graph, alignment=ALIGN)
        self.blob = Blob()
        self.body: list[str] = []
        self.statics: list[str] = []
        self.n = 0
        self._alive: list = []

    def fresh(self, hint: str) -> str:
        self.n += 1
        return f"{hint}{self.n}"

    def _root(self, v: Value) -> Value:
        while v.data is None and v.producer is not None and v.producer.op in ALIAS_OPS:
            v = v.producer.input(0)
        return v

    def ptr(self, v: Value, ct: str | None = None) -> str:
        ct = ct or CTYPES[v.tensor_type.dtype]
        loc = self.plan.location(v)
        if loc.kind == "const":
            root = self._root(v)
            return f"((const {ct} *)(W + {self.blob.add(root.data, ('raw', id(root)))}))"
        if loc.kind == "input":
            return f"(({ct} *)inputs[{loc.index}])"
        if loc.kind == "output":
            return f"(({ct} *)outputs[{loc.index}])"
        return f"(({ct} *)(A + {loc.index}))"

    def emit(self, s: str) -> None:
        self.body.append(s)

    # -- loop nests ----------------------------------------------------------------------------
    def loops(self, shape, strides_list, body: list[str]) -> None:
        dims = [int(d) for d in shape]
        keep = [i for i, d in enumerate(dims) if d != 1]
        dims = [dims[i] for i in keep]
        sts = [[s[i] for i in keep] for s in strides_list]
        d = len(dims) - 1
        while d > 0:
            if all(s[d - 1] == s[d] * dims[d] for s in sts):
                dims[d - 1] *= dims[d]
                del dims[d]
                for s in sts:
                    s[d - 1] = s[d]
                    del s[d]
            d -= 1
        total = int(np.prod(dims)) if dims else 1
        if total == 0:
            return
        names = [f"j{k}" for k in range(len(dims))]

        def idx(k: int) -> str:
            terms = [f"{n} * {s}L" if s != 1 else n for n, s in zip(names, sts[k]) if s]
            return " + ".join(terms) or "0"

        self.emit("{")
        for k, (nm, ext) in enumerate(zip(names, dims)):
            if k == 0 and total >= 65536 and (len(dims) > 1 or ext >= 65536):
                self.emit("#pragma omp parallel for schedule(static)")
            self.emit(f"for (long {nm} = 0; {nm} < {ext}L; {nm}++) {{")
        subs = {f"i{k}": idx(k) for k in range(len(sts))}
        for line in body:
            self.emit("  " + line.format(**subs))
        for _ in dims:
            self.emit("}")
        self.emit("}")

    def copy(self, shape, out_ptr, out_st, out_base, in_ptr, in_st, in_base) -> None:
        ob = f"{out_base} + " if out_base else ""
        ib = f"{in_base} + " if in_base else ""
        self.loops(shape, [out_st, in_st], [f"{out_ptr}[{ob}{{i0}}] = {in_ptr}[{ib}{{i1}}];"])

    # -- operators -----------------------------------------------------------------------------
    def node(self, node) -> None:
        if node.op in ALIAS_OPS:
            return
        if node.op == "FusedElementwise" or ops.is_elementwise(node.op):
            self.elementwise(node)
            return
        fn = getattr(self, f"op_{node.op}", None)
        if fn is None:
            raise CBackendError(f"C baseline emitter has no lowering for {node.op}")
        fn(node)

    def elementwise(self, node) -> None:
        if node.op == "FusedElementwise":
            program = [(str(o), dict(a), [int(x) for x in args]) for o, a, args in node.attrs["program"]]
        else:
            program = [(node.op, dict(node.attrs), [i if v is not None else -1 for i, v in enumerate(node.inputs)])]
        out = node.output
        shape = out.tensor_type.shape
        if out.tensor_type.dtype != "float32":
            raise CBackendError("C baseline emitter: float32 elementwise only")
        leaves = list(node.inputs)
        exprs, strides = [], [_strides(shape)]
        for v in leaves:
            if v is None:
                exprs.append("")
            elif v.data is not None and v.data.size == 1:
                exprs.append(_lit(v.data.reshape(()).item()))
            else:
                exprs.append(f"{self.ptr(v)}[{{i{len(strides)}}}]")
                strides.append(_bstrides(v.tensor_type.shape, shape))
        temps, lines = [], []
        for k, (op, attrs, args) in enumerate(program):
            a = [exprs[x] if x < len(leaves) else temps[x - len(leaves)] for x in args if x >= 0]
            if op == "Clip":
                lo = a[1] if len(a) > 1 else _lit(attrs.get("min", -np.inf))
                hi = a[2] if len(a) > 2 else _lit(attrs.get("max", np.inf))
                e = f"fminf(fmaxf({a[0]}, {lo}), {hi})"
            elif op == "Gelu":
                e = f"{'mgc_gelu_tanhf' if attrs.get('approximate') == 'tanh' else 'mgc_gelu_erff'}({a[0]})"
            elif op == "Where":  # a bool condition leaf (uint8_t), float branches (c.py:419-420)
                e = f"({a[0]} ? {a[1]} : {a[2]})"
            elif op in EXPR:
                e = EXPR[op].format(*a)
            else:
                raise CBackendError(f"C baseline emitter: elementwise {op}")
            lines.append(f"float v{k} = {e};")
            temps.append(f"v{k}")
        lines.append(f"{self.ptr(out)}[{{i0}}] = {temps[-1]};")
        self.loops(shape, strides, lines)

    def op_Transpose(self, node) -> None:
        x = node.input(0)
        perm = ops.transpose_perm(node, x.tensor_type.rank)
        src = _strides(x.tensor_type.shape)
        shape = node.output.tensor_type.shape
        self.copy(shape, self.ptr(node.output), _strides(shape), 0, self.ptr(x), [src[p] for p in perm], 0)

    def op_Split(self, node) -> None:
        x = node.input(0)
        xt = x.tensor_type
        axis = int(node.attrs.get("axis", 0))
        axis = axis + xt.rank if axis < 0 else axis
        src = _strides(xt.shape)
        off = 0
        for o in node.outputs:
            t = o.tensor_type
            if o.users or o in self.g.outputs:
                self.copy(t.shape, self.ptr(o), _strides(t.shape), 0, self.ptr(x), src, off * src[axis])
            off += t.shape[axis]

    def op_Concat(self, node) -> None:
        ot = node.output.tensor_type
        axis = int(node.attrs.get("axis", 0))
        axis = axis + ot.rank if axis < 0 else axis
        ost = _strides(ot.shape)
        off = 0
        for v in node.inputs:
            if v is None:
                continue
            t = v.tensor_type
            self.copy(t.shape, self.ptr(node.output), ost, off * ost[axis], self.ptr(v), _strides(t.shape), 0)
            off += t.shape[axis]

    def op_Gather(self, node) -> None:
        x, idx = node.input(0), node.input(1)
        xt, it = x.tensor_type, idx.tensor_type
        axis = int(node.attrs.get("axis", 0))
        axis = axis + xt.rank if axis < 0 else axis
        outer = int(np.prod(xt.shape[:axis])) if axis else 1
        dim = xt.shape[axis]
        inner = int(np.prod(xt.shape[axis + 1 :])) if axis + 1 < xt.rank else 1
        ct, ict = CTYPES[xt.dtype], CTYPES[it.dtype]
        self.emit("{")
        self.emit(f"const {ict} *ix = {self.ptr(idx)}; const {ct} *src = {self.ptr(x)}; {ct} *dst = {self.ptr(node.output)};")
        self.emit(f"for (long t = 0; t < {it.size}L; t++) {{")
        self.emit(f"  long k = (long)ix[t]; if (k < 0) k += {dim}L; if (k < 0 || k >= {dim}L) return 1;")
        self.emit(f"  for (long o = 0; o < {outer}L; o++) memcpy(dst + (o * {it.size}L + t) * {inner}L, "
                  f"src + (o * {dim}L + k) * {inner}L, {inner * xt.itemsize});")
        self.emit("}")
        self.emit("}")

    def op_Softmax(self, node) -> None:
        x = node.input(0)
        xt = x.tensor_type
        axis = int(node.attrs.get("axis", -1))
        axis = axis + xt.rank if axis < 0 else axis
        outer = int(np.prod(xt.shape[:axis])) if axis else 1
        inner = int(np.prod(xt.shape[axis + 1 :])) if axis + 1 < xt.rank else 1
        self.emit(f"mgc_softmax({outer}L, {xt.shape[axis]}L, {inner}L, {self.ptr(x)}, {self.ptr(node.output)}, 0);")

    def op_LayerNormalization(self, node) -> None:
        x = node.input(0)
        xt = x.tensor_type
        axis = int(node.attrs.get("axis", -1))
        axis = axis + xt.rank if axis < 0 else axis
        cols = int(np.prod(xt.shape[axis:]))
        s, b = node.optional_input(1), node.optional_input(2)
        self.emit(f"mgc_layer_norm({xt.size // cols}L, {cols}L, {self.ptr(x)}, "
                  f"{self.ptr(s, 'float') if s is not None else 'NULL'}, {self.ptr(b, 'float') if b is not None else 'NULL'}, "
                  f"{_lit(float(node.attrs.get('epsilon', 1e-5)))}, {self.ptr(node.output)});")

    def op_MaxPool(self, node, is_max: int = 1) -> None:
        x = node.input(0)
        if ops.conv_layout(node) != "NHWC":
            raise CBackendError("C baseline emitter: NHWC pooling only")
        nb, h, w, c = x.tensor_type.shape
        k = [int(v) for v in node.attrs["kernel_shape"]]
        g = ops.window_geometry(node, (h, w), (k[0], k[1]), bool(node.attrs.get("ceil_mode", 0)))
        pt, pl, pb, pr = g.pads
        self.emit(f"mgc_pool_nhwc({is_max}, {nb}, {h}, {w}, {c}, {k[0]}, {k[1]}, {g.strides[0]}, {g.strides[1]}, "
                  f"{g.dilations[0]}, {g.dilations[1]}, {pt}, {pl}, {pb}, {pr}, {g.out_hw[0]}, {g.out_hw[1]}, "
                  f"{int(node.attrs.get('count_include_pad', 0))}, {self.ptr(x)}, {self.ptr(node.output)});")

    def op_AveragePool(self, node) -> None:
        self.op_MaxPool(node, 0)

    def op_GlobalAveragePool(self, node) -> None:
        x = node.input(0)
        xt = x.tensor_type
        if ops.conv_layout(node) == "NHWC":
            outer, n, inner = xt.shape[0], int(np.prod(xt.shape[1:-1])), xt.shape[-1]
        else:
            outer, n, inner = xt.shape[0] * xt.shape[1], int(np.prod(xt.shape[2:])), 1
        self.emit(f"mgc_reduce_mid(0, {outer}L, {n}L, {inner}L, {self.ptr(x)}, {self.ptr(node.output)});")

    def _gemm(self, m, n, k, a_spec, b_spec, c, ldc, batch=1, offs=("NULL",) * 4, bias="NULL", bias_mode=0,
              res="NULL", ldr=0, act="none", lo=0.0, hi=6.0) -> None:
        self.emit("{ mgc_gemm_args g; memset(&g, 0, sizeof g);")
        self.emit(f"g.M = {m}; g.N = {n}; g.K = {k}; {a_spec} {b_spec}")
        self.emit(f"g.c = {c}; g.ldc = {ldc}L; g.ep.alpha = 1.0f; g.ep.beta = 1.0f;")
        self.emit(f"g.ep.bias = {bias}; g.ep.bias_mode = {bias_mode}; g.ep.res = {res}; g.ep.ldr = {ldr}L;")
        self.emit(f"g.ep.act = {ACT[act]}; g.ep.lo = {_lit(lo)}; g.ep.hi = {_lit(hi)};")
        self.emit(f"mgc_gemm(&g, {batch}, {offs[0]}, {offs[1]}, {offs[2]}, {offs[3]}); }}")

    def _offsets(self, values) -> str:
        if not any(values):
            return "NULL"
        name = self.fresh("off")
        self.statics.append(f"static const long {name}[{len(values)}] = {{{', '.join(map(str, values))}}};")
        return name

    def _packed(self, mat, key) -> str:
        off = self.blob.add(pack_b_panels(mat), key)
        return f"g.b.kind = MGC_PACKED; g.b.p = (const float *)(W + {off});"

    @staticmethod
    def _strided(f, p, rs, cs) -> str:
        return f"g.{f}.kind = MGC_STRIDED; g.{f}.p = {p}; g.{f}.rs = {rs}L; g.{f}.cs = {cs}L;"

    def _act(self, node):
        return (str(node.attrs.get("activation", "none")), float(node.attrs.get("clip_min", 0.0)),
                float(node.attrs.get("clip_max", 6.0)))

    def op_FusedGemm(self, node) -> None:
        a, b = node.input(0), node.input(1)
        trans = int(node.attrs.get("trans_b", 0))
        bt = b.tensor_type
        k, n = (bt.shape[1], bt.shape[0]) if trans else bt.shape
        m = a.tensor_type.size // max(k, 1)
        if b.data is None:
            raise CBackendError("C baseline emitter: constant FusedGemm weights only")
        bspec = self._packed(b.data.T if trans else b.data, ("packed", id(b), trans))
        bias, res = node.optional_input(2), node.optional_input(3)
        act, lo, hi = self._act(node)
        self._gemm(m, n, k, self._strided("a", self.ptr(a), k, 1), bspec, self.ptr(node.output), n,
                   bias=self.ptr(bias, "float") if bias is not None else "NULL", bias_mode=1 if bias is not None else 0,
                   res=self.ptr(res) if res is not None else "NULL", ldr=n, act=act, lo=lo, hi=hi)

    def op_MatMul(self, node) -> None:
        a, b = node.input(0), node.input(1)
        at, bt = a.tensor_type, b.tensor_type
        ash = (1, *at.shape) if at.rank == 1 else at.shape
        bsh = (*bt.shape, 1) if bt.rank == 1 else bt.shape
        m, k, n = ash[-2], ash[-1], bsh[-1]
        batch_shape = tuple(int(d) for d in np.broadcast_shapes(ash[:-2], bsh[:-2]))
        a_bs, b_bs = _bstrides(ash[:-2], batch_shape), _bstrides(bsh[:-2], batch_shape)
        ao, bo, co = [], [], []
        for idx in (np.ndindex(*batch_shape) if batch_shape else [()]):
            ao.append(sum(i * s for i, s in zip(idx, a_bs)) * m * k)
            bo.append(sum(i * s for i, s in zip(idx, b_bs)) * k * n)
            co.append(len(co) * m * n)
        if b.data is not None and not any(bo):
            bspec = self._packed(b.data.reshape(k, n), ("packed", id(b), 0))
        else:
            bspec = self._strided("b", self.ptr(b), n, 1)
        self._gemm(m, n, k, self._strided("a", self.ptr(a), k, 1), bspec, self.ptr(node.output), n, batch=len(co),
                   offs=(self._offsets(ao), self._offsets(bo), self._offsets(co), "NULL"))

    def op_FusedConv(self, node) -> None:
        x, w = node.input(0), node.input(1)
        if ops.conv_layout(node) != "NHWC":
            raise CBackendError("C baseline emitter: NHWC convolution only (compile at -O3)")
        nb, h, wd, c = x.tensor_type.shape
        kh, kw, cg, kout = w.tensor_type.shape
        group = int(node.attrs.get("group", 1))
        g = ops.window_geometry(node, (h, wd), (kh, kw))
        oh, ow = g.out_hw
        pt, pl = g.pads[0], g.pads[1]
        bias_v, res_v = node.optional_input(2), node.optional_input(3)
        act, lo, hi = self._act(node)
        bias = self.ptr(bias_v, "float") if bias_v is not None else "NULL"
        res = self.ptr(res_v) if res_v is not None else "NULL"
        if group > 1 and cg == 1 and kout == group:
            self.emit(f"mgc_depthwise_nhwc({nb}, {h}, {wd}, {c}, {kh}, {kw}, {g.strides[0]}, {g.strides[1]}, "
                      f"{g.dilations[0]}, {g.dilations[1]}, {pt}, {pl}, {oh}, {ow}, {self.ptr(x)}, {self.ptr(w)}, "
                      f"{bias}, {res}, {ACT[act]}, {_lit(lo)}, {_lit(hi)}, {self.ptr(node.output)});")
            return
        kg = kout // group
        in_offs = self._offsets([i * h * wd * c for i in range(nb)])
        out_offs = self._offsets([i * oh * ow * kout for i in range(nb)])
        for gi in range(group):
            wmat = w.data[:, :, :, gi * kg : (gi + 1) * kg].reshape(kh * kw * cg, kg)
            bspec = self._packed(wmat, ("conv", id(w), gi))
            if kh == kw == 1 and g.strides == (1, 1) and g.pads == (0, 0, 0, 0):
                aspec = self._strided("a", f"({self.ptr(x)} + {gi * cg})", c, 1)
            else:
                aspec = (f"g.a.kind = MGC_CONV_NHWC; g.a.p = {self.ptr(x)}; g.a.H = {h}; g.a.W = {wd}; g.a.C = {c}; "
                         f"g.a.KH = {kh}; g.a.KW = {kw}; g.a.SH = {g.strides[0]}; g.a.SW = {g.strides[1]}; "
                         f"g.a.DH = {g.dilations[0]}; g.a.DW = {g.dilations[1]}; g.a.PT = {pt}; g.a.PL = {pl}; "
                         f"g.a.OW = {ow}; g.a.c_off = {gi * cg}; g.a.cg = {cg};")
            self._gemm(oh * ow, kg, kh * kw * cg, aspec, bspec, f"({self.ptr(node.output)} + {gi * kg})", kout,
                       batch=nb, offs=(in_offs, "NULL", out_offs, out_offs if res != "NULL" else "NULL"),
                       bias=f"({bias} + {gi * kg})" if bias != "NULL" else "NULL",
                       bias_mode=1 if bias != "NULL" else 0,
                       res=f"({res} + {gi * kg})" if res != "NULL" else "NULL", ldr=kout, act=act, lo=lo, hi=hi)

    def generate(self) -> str:
        for node in self.g.nodes:
            self.emit(f"/* {node.op} */")
            self.node(node)
        for value, j in self.plan.copies:
            self.emit(f"memcpy(outputs[{j}], {self.ptr(value)}, {value.tensor_type.nbytes});")
        arena = max(self.plan.arena_bytes, ALIGN)
        head = ['#include "mgc_runtime.h"', *self.statics,
                f"size_t mgc_arena_bytes(void) {{ return {arena}UL; }}",
                f"size_t mgc_weights_bytes(void) {{ return {self.blob.nbytes}UL; }}",
                "int mgc_run(const void *const *inputs, void *const *outputs, unsigned char *A, const unsigned char *W) {",
                "(void)inputs; (void)outputs; (void)A; (void)W;"]
        return "\n".join(head + self.body + ["return 0;", "}", ""])


def blob_digest(blob: np.ndarray) -> str:
    return hashlib.sha256(blob.tobytes()).hexdigest()[:24]


def build_library(source: str, out: Path) -> None:
    """Compile one generated model against the reference header and kernels (needs
    /root/reference, i.e. only in the build container)."""
    kernels = REF_OUT / "mgc_kernels.o"
    if not kernels.exists():
        subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    src = out.with_suffix(".c")
    src.write_text(source)
    cmd = ["gcc", "-O3", "-std=c11", "-fPIC", "-shared", "-ffp-contract=fast", "-fno-math-errno",
           "-march=x86-64-v3", "-fopenmp", "-I", str(REF_RUNTIME), str(src), str(kernels), "-o", str(out), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True)


class CModel:
    """ctypes wrapper of one built C-backend model (the reference's CompiledModel.run)."""

    def __init__(self, library: Path, graph: Graph, weights: np.ndarray) -> None:
        self.lib = ctypes.CDLL(str(library))
        self.lib.mgc_run.restype = ctypes.c_int
        self.lib.mgc_run.argtypes = [ctypes.c_void_p] * 4
        self.lib.mgc_arena_bytes.restype = ctypes.c_size_t
        self.lib.mgc_weights_bytes.restype = ctypes.c_size_t
        if int(self.lib.mgc_weights_bytes()) != weights.nbytes:
            raise CBackendError("weights blob does not match the library")
        raw = np.empty(weights.nbytes + 64, np.uint8)
        s = (-raw.ctypes.data) % 64
        self.weights = raw[s : s + weights.nbytes]
        self.weights[:] = weights
        n = int(self.lib.mgc_arena_bytes())
        raw = np.empty(n + 64, np.uint8)
        s = (-raw.ctypes.data) % 64
        self.arena = raw[s : s + n]
        self.graph = graph

    def run(self, feeds: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
        ins = [np.ascontiguousarray(feeds[v.name]) for v in self.graph.inputs]
        outs = {name: np.empty(v.type.shape, np.dtype(v.type.dtype)) for name, v in self.graph.named_outputs()}
        ip = (ctypes.c_void_p * max(len(ins), 1))(*[a.ctypes.data for a in ins])
        op = (ctypes.c_void_p * max(len(outs), 1))(*[a.ctypes.data for a in outs.values()])
        code = self.lib.mgc_run(ctypes.addressof(ip), ctypes.addressof(op), self.arena.ctypes.data, self.weights.ctypes.data)
        if code:
            raise CBackendError("compiled model reported an out-of-range Gather index")
        return outs


def compile_c(graph: Graph, out: Path) -> CModel:
    """Generate, build (reference header required) and load the C-backend model of an
    optimized, scheduled graph."""
    em = CEmitter(graph)
    source = em.generate()
    build_library(source, out)
    return CModel(out, graph, em.blob.bytes())


def _baseline_graph(workload: str, batch: int):
    from ml_graph_compiler import builders
    from ml_graph_compiler.passes import optimize
    from ml_graph_compiler.schedule import schedule

    g = builders.single_gemm() if workload == "single_gemm" else builders.CONFIGS[workload](batch=batch)
    optimize(g, "O3")
    schedule(g)
    return g


def baseline_path(workload: str, batch: int) -> Path:
    return REF_OUT / f"{workload}_b{batch}_cref.so"


def build_baselines(workloads=tuple(BASELINES)) -> list[Path]:
    """Prebuild the per-workload C libraries, at every batch of BASELINES, into oracle/_ref (run
    where /root/reference is)."""
    built = []
    REF_OUT.mkdir(exist_ok=True)
    for wl in workloads:
        for batch in BASELINES[wl]:
            g = _baseline_graph(wl, batch)
            em = CEmitter(g)
            source = em.generate()
            lib = baseline_path(wl, batch)
            build_library(source, lib)
            meta = {"workload": wl, "batch": batch, "weights_digest": blob_digest(em.blob.bytes())}
            lib.with_suffix(".json").write_text(json.dumps(meta))
            built.append(lib)
    return built


def load_baseline(workload: str, batch: int = 1) -> tuple[CModel, Graph, dict]:
    """A prebuilt baseline library with its O3 graph and regenerated weights. Raises
    CBackendError (never skips) when the library was not built or its weights differ."""
    lib = baseline_path(workload, batch)
    if not lib.exists() or not lib.with_suffix(".json").exists():
        raise CBackendError(f"{lib.name} is not built: run __graft_entry__.build() where /root/reference exists")
    meta = json.loads(lib.with_suffix(".json").read_text())
    g = _baseline_graph(workload, batch)
    em = CEmitter(g)
    em.generate()
    blob = em.blob.bytes()
    if blob_digest(blob) != meta["weights_digest"]:
        raise CBackendError("regenerated weights differ from the prebuilt baseline's")
    return CModel(lib, g, blob), g, meta


def load_baseline_with_weights(workload: str, batch: int, graph: Graph) -> CModel:
    """The prebuilt library of ``workload`` at ``batch`` run with the constants of ``graph``: the
    same builder graph with other constant values (for example calibrated BatchNorm
    statistics), optimized and scheduled. The C generated for ``graph`` must equal the
    baseline's (the library depends only on shapes, the weights blob holds every constant), so
    only the blob differs; raises CBackendError otherwise."""
    lib = baseline_path(workload, batch)
    if not lib.exists():
        raise CBackendError(f"{lib.name} is not built: run __graft_entry__.build() where /root/reference exists")
    base = CEmitter(_baseline_graph(workload, batch)).generate()
    em = CEmitter(graph)
    if em.generate() != base:
        raise CBackendError("the graph's generated C differs from the prebuilt baseline's")
    return CModel(lib, graph, em.blob.bytes())


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_baseline(workload: str, seconds_budget: float = 20.0, threads: int | None = None) -> dict:
    """Time the reference C backend on this host: warmup, then repeat runs until the budget is
    spent (at least 3); median seconds per run -> units/s."""
    from ml_graph_compiler.builders import random_feeds

    model, g, meta = load_baseline(workload)
    if threads:  # the reference runtime's own thread knob (mgc_kernels.c:34-70)
        model.lib.mgc_set_num_threads(int(threads))
    model.lib.mgc_get_max_threads.restype = ctypes.c_int
    n_threads = int(model.lib.mgc_get_max_threads())
    feeds = random_feeds(g, 0, int_high=30522 if workload in ("bert_base", "gpt2") else 100)
    model.run(feeds)
    times = []
    t_end = time.perf_counter() + seconds_budget
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        model.run(feeds)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    units = 1 if workload == "single_gemm" else meta["batch"]
    unit = {"single_gemm": "calls/s", "bert_base": "seq/s", "gpt2": "seq/s"}.get(workload, "img/s")
    return {
        "value": round(units / med, 3),
        "unit": unit,
        "cores": n_threads,
        "kind": "reference",
        "sample": (f"{workload} batch {meta['batch']}, {len(times)} runs (median {med * 1e3:.1f} ms) of the "
                   f"reference's generated-C backend (its mgc_kernels.c, -O3 -fopenmp -march=x86-64-v3) "
                   f"on {n_threads} OpenMP threads of '{_cpu_model()}'"),
    }
