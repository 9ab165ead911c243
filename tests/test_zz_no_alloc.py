"""mgc_hip_gemm_noalloc against mgc_hip_gemm, both through the C ABI.

mgc_hip_gemm_noalloc keeps its K-split partials in the library's own per-GPU device array
instead of a caller workspace. The existing entry point, mgc_hip_gemm, runs inside a compiled
model (the emitter's call, with the planner's workspace); the new one is called directly with
device buffers this test allocates for the operands (the caller still owns inputs and outputs).
Two calls in a row on the same GPU, the second with a smaller input, must each match the
compiled model bit for bit (same kernels, same K split) and the oracle within the single-GEMM
tolerance (1e-4 max-abs). An explicit K split that needs more than the scratch holds, and
operands outside a kernel's limits, are rejected as argument errors; an error left pending on the
thread before a call does not fail it.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from capi import MGC_ERR_ARGS, MGC_OK, MGC_OP_STRIDED, GemmArgs, Hip, Operand, bind
from ml_graph_compiler.codegen import compile_graph
from ml_graph_compiler.codegen.build import load_kernel_library
from ml_graph_compiler.ir import Graph, TensorType
from ml_graph_compiler.passes import optimize
from ml_graph_compiler.schedule import schedule
from ml_graph_compiler.shape_inference import infer_shapes
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu

MGC_ACT_RELU = 1
SCRATCH_FLOATS = 1 << 23


def _graph(m: int, n: int, k: int, seed: int):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    g = Graph("noalloc_ref")
    x = g.add_input("x", TensorType("float32", (m, k)))
    y = g.add_node("MatMul", [x, g.constant(w, "w")], 1, {}, name="mm").output
    y = g.add_node("Add", [y, g.constant(bias, "b")], 1, {}, name="bias").output
    y = g.add_node("Relu", [y], 1, {}, name="relu").output
    g.add_output(y, "y")
    infer_shapes(g)
    feeds = {"x": rng.standard_normal((m, k)).astype(np.float32)}
    return g, w, bias, feeds


def _noalloc(lib, hip: Hip, m: int, n: int, k: int, x: np.ndarray, w: np.ndarray, bias: np.ndarray,
             split_k: int = 0, k1: int = 0) -> tuple[int, np.ndarray | None]:
    args = GemmArgs()
    args.M, args.N, args.K = m, n, k
    args.a = Operand(kind=MGC_OP_STRIDED, p=hip.upload(x), rs=k, cs=1)
    # B stored [N][K] (k contiguous), the layout the emitter packs constant weights in
    args.b = Operand(kind=MGC_OP_STRIDED, p=hip.upload(np.ascontiguousarray(w.T)), rs=1, cs=k)
    c = hip.empty(m * n * 4)
    args.c, args.ldc = c, n
    args.alpha, args.beta = 1.0, 1.0
    args.bias, args.bias_mode = hip.upload(bias), 1
    args.act, args.lo, args.hi = MGC_ACT_RELU, 0.0, 6.0
    args.split_k = split_k
    args.k1 = k1
    code = lib.mgc_hip_gemm_noalloc(None, ctypes.byref(args))
    return code, (hip.download(c, (m, n)) if code == MGC_OK else None)


def test_noalloc_gemm_matches_mgc_hip_gemm(hip_cache):
    lib = load_kernel_library()
    bind(lib)
    hip = Hip()
    try:
        # two calls in a row, the second smaller; both shapes split K (the scratch holds
        # partials of the first when the second runs)
        for m, n, k, seed in ((256, 1024, 4096, 1), (64, 768, 3072, 2)):
            need = int(lib.mgc_hip_gemm_workspace(m, n, k, 1))
            print(f"[gpu] noalloc GEMM {m}x{n}x{k}: K-split scratch {need} floats", flush=True)
            assert 0 < need <= SCRATCH_FLOATS
            g, w, bias, feeds = _graph(m, n, k, seed)
            expected = oracle.run_graph(g, feeds)["y"]
            optimize(g, "O3")
            schedule(g)
            model = compile_graph(g, cache_dir=hip_cache, name=f"noalloc_ref_{m}")
            try:
                want = model.run(feeds)["y"]
            finally:
                model.release()
            code, got = _noalloc(lib, hip, m, n, k, feeds["x"], w, bias)
            assert code == MGC_OK, lib.mgc_hip_last_error()
            err = float(np.max(np.abs(got.astype(np.float64) - expected)))
            same = bool(np.array_equal(got, want))
            print(f"[gpu] noalloc {m}x{n}x{k}: max-abs vs oracle {err:.3e}, identical to mgc_hip_gemm: {same}",
                  flush=True)
            assert err <= 1e-4
            np.testing.assert_array_equal(got, want)
        # an explicit split whose partials exceed the scratch is refused, before any launch
        m, n, k = 2048, 4096, 256
        code, _ = _noalloc(lib, hip, m, n, k, np.zeros((m, k), np.float32), np.zeros((k, n), np.float32),
                           np.zeros(n, np.float32), split_k=2)
        assert code == MGC_ERR_ARGS
        assert b"more than" in lib.mgc_hip_last_error()
        # operands outside a kernel's limits are argument errors too: a concatenated-K second
        # source that is not an NHWC image
        code, _ = _noalloc(lib, hip, 64, 64, 64, np.zeros((64, 64), np.float32), np.zeros((64, 64), np.float32),
                           np.zeros(64, np.float32), k1=32)
        assert code == MGC_ERR_ARGS, lib.mgc_hip_last_error()
        assert b"concatenated-K" in lib.mgc_hip_last_error()
        # an error the caller left pending on the thread (a failed hipSetDevice) is not reported
        # by the next call, which succeeds
        assert hip.lib.hipSetDevice(1 << 20) != 0
        m, n, k = 64, 768, 3072
        g, w, bias, feeds = _graph(m, n, k, 2)
        code, got = _noalloc(lib, hip, m, n, k, feeds["x"], w, bias)
        assert code == MGC_OK, lib.mgc_hip_last_error()
        assert float(np.max(np.abs(got.astype(np.float64) - oracle.run_graph(g, feeds)["y"]))) <= 1e-4
    finally:
        hip.free()
