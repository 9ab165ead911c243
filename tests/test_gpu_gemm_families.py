"""Every GEMM kernel family, forced through mgc_hip_gemm_args.kernel, on edge shapes.

The library picks a family and K split from the shape (`choose_tiles`, `wave_split`,
`use_tile16`, `use_stream`, the quarter-tile rule), so each family normally runs only at the
shapes its rule sends it. This test drives mgc_hip_gemm directly through the C ABI
(mgc_hip_exec_create on the null stream) with the family and split pinned, as the reference's
tests pin its C kernels' blocking to reach their edge paths (tests/test_codegen.py:444-455)
and sweep GEMM shapes with a property test (:488-516):

* M, N in {1, 3, 31, 33, 63, 65, 129} (N also 4 and 68); K in {1, 2, 31, 33, 64, 65, 4097} plus the multiples of
  four {4, 8, ..., 32, 36, 68, 4096} that the k-contiguous DMA kernels (and, up to 32, the
  streaming kernel) need;
* every family: 64 x 64 DMA tiles, quarter tiles, 128 x 32 tiles, 32 x 32 and 16 x 16 wave
  splits, the short-K streaming kernel and the register-staged kernel, each family that takes a
  K split also with split 2 and 3 (empty K chunks included);
* a rotating epilogue per shape: column or row bias or none, a residual with beta, alpha != 1,
  and each of the seven activations.

Each call's output (the buffer is NaN-filled before the call, so an element the kernel skips
fails) is compared with float64 numpy plus the oracle's activations at the single-GEMM bound
(1e-4 absolute + 1e-4 relative). A family the operands do not suit (the DMA kernels need
K % 4 == 0, the streaming kernel K <= 32 (48 over an image) and relu / clip / none with a
column bias, quarter
tiles no K split) must refuse the call with MGC_ERR_ARGS, naming the family; the test
predicts which calls are refused from those documented rules and checks both ways. NHWC
implicit-GEMM convolutions (3 x 3, strides 1 and 2, ragged images) run through every family
that reads an image as well.
"""

from __future__ import annotations

import ctypes
import itertools

import numpy as np
import pytest

from capi import ACTS, GEMM_FAMILIES, MGC_ERR_ARGS, MGC_OK, MGC_OP_CONV_NHWC, MGC_OP_STRIDED, GemmArgs, Hip, Operand, bind
from ml_graph_compiler.codegen.build import load_kernel_library
from oracle import interpreter as oracle

pytestmark = pytest.mark.gpu

MN = (1, 3, 31, 33, 63, 65, 129)
K_ANY = (1, 2, 31, 33, 64, 65, 4097)
K_VEC = (4, 8, 12, 16, 20, 24, 28, 32, 36, 68, 4096)
N_VEC = (4, 68)  # column counts the streaming kernel takes (N % 4 == 0)
SPLIT_FAMILIES = ("tiled", "narrow", "wsplit", "wsplit16", "register")
FAMILIES = ("tiled", "quarter", "narrow", "wsplit", "wsplit16", "stream", "register")
LO, HI = -0.5, 0.75


def _epilogue(i: int) -> dict:
    """The i-th epilogue of the rotation: activation, bias mode, residual, alpha."""
    return {"act": ACTS[i % 7], "bias_mode": (0, 1, 2)[(i // 7) % 3], "residual": (i // 3) % 2 == 1,
            "alpha": 1.0 if i % 5 else 0.5, "beta": 1.0 if i % 4 else -0.75}


def _expected(a64: np.ndarray, b64: np.ndarray, ep: dict, bias, res) -> np.ndarray:
    y = ep["alpha"] * (a64 @ b64)
    if ep["bias_mode"] == 1:
        y = y + bias.astype(np.float64)[None, :]
    elif ep["bias_mode"] == 2:
        y = y + bias.astype(np.float64)[:, None]
    if ep["residual"]:
        y = y + ep["beta"] * res.astype(np.float64)
    return oracle.activation(y, {"activation": ep["act"], "clip_min": LO, "clip_max": HI})


class Runner:
    """mgc_hip_gemm on an exec context over the null stream, with device buffers reused
    across calls (sized for the largest operand)."""

    def __init__(self) -> None:
        self.lib = load_kernel_library()
        bind(self.lib)
        self.hip = Hip()
        self.x = self.lib.mgc_hip_exec_create(None)
        assert self.x, self.lib.mgc_hip_last_error()
        cap = 129 * 4097 + 64
        self.a, self.b = self.hip.alloc(4 * cap), self.hip.alloc(4 * cap)
        self.c, self.r = self.hip.alloc(4 * 129 * 129), self.hip.alloc(4 * 129 * 129)
        self.bias = self.hip.alloc(4 * 129)
        self.ws_floats = 3 * 129 * 129
        self.ws = self.hip.alloc(4 * self.ws_floats)

    def close(self) -> None:
        self.lib.mgc_hip_exec_destroy(self.x)
        self.hip.free()

    def run(self, args: GemmArgs, m: int, n: int) -> tuple[int, np.ndarray | None]:
        self.hip.put(self.c, np.full(m * n, np.nan, np.float32))
        args.c, args.ldc = self.c, n
        args.workspace, args.workspace_floats = self.ws, self.ws_floats
        self.lib.mgc_hip_gemm(self.x, ctypes.byref(args))
        code = self.lib.mgc_hip_exec_status(self.x)
        return code, (self.hip.download(self.c, (m, n)) if code == MGC_OK else None)

    def epilogue(self, args: GemmArgs, ep: dict, m: int, n: int, rng) -> tuple[np.ndarray, np.ndarray]:
        bias = rng.standard_normal(max(m, n)).astype(np.float32)
        res = rng.standard_normal((m, n)).astype(np.float32)
        args.alpha, args.beta = ep["alpha"], ep["beta"]
        args.act, args.lo, args.hi = ACTS.index(ep["act"]), LO, HI
        if ep["bias_mode"]:
            args.bias, args.bias_mode = self.hip.put(self.bias, bias), ep["bias_mode"]
        if ep["residual"]:
            args.res, args.ldr = self.hip.put(self.r, res), n
        return bias[: (n if ep["bias_mode"] == 1 else m)], res


def _accepts(family: str, k: int, split: int, ep: dict, conv: bool = False, cg: int = 0, n: int = 4) -> bool:
    """Whether the library must run (True) or refuse (False) this forced call, from the
    families' documented limits (include/mgc_hip.h)."""
    dma = k % 4 == 0 and (not conv or cg % 4 == 0)
    if family == "register":
        return True
    if not dma:
        return False
    if family == "quarter":
        return split == 1 and (not conv or cg % 64 == 0)
    if family == "stream":
        return (k <= (48 if conv else 32) and split == 1 and ep["bias_mode"] != 2
                and ep["act"] in ("none", "relu", "clip"))
    return True


@pytest.fixture(scope="module")
def runner():
    r = Runner()
    yield r
    r.close()


def _check(got: np.ndarray, want: np.ndarray, what: str) -> float:
    err = np.abs(got.astype(np.float64) - want)
    bound = 1e-4 + 1e-4 * np.abs(want)
    assert np.isfinite(got).all(), f"{what}: non-finite output (an element left unwritten?)"
    assert (err <= bound).all(), f"{what}: max-abs {err.max():.3e}"
    return float(err.max())


@pytest.mark.parametrize("family", FAMILIES)
def test_forced_family_on_edge_shapes(family, runner):
    rng = np.random.default_rng(GEMM_FAMILIES[family])
    splits = (1, 2, 3) if family in SPLIT_FAMILIES else (1,)
    ran = refused = 0
    worst = 0.0
    for i, (m, n, k) in enumerate(itertools.product(MN, MN + N_VEC, K_ANY + K_VEC)):
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = (rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32)
        runner.hip.put(runner.a, a)
        runner.hip.put(runner.b, np.ascontiguousarray(b.T))  # packed [N][K]
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        for split in splits:
            ep = _epilogue(i + split)
            if family == "stream" and i % 4:
                # mostly epilogues the streaming kernel takes; every fourth shape keeps the
                # rotation (refusals of gelu, tanh, sigmoid and row biases)
                ep["act"], ep["bias_mode"] = ("none", "relu", "clip")[i % 3], (0, 1)[(i // 3) % 2]
            args = GemmArgs()
            args.M, args.N, args.K = m, n, k
            args.a = Operand(kind=MGC_OP_STRIDED, p=runner.a, rs=k, cs=1)
            args.b = Operand(kind=MGC_OP_STRIDED, p=runner.b, rs=1, cs=k)
            args.split_k = split
            args.kernel = GEMM_FAMILIES[family]
            bias, res = runner.epilogue(args, ep, m, n, rng)
            code, got = runner.run(args, m, n)
            what = f"{family} split {split} {m}x{n}x{k} {ep}"
            if not _accepts(family, k, split, ep, n=n):
                assert code == MGC_ERR_ARGS, f"{what}: expected a refusal, got {code}"
                assert f"kernel family {GEMM_FAMILIES[family]}".encode() in runner.lib.mgc_hip_last_error()
                refused += 1
                continue
            assert code == MGC_OK, f"{what}: {runner.lib.mgc_hip_last_error()}"
            worst = max(worst, _check(got, _expected(a64, b64, ep, bias, res), what))
            ran += 1
    print(f"[gpu] family {family}: {ran} calls checked (max-abs {worst:.2e}), {refused} refused", flush=True)
    assert ran > 0


CONVS = [  # (images, H, W, C, Kout, stride, pad)
    (1, 7, 9, 4, 5, 1, 1),
    (2, 9, 8, 4, 40, 2, 1),   # K 36: also the streaming kernel, two 32-column blocks, ragged rows
    (2, 11, 6, 16, 33, 2, 1),
    (1, 9, 9, 64, 65, 1, 1),
    (3, 6, 10, 8, 3, 2, 0),
    (1, 13, 5, 128, 17, 1, 0),
]


@pytest.mark.parametrize("family", FAMILIES)
def test_forced_family_on_nhwc_convolutions(family, runner):
    """3 x 3 NHWC convolutions as implicit GEMMs (A read through im2col, B packed [Kout][9 C])
    through every family, against a direct float64 convolution (the streaming kernel takes the
    windows of K = 9 C <= 48: the 4-channel cases)."""
    rng = np.random.default_rng(100 + GEMM_FAMILIES[family])
    for j, (nimg, h, w, c, kout, s, pad) in enumerate(CONVS):
        oh, ow = (h + 2 * pad - 3) // s + 1, (w + 2 * pad - 3) // s + 1
        m, k = nimg * oh * ow, 9 * c
        x = rng.standard_normal((nimg, h, w, c)).astype(np.float32)
        wt = (rng.standard_normal((3, 3, c, kout)) / np.sqrt(k)).astype(np.float32)  # HWIO
        runner.hip.put(runner.a, x)
        runner.hip.put(runner.b, np.ascontiguousarray(wt.reshape(k, kout).T))
        xp = np.pad(x.astype(np.float64), ((0, 0), (pad, pad), (pad, pad), (0, 0)))
        cols = np.stack([xp[:, i:i + s * oh:s, jj:jj + s * ow:s, :] for i in range(3) for jj in range(3)], axis=3)
        a64 = cols.reshape(m, k)  # rows (n, oh, ow), columns (kh, kw, c)
        for split in ((1, 2) if family in SPLIT_FAMILIES else (1,)):
            ep = _epilogue(3 * j + split)
            args = GemmArgs()
            args.M, args.N, args.K = m, kout, k
            args.a = Operand(kind=MGC_OP_CONV_NHWC, p=runner.a, rs=0, cs=0, H=h, W=w, C=c, KH=3, KW=3, SH=s, SW=s,
                             DH=1, DW=1, PT=pad, PL=pad, OH=oh, OW=ow, cg=c)
            args.b = Operand(kind=MGC_OP_STRIDED, p=runner.b, rs=1, cs=k)
            args.split_k = split
            args.kernel = GEMM_FAMILIES[family]
            bias, res = runner.epilogue(args, ep, m, kout, rng)
            code, got = runner.run(args, m, kout)
            what = f"{family} split {split} conv {nimg}x{h}x{w}x{c}->{kout} s{s} p{pad} {ep}"
            if not _accepts(family, k, split, ep, conv=True, cg=c, n=kout):
                assert code == MGC_ERR_ARGS, f"{what}: expected a refusal, got {code}"
                continue
            assert code == MGC_OK, f"{what}: {runner.lib.mgc_hip_last_error()}"
            _check(got, _expected(a64, wt.reshape(k, kout).astype(np.float64), ep, bias, res), what)
    print(f"[gpu] family {family}: convolutions checked", flush=True)


def test_unknown_family_and_unfit_split_are_refused(runner):
    rng = np.random.default_rng(7)
    m, n, k = 33, 65, 64
    runner.hip.put(runner.a, rng.standard_normal((m, k)).astype(np.float32))
    runner.hip.put(runner.b, rng.standard_normal((n, k)).astype(np.float32))
    for kernel, split, workspace in ((8, 1, True), (-1, 1, True), (1, 2, False)):
        args = GemmArgs()
        args.M, args.N, args.K = m, n, k
        args.a = Operand(kind=MGC_OP_STRIDED, p=runner.a, rs=k, cs=1)
        args.b = Operand(kind=MGC_OP_STRIDED, p=runner.b, rs=1, cs=k)
        args.alpha = 1.0
        args.kernel, args.split_k = kernel, split
        runner.hip.put(runner.c, np.full(m * n, np.nan, np.float32))
        args.c, args.ldc = runner.c, n
        if workspace:
            args.workspace, args.workspace_floats = runner.ws, runner.ws_floats
        runner.lib.mgc_hip_gemm(runner.x, ctypes.byref(args))
        assert runner.lib.mgc_hip_exec_status(runner.x) == MGC_ERR_ARGS
        assert b"kernel family" in runner.lib.mgc_hip_last_error()
    # the context is clean again after a refusal
    assert runner.lib.mgc_hip_exec_status(runner.x) == MGC_OK
