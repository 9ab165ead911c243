"""Load and run a hip-compiled model through ctypes (reference: codegen/runtime_lib.py:1-256).

``HipCompiledModel`` keeps the reference CompiledModel's surface (inputs/outputs, run, benchmark,
profile, save/load, the thread and blocking knobs, report) so that callers switch backends by
passing ``backend="hip"``. Differences that follow from the device:

* mgc_hip_init allocates the model's single HBM block and uploads the weights once; ``run``
  stages host inputs into it, replays the captured hipGraph and copies the outputs back.
* ``run_device`` takes device pointers (for example torch tensors' data_ptr) and skips the copies;
  ``benchmark_device`` times graph replays on resident inputs with hipEvents.
* ``profile`` returns per-node seconds measured by hipEvent pairs in eager replays.
* A missing GPU or HIP failure raises CodegenError; an out-of-range Gather raises GraphError.
"""

from __future__ import annotations

import ctypes
import json
import shutil
import threading
import time
from collections.abc import Mapping, Sequence
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import numpy as np

from ..errors import CodegenError, GraphError, ModelImportError
from ..ir import Graph, TensorType, numpy_dtype
from ..memory import Strategy
from .build import (BuildOptions, BuildResult, build_model_library, gemm_layer_norm_workspace_floats,
                    gemm_workspace_floats, load_kernel_library)
from .hip import GeneratedModel, generate_hip

BACKENDS = ("hip",)


@dataclass
class CompileReport:
    nodes: int
    c_lines: int
    arena_bytes: int
    weights_bytes: int
    codegen_seconds: float
    build_seconds: float
    cached: bool
    openmp: bool = False
    kernels: dict[str, int] = field(default_factory=dict)
    plan: dict[str, object] = field(default_factory=dict)
    backend: str = "hip"


def _aligned_copy(weights: np.ndarray, alignment: int = 256) -> np.ndarray:
    raw = np.empty(weights.nbytes + alignment, np.uint8)
    start = (-raw.ctypes.data) % alignment
    out = raw[start : start + weights.nbytes]
    out[:] = weights
    return out


class HipCompiledModel:
    """A model compiled for MI355X: ``run(feeds)`` returns outputs as numpy arrays.

    Calls are serialized with a lock because they share the model's arena and hipGraph."""

    backend = "hip"

    def __init__(
        self,
        library: Path,
        weights: np.ndarray,
        inputs: list[tuple[str, TensorType]],
        outputs: list[tuple[str, TensorType]],
        report: CompileReport | None = None,
    ) -> None:
        self.kernels = load_kernel_library()
        self.library_path = Path(library)
        self.lib = ctypes.CDLL(str(library))
        lib = self.lib
        vp = ctypes.c_void_p
        lib.mgc_run.restype = ctypes.c_int
        lib.mgc_run.argtypes = [vp] * 4
        lib.mgc_run_device.restype = ctypes.c_int
        lib.mgc_run_device.argtypes = [vp] * 4
        lib.mgc_arena_bytes.restype = ctypes.c_size_t
        lib.mgc_weights_bytes.restype = ctypes.c_size_t
        lib.mgc_hip_init.restype = ctypes.c_int
        lib.mgc_hip_init.argtypes = [vp, ctypes.POINTER(vp), ctypes.POINTER(vp)]
        lib.mgc_hip_upload.restype = ctypes.c_int
        lib.mgc_hip_upload.argtypes = [vp]
        lib.mgc_hip_launch.restype = ctypes.c_int
        lib.mgc_hip_launch.argtypes = [ctypes.c_int]
        lib.mgc_hip_sync.restype = ctypes.c_int
        lib.mgc_hip_download.restype = ctypes.c_int
        lib.mgc_hip_download.argtypes = [vp]
        lib.mgc_hip_time_graph.restype = ctypes.c_double
        lib.mgc_hip_time_graph.argtypes = [ctypes.c_int]
        lib.mgc_get_max_threads.restype = ctypes.c_int
        lib.mgc_has_openmp.restype = ctypes.c_int
        lib.mgc_has_neon.restype = ctypes.c_int
        lib.mgc_set_num_threads.argtypes = [ctypes.c_int]
        lib.mgc_set_blocking.argtypes = [ctypes.c_int] * 3
        expected = int(lib.mgc_weights_bytes())
        if weights.nbytes != expected:
            raise CodegenError(f"weights blob has {weights.nbytes} bytes, library expects {expected}")
        self.weights = weights if weights.ctypes.data % 256 == 0 else _aligned_copy(weights)
        self.inputs = inputs
        self.outputs = outputs
        self.report = report
        self.node_names: list[tuple[str, str]] = []
        self.node_flops: list[int] = []
        self._lock = threading.Lock()
        self._in_ptrs = (vp * max(len(inputs), 1))()
        self._out_ptrs = (vp * max(len(outputs), 1))()
        self._profiled = False
        if int(self.kernels.mgc_hip_device_count()) < 1:
            raise CodegenError("no HIP device is visible; the hip backend runs on an MI355X (gfx950) GPU")
        self._A, self._W = vp(), vp()
        code = lib.mgc_hip_init(self.weights.ctypes.data, ctypes.byref(self._A), ctypes.byref(self._W))
        self._check(code, "mgc_hip_init")
        self._released = False

    # -- errors --------------------------------------------------------------------------------
    def _check(self, code: int, what: str) -> None:
        if code == 0:
            return
        if code == 1:
            raise GraphError("compiled model reported an out-of-range Gather index")
        detail = self.kernels.mgc_hip_last_error().decode(errors="replace")
        raise CodegenError(f"{what} failed with status {code}: {detail}")

    # -- reference CompiledModel surface --------------------------------------------------------
    @property
    def openmp(self) -> bool:
        return bool(self.lib.mgc_has_openmp())

    @property
    def neon(self) -> bool:
        return bool(self.lib.mgc_has_neon())

    def set_threads(self, n: int) -> None:
        self.lib.mgc_set_num_threads(int(n))

    def max_threads(self) -> int:
        return int(self.lib.mgc_get_max_threads())

    def set_blocking(self, mc: int, kc: int, npb: int) -> None:
        self.lib.mgc_set_blocking(int(mc), int(kc), int(npb))

    def _stage_inputs(self, feeds: Mapping[str, np.ndarray]) -> list[np.ndarray]:
        names = [n for n, _ in self.inputs]
        missing, extra = set(names) - set(feeds), set(feeds) - set(names)
        if missing or extra:
            raise GraphError(f"inputs: missing {sorted(missing)}, unexpected {sorted(extra)}")
        arrays = []
        for i, (name, t) in enumerate(self.inputs):
            a = np.asarray(feeds[name], order="C")
            if a.shape != t.shape or a.dtype != numpy_dtype(t.dtype):
                raise GraphError(f"input {name!r}: expected {t}, got {a.dtype}{list(a.shape)}")
            arrays.append(a)
            self._in_ptrs[i] = a.ctypes.data
        return arrays

    def run(self, feeds: Mapping[str, np.ndarray]) -> dict[str, np.ndarray]:
        arrays = self._stage_inputs(feeds)
        results: dict[str, np.ndarray] = {}
        for j, (name, t) in enumerate(self.outputs):
            out = np.empty(t.shape, numpy_dtype(t.dtype))
            results[name] = out
            self._out_ptrs[j] = out.ctypes.data
        with self._lock:
            code = self.lib.mgc_run(ctypes.addressof(self._in_ptrs), ctypes.addressof(self._out_ptrs), self._A, self._W)
        del arrays
        self._check(code, "mgc_run")
        return results

    def run_device(self, inputs: Sequence[int], outputs: Sequence[int]) -> None:
        """Run on device buffers given as integer addresses (graph input / output order)."""
        if len(inputs) != len(self.inputs) or len(outputs) != len(self.outputs):
            raise GraphError("run_device: wrong number of buffers")
        vp = ctypes.c_void_p
        ins = (vp * max(len(inputs), 1))(*inputs)
        outs = (vp * max(len(outputs), 1))(*outputs)
        with self._lock:
            code = self.lib.mgc_run_device(ctypes.addressof(ins), ctypes.addressof(outs), self._A, self._W)
        self._check(code, "mgc_run_device")

    def benchmark(self, feeds: Mapping[str, np.ndarray], warmup: int = 3, repeat: int = 20) -> list[float]:
        """Wall-clock seconds of ``repeat`` host-to-host runs (H2D + graph + D2H)."""
        for _ in range(warmup):
            self.run(feeds)
        times = []
        for _ in range(repeat):
            t0 = time.perf_counter()
            self.run(feeds)
            times.append(time.perf_counter() - t0)
        return times

    def upload(self, feeds: Mapping[str, np.ndarray]) -> None:
        arrays = self._stage_inputs(feeds)
        with self._lock:
            code = self.lib.mgc_hip_upload(ctypes.addressof(self._in_ptrs))
        del arrays
        self._check(code, "mgc_hip_upload")

    def launch(self, replays: int = 1) -> None:
        """Enqueue graph replays on the staged inputs without waiting."""
        with self._lock:
            self._check(self.lib.mgc_hip_launch(int(replays)), "mgc_hip_launch")

    def sync(self) -> None:
        with self._lock:
            self._check(self.lib.mgc_hip_sync(), "mgc_hip_sync")

    def download(self) -> dict[str, np.ndarray]:
        results = {}
        for j, (name, t) in enumerate(self.outputs):
            out = np.empty(t.shape, numpy_dtype(t.dtype))
            results[name] = out
            self._out_ptrs[j] = out.ctypes.data
        with self._lock:
            code = self.lib.mgc_hip_download(ctypes.addressof(self._out_ptrs))
        self._check(code, "mgc_hip_download")
        return results

    def benchmark_device(self, feeds: Mapping[str, np.ndarray], warmup: int = 3, replays: int = 20) -> float:
        """Milliseconds per forward: ``replays`` graph replays on resident inputs between two
        hipEvents on the model stream (no host copies inside the timed region)."""
        self.upload(feeds)
        self.launch(warmup)
        self.sync()
        with self._lock:
            ms = float(self.lib.mgc_hip_time_graph(int(replays)))
        if ms < 0:
            self._check(2, "mgc_hip_time_graph")
        self.sync()
        return ms / max(replays, 1)

    def _profile_api(self) -> None:
        if not hasattr(self.lib, "mgc_profile_data"):
            raise CodegenError("the model was not compiled with profile=True")
        self.lib.mgc_profile_data.restype = ctypes.POINTER(ctypes.c_double)
        self.lib.mgc_profile_size.restype = ctypes.c_int
        self.lib.mgc_hip_profile_run.restype = ctypes.c_int
        self.lib.mgc_hip_profile_run.argtypes = [ctypes.c_int]

    def profile_run(self, replays: int = 1) -> None:
        """Eager replays on the staged inputs with a hipEvent pair around every node."""
        self._profile_api()
        with self._lock:
            self._check(self.lib.mgc_hip_profile_run(int(replays)), "mgc_hip_profile_run")
        self._profiled = True

    def profile_reset(self) -> None:
        self._profile_api()
        self.lib.mgc_hip_profile_reset()

    def profile(self) -> list[tuple[str, str, float]]:
        """(op, node name, accumulated seconds) per node; needs a model built with profile=True.
        Runs one profiled pass first when none has run yet."""
        self._profile_api()
        if not self._profiled:
            self.profile_run(1)
        data = self.lib.mgc_profile_data()
        n = int(self.lib.mgc_profile_size())
        return [(op, name, float(data[i])) for i, (op, name) in enumerate(self.node_names[:n])]

    def release(self) -> None:
        if not getattr(self, "_released", True):
            self.lib.mgc_hip_release()
            self._released = True

    def __del__(self) -> None:
        try:
            self.release()
        except Exception:
            pass

    # -- persistence ---------------------------------------------------------------------------
    def save(self, directory: str | Path) -> Path:
        d = Path(directory)
        d.mkdir(parents=True, exist_ok=True)
        lib = d / self.library_path.name
        if lib.resolve() != self.library_path.resolve():
            lib.write_bytes(self.library_path.read_bytes())
        source = getattr(self.weights, "filename", None)
        target = d / "weights.bin"
        if source is not None and Path(source).exists():
            if Path(source).resolve() != target.resolve():
                shutil.copyfile(source, target)
        else:
            np.asarray(self.weights).tofile(target)
        meta = {
            "backend": "hip",
            "library": lib.name,
            "inputs": [[n, t.dtype, list(t.shape)] for n, t in self.inputs],
            "outputs": [[n, t.dtype, list(t.shape)] for n, t in self.outputs],
            "report": self.report.__dict__ if self.report else None,
            "nodes": [list(p) for p in self.node_names],
            "node_flops": list(self.node_flops),
        }
        (d / "model.json").write_text(json.dumps(meta, indent=2) + "\n")
        return d

    @classmethod
    def load(cls, directory: str | Path) -> HipCompiledModel:
        d = Path(directory)
        meta = json.loads((d / "model.json").read_text())
        if meta.get("backend", "hip") != "hip":
            raise CodegenError(f"{d} holds a {meta.get('backend')} model, not a hip one")
        weights = np.memmap(d / "weights.bin", dtype=np.uint8, mode="r")
        io = {k: [(n, TensorType(dt, tuple(s))) for n, dt, s in meta[k]] for k in ("inputs", "outputs")}
        model = cls(d / meta["library"], weights, io["inputs"], io["outputs"])
        model.node_names = [(str(op), str(name)) for op, name in meta.get("nodes", [])]
        model.node_flops = [int(f) for f in meta.get("node_flops", [])]
        return model


def compile_graph(
    graph: Graph,
    options: BuildOptions | None = None,
    cache_dir: str | Path | None = None,
    strategy: Strategy = "greedy_by_size",
    inplace: bool = True,
    name: str = "model",
    profile: bool = False,
    backend: str = "hip",
) -> HipCompiledModel:
    """Generate hip host code for an optimized, scheduled graph, build it and load it.

    The weights blob is written next to the library under its content hash and memory-mapped
    read-only until the device upload."""
    if backend not in BACKENDS:
        raise CodegenError(f"backend {backend!r} is not part of this build (available: {', '.join(BACKENDS)})")
    t0 = time.perf_counter()
    generated: GeneratedModel = generate_hip(graph, strategy, inplace, profile, gemm_workspace_floats,
                                             gemm_layer_norm_workspace_floats)
    codegen_seconds = time.perf_counter() - t0
    t0 = time.perf_counter()
    built: BuildResult = build_model_library(
        generated.source, options, Path(cache_dir) if cache_dir is not None else None, name
    )
    weights_path = built.directory / f"weights-{generated.weights.digest()}.bin"
    if not weights_path.exists():
        generated.weights.write(weights_path)
    weights = np.memmap(weights_path, dtype=np.uint8, mode="r")
    report = CompileReport(
        nodes=len(graph.nodes),
        c_lines=generated.lines,
        arena_bytes=generated.arena_bytes,
        weights_bytes=int(generated.weights.nbytes),
        codegen_seconds=round(codegen_seconds, 4),
        build_seconds=round(time.perf_counter() - t0, 4),
        cached=built.cached,
        kernels=generated.kernels,
        plan=generated.plan.summary(),
    )
    model = HipCompiledModel(built.library, weights, generated.inputs, generated.outputs, report)
    model.node_names = [(n.op, n.name) for n in graph.nodes]
    model.node_flops = list(generated.node_flops)
    return model


def compile_model(
    model: Any,
    opt: str = "O3",
    input_shapes: dict[str, tuple[int, ...]] | None = None,
    dims: dict[str, int] | None = None,
    reschedule: bool = True,
    **kwargs: Any,
) -> HipCompiledModel:
    """A model to a loaded hip model: import, optimize, schedule, compile.

    ``model`` is an IR Graph, an ONNX file path, serialized ONNX bytes, a decoded
    ``onnx_proto.ModelProto``, or the name of a bundled sample/config; ``input_shapes`` and
    ``dims`` bind the symbolic dimensions of an ONNX model's inputs."""
    from ..builders import CONFIGS, SAMPLES
    from ..onnx_import import from_onnx
    from ..onnx_proto import ModelProto
    from ..passes import optimize
    from ..schedule import schedule

    if isinstance(model, Graph):
        graph = model
    elif isinstance(model, str) and model in SAMPLES:
        graph = SAMPLES[model]()
    elif isinstance(model, str) and model in CONFIGS:
        graph = CONFIGS[model]()
    elif isinstance(model, (ModelProto, bytes, bytearray, memoryview)) or (
        isinstance(model, (str, Path)) and Path(model).is_file()
    ):
        graph = from_onnx(model, input_shapes, dims)
    else:
        raise ModelImportError(
            f"{model!r} is neither an ONNX file nor a bundled sample or config "
            f"({', '.join(sorted(SAMPLES) + sorted(CONFIGS))})"
        )
    optimize(graph, opt)
    if reschedule:
        schedule(graph)
    return compile_graph(graph, **kwargs)
