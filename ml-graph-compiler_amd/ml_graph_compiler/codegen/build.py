"""Native builds of the hip backend (reference counterpart: codegen/build.py:1-209).

Two artefacts:

* libmgc_hip.so, the kernel library and model runtime: every csrc/*.hip file compiled by hipcc
  for gfx950 (MI355X) and linked once, in-tree, by ``build_kernel_library`` (driven by
  __graft_entry__.build()). Packed FP32 instructions are disabled (-packed-fp32-ops).
* lib<name>.so per model: the emitter's host C++ compiled by g++ against include/mgc_hip.h and
  linked to libmgc_hip.so, cached under a key hashing the source, the kernel library and the
  flags, so compiling an unchanged model is free.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field
from pathlib import Path

from ..errors import CodegenError

CODEGEN_DIR = Path(__file__).resolve().parent
PACKAGE_ROOT = CODEGEN_DIR.parent  # .../ml-graph-compiler_amd/ml_graph_compiler
CSRC_DIR = PACKAGE_ROOT.parent / "csrc"
INCLUDE_DIR = PACKAGE_ROOT.parent.parent / "include"
LIB_DIR = PACKAGE_ROOT / "_lib"
KERNEL_LIB = LIB_DIR / "libmgc_hip.so"
ARCH = "gfx950"
HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wno-unused-value",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def find_hipcc() -> str:
    for candidate in (os.environ.get("MGC_HIPCC"), "hipcc", "/opt/rocm/bin/hipcc"):
        if candidate and shutil.which(candidate):
            return candidate
    raise CodegenError("hipcc not found (set MGC_HIPCC or install ROCm)")


def find_cxx() -> str:
    for candidate in (os.environ.get("MGC_CXX"), os.environ.get("CXX"), "g++", "c++", "clang++"):
        if candidate and shutil.which(candidate):
            return candidate
    raise CodegenError("no C++ compiler found (set MGC_CXX or CXX)")


def _run(cmd: list[str], what: str) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True, check=False)
    if proc.returncode != 0:
        raise CodegenError(f"{what} failed:\n{' '.join(cmd)}\n{proc.stderr[-4000:]}")


def kernel_sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def build_kernel_library(jobs: int = 4) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libmgc_hip.so in-tree (always rebuilds)."""
    hipcc = find_hipcc()
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    sources = kernel_sources()
    if not sources:
        raise CodegenError(f"no kernel sources under {CSRC_DIR}")
    objects = [obj_dir / (src.stem + ".o") for src in sources]

    def compile_one(pair: tuple[Path, Path]) -> None:
        src, obj = pair
        _run([hipcc, *HIPCC_FLAGS, "-I", str(INCLUDE_DIR), "-I", str(CSRC_DIR), "-c", str(src), "-o", str(obj)],
             f"hipcc {src.name}")

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        list(pool.map(compile_one, zip(sources, objects)))
    tmp = KERNEL_LIB.with_suffix(f".so.tmp{os.getpid()}")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libmgc_hip.so", *map(str, objects),
          "-o", str(tmp)], "link libmgc_hip.so")
    tmp.replace(KERNEL_LIB)
    return KERNEL_LIB


def kernel_library_path() -> Path:
    if not KERNEL_LIB.exists():
        raise CodegenError(
            f"{KERNEL_LIB} is not built; run __graft_entry__.build() (hipcc --offload-arch={ARCH})"
        )
    return KERNEL_LIB


_KERNEL_HANDLE: ctypes.CDLL | None = None


def load_kernel_library() -> ctypes.CDLL:
    """Load libmgc_hip.so once, globally, so model libraries resolve against this copy."""
    global _KERNEL_HANDLE
    if _KERNEL_HANDLE is None:
        lib = ctypes.CDLL(str(kernel_library_path()), mode=ctypes.RTLD_GLOBAL)
        lib.mgc_hip_gemm_workspace.restype = ctypes.c_long
        lib.mgc_hip_gemm_workspace.argtypes = [ctypes.c_int] * 4
        lib.mgc_hip_gemm_layer_norm_workspace.restype = ctypes.c_long
        lib.mgc_hip_gemm_layer_norm_workspace.argtypes = [ctypes.c_int] * 3
        lib.mgc_hip_last_error.restype = ctypes.c_char_p
        lib.mgc_hip_version.restype = ctypes.c_char_p
        lib.mgc_hip_device_count.restype = ctypes.c_int
        _KERNEL_HANDLE = lib
    return _KERNEL_HANDLE


def gemm_workspace_floats(m: int, n: int, k: int, batch: int) -> int:
    """Workspace the kernel library wants for one GEMM (asked at compile time)."""
    return int(load_kernel_library().mgc_hip_gemm_workspace(m, n, k, batch))


def gemm_layer_norm_workspace_floats(m: int, n: int, k: int) -> int:
    """Split-K workspace of a GEMM whose reduction also runs the LayerNorm of its rows (0: the
    library cannot fuse that shape)."""
    return int(load_kernel_library().mgc_hip_gemm_layer_norm_workspace(m, n, k))


def _file_digest(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()[:16]


@dataclass(frozen=True)
class BuildOptions:
    """Host compiler settings for the generated model code."""

    opt_level: str = "-O2"
    extra_flags: tuple[str, ...] = field(default_factory=tuple)


def default_cache_dir() -> Path:
    base = os.environ.get("MGC_CACHE_DIR")
    if base:
        return Path(base)
    return Path(os.environ.get("XDG_CACHE_HOME", Path.home() / ".cache")) / "ml-graph-compiler-hip"


@dataclass
class BuildResult:
    library: Path
    directory: Path
    command: list[str]
    cached: bool


def build_model_library(
    source: str,
    options: BuildOptions | None = None,
    cache_dir: Path | None = None,
    name: str = "model",
) -> BuildResult:
    """Compile one model's generated host code into lib<name>.so (cached)."""
    options = options or BuildOptions()
    cxx = find_cxx()
    lib_path = kernel_library_path()
    cache = Path(cache_dir) if cache_dir is not None else default_cache_dir()
    flags = [options.opt_level, "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-variable",
             "-Wno-unused-function", *options.extra_flags]
    digest = hashlib.sha256()
    for part in (source, _file_digest(lib_path), (INCLUDE_DIR / "mgc_hip.h").read_text(), cxx, *flags):
        digest.update(part.encode())
        digest.update(b"\0")
    directory = cache / f"{name}-{digest.hexdigest()[:20]}"
    library = directory / f"lib{name}.so"
    src_path = directory / f"{name}.cpp"
    command = [cxx, *flags, "-I", str(INCLUDE_DIR), str(src_path), "-L", str(LIB_DIR), "-lmgc_hip",
               f"-Wl,-rpath,{LIB_DIR}", "-o", str(library)]
    if library.exists():
        return BuildResult(library, directory, command, True)
    directory.mkdir(parents=True, exist_ok=True)
    src_path.write_text(source)
    tmp = library.with_suffix(f".so.tmp{os.getpid()}")
    _run([*command[:-1], str(tmp)], "hip model build")
    tmp.replace(library)
    return BuildResult(library, directory, command, False)
