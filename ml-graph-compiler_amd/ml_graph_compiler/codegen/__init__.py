"""hip code-generation backend: emitter, native builds and the ctypes runtime."""

from .build import BuildOptions, build_kernel_library, build_model_library, kernel_library_path, load_kernel_library
from .hip import GeneratedModel, HipEmitter, WeightsBuilder, generate_hip, pack_b_nk
from .runtime_lib import CompileReport, HipCompiledModel, compile_graph, compile_model

CompiledModel = HipCompiledModel

__all__ = [
    "BuildOptions",
    "CompileReport",
    "CompiledModel",
    "GeneratedModel",
    "HipCompiledModel",
    "HipEmitter",
    "WeightsBuilder",
    "build_kernel_library",
    "build_model_library",
    "compile_graph",
    "compile_model",
    "generate_hip",
    "kernel_library_path",
    "load_kernel_library",
    "pack_b_nk",
]
