"""Exception hierarchy of the compiler (reference: src/ml_graph_compiler/errors.py:1-27).

Every error this package raises derives from CompilerError; the subclasses say which stage
rejected the input, so callers can catch e.g. GraphError for bad feeds or an out-of-range
Gather index, and CodegenError for an unsupported operator or a failed hipcc/g++ build.
"""

from __future__ import annotations


class CompilerError(Exception):
    """Base class of every error raised by ml_graph_compiler."""


class GraphError(CompilerError):
    """A malformed graph (not SSA, cyclic, wrong types) or invalid run-time feeds."""


class ModelImportError(CompilerError):
    """A model file that cannot be imported."""


class UnsupportedOpError(CompilerError):
    """An operator or attribute value that a compiler stage does not support."""


class ShapeError(CompilerError):
    """Shape or type inference failed."""


class CodegenError(CompilerError):
    """Code generation, the native build, or loading the built library failed."""
