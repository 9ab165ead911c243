"""ml-graph-compiler with an MI355X-native `hip` code-generation backend.

The SSA IR, operator table, O0-O3 pass pipelines, memory-aware scheduler and static arena
planner behave as in the reference compiler; `codegen.compile_graph(graph, backend="hip")` lowers
the scheduled graph to hand-written gfx950 kernels in libmgc_hip.so.
"""

__version__ = "0.1.0"
