"""Test infrastructure: CPU oracles for the hip backend.

NOT PART OF THE PRODUCT. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
may import anything from this package, and only as the checker (or, for cpu_baseline, as the
timed CPU reference). The compiler and the compiled models never import it.

* ``oracle.interpreter`` restates the reference's numpy interpreter (interpreter.py, ops.py).
* ``oracle.cbackend`` restates the reference's generated-C emitter for the operators of the
  benchmark graphs and links the reference's own C kernels, built from
  /root/reference/src/ml_graph_compiler/codegen/runtime/mgc_kernels.c into oracle/_ref/ by
  oracle/Makefile (see that file).
"""
