"""ORACLE - test infrastructure only.

CPU restatement of the reference's conv/GEMM path (spinn_cpu.c, cpu_runtime.c)
and the build recipe for the reference's own CPU runtime (Makefile `ref`).
Imported only by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg, as the reference results or the timed baseline - never by the product path.
"""
