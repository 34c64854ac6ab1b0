"""CPU oracle of the MXFP4 W4A16 GEMM -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package; the product package (cdna3-bench_amd/mxfp4_cdna3) never does.
"""
