"""TEST INFRASTRUCTURE ONLY: CPU oracle for the FP8 hot path (see oracle.py).

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg. The product package practice_cuda_amd never imports it.
"""
