"""CPU oracle of cider's quantize -> int8 GEMM -> dequant path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker; never by the product package.
"""
