"""CPU oracle for the decoder matmul + decode-attention path: test infrastructure only (the
checker for tests/, __graft_entry__.smoke() and bench.py's cpu_baseline). Never imported by the
product package."""
