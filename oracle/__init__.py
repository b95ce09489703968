"""CPU oracle for the quantized-weight path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package.  The product path (infer_amd) never does.
"""
