"""CPU oracle for the rldx_amd hot path — test infrastructure only.

Only tests/, __graft_entry__.smoke() (as the checker) and bench.py's
cpu_baseline leg may import this package.  Product code never does.
"""
