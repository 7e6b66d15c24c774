"""CPU oracle (test infrastructure only): NumPy and C restatements of the
reference's RNS algorithm.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may use it, and only as the checker."""
