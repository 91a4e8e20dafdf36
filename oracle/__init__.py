"""Oracle for parity tests — test infrastructure, never a product code path.

``oracle.reference_ops`` restates the reference's pure-torch fused ops on the
CPU, op for op. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import it, and only as the reference results or the CPU baseline.
"""
