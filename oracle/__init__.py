"""CPU oracle for vAi's matmul hot path -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker. The product library never calls it.
"""
