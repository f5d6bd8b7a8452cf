"""CPU oracle for the SageAttention quantized path -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import it.
"""
