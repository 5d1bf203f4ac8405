"""Test infrastructure: CPU restatement of the reference KAD-Conv forward.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker; the product package never does.
"""
