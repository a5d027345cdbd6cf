"""CPU oracle of the static-lm attention hot path -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker.  The product never does.
"""
