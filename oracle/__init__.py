"""CPU oracle for the SSD forward and decode step -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker.  See ssd_oracle.py.
"""
