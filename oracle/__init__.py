"""CPU oracle for the gated-delta-rule hot path.

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the reference that results are compared
with.  The product path never imports it.
"""
