"""CPU oracle for the block sparse attention path -- test infrastructure only
(used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg)."""
