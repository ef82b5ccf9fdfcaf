"""CPU oracle of the decode/verify step (test infrastructure only: tests/, __graft_entry__.smoke(), bench.py's
cpu_baseline leg)."""
