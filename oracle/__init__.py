"""ORACLE — CPU restatement of the reference's population-training hot path. Test infrastructure only: imported by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the noise_amd package."""
