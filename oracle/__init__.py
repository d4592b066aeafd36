"""Oracle package: CPU restatement of the reference MoE hot path.

TEST INFRASTRUCTURE ONLY — imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the torchtitan_amd product code.
"""
