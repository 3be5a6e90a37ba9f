"""The oracle: a CPU restatement of colizig's MoE expert path (cz_oracle.c).

TEST INFRASTRUCTURE ONLY - imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package colizig_amd.
"""
