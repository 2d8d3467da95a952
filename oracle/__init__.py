"""CPU restatement of the reference decoder (the checker).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it; the product library never does.
"""
