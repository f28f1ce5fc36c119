"""CPU restatement of the reference oracles -- test infrastructure only.

Importable by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
always as the checker.  The product package fe2o3_amd never imports it.
"""
