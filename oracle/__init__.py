"""CPU oracle of the MoE expert path -- test infrastructure only.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
as the checker; never by the product package.
"""
