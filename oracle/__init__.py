"""CPU oracle of the group-64 linear path: test infrastructure only.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg;
never by the product package actune_amd.
"""
