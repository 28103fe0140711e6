"""CPU oracle of the GDN hot path -- test infrastructure only (see gdn_oracle.py).

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import it; the shipped package
never does.
"""
