"""CPU oracle of the reference's AWQ W4A16 path: test infrastructure, never imported by the product.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it (see awq_oracle.py).
"""
