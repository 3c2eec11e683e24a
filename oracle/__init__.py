"""CPU oracle of the tensor-ring operator: test infrastructure, never the product.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it.
"""
