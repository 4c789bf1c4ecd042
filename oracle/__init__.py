"""CPU oracle (test infrastructure: the checker, never the product).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package.
"""
