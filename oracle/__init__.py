"""CPU oracle of the W4A8 ConvRot QLinear path: test infrastructure, never part of the product.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package.
"""
