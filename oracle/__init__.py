"""CPU oracle for MLX-format affine quantized matmul — TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg,
never by the product package helios_amd.
"""
