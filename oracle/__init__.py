"""CPU oracle of the batch-invariant kernels — test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package; the product path (mlx-batch-invariant_amd/) never does.
"""
