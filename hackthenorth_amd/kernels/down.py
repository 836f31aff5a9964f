"""Batch-one down projection with residual (dryft/engine/kernels/down.py:27).

The reference splits K into fp32 partials for parallelism and rounds the sum
to bf16 before adding the residual. Here one wave reduces a whole row (the
grid already spans the CUs at these sizes), with the same two roundings:
out = bf16(bf16(sum_k x_k w_nk) + residual_n).
"""
from .projection import residual_projection


def down_residual(x, w, residual):
    """w may be a bf16 [H, I] tensor or a QuantizedWeight of that shape."""
    n, k = w.shape
    if x.numel() != k or residual.numel() != n:
        raise ValueError("down projection requires one activation and residual row")
    return residual_projection(x, w, residual, "down projection")
