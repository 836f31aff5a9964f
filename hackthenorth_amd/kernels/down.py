"""Batch-one down projection with residual (dryft/engine/kernels/down.py:27).

The reference splits K into fp32 partials for parallelism and rounds the sum
to bf16 before adding the residual. Here one wave reduces a whole row (the
grid already spans the CUs at these sizes), with the same two roundings:
out = bf16(bf16(sum_k x_k w_nk) + residual_n).
"""
import torch

from .. import _lib


def down_residual(x, w, residual):
    n, k = w.shape
    if x.numel() != k or residual.numel() != n:
        raise ValueError("down projection requires one activation and residual row")
    if any(t.dtype != torch.bfloat16 or not t.is_contiguous() for t in (x, w, residual)):
        raise ValueError("down projection requires contiguous BF16 tensors")
    _lib.require_gpu(x, w, residual)
    out = torch.empty_like(residual)
    _lib.call("htn_gemv_residual", _lib.ptr(x), _lib.ptr(w), _lib.ptr(residual), _lib.ptr(out),
              n, k, _lib.stream(x.device))
    return out
