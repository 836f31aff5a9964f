"""Multi-row down projection with residual, optionally fused with the next
RMSNorm (dryft/engine/kernels/split_down.py:46,85).

out = bf16(bf16(W x) + residual); normalized = rms_norm(out) * gain with the
reference's roundings. The reference splits K in two for parallelism; the
MFMA kernel picks its own K split and sums the fp32 partials in a fixed order.
`warps` was a Triton launch parameter and is ignored.
"""
import torch

from .rows import residual_norm_rows, residual_rows


def _weight(weight):
    return weight if weight.is_contiguous() else weight.contiguous()


def split_down_residual(x, weight, residual):
    """Contiguous bf16 x [M, K], residual [M, N] and weight [N, K] -> [M, N]."""
    return residual_rows(x, _weight(weight), residual)


def split_down_residual_norm(x, weight, residual, gain, eps, warps=16):
    """(out, normalized) where normalized is the next layer's RMSNorm input."""
    shape = residual.shape
    rows = x.reshape(-1, x.shape[-1])
    out, normed = residual_norm_rows(rows, _weight(weight), residual.reshape(-1, shape[-1]),
                                     gain, eps)
    return out.reshape(shape), normed.reshape(shape)
