"""RMSNorm and residual-add + RMSNorm (dryft/engine/kernels/rmsnorm.py:35,84).

Normalize in fp32, round to bf16, then multiply by the gain and round again:
out = bf16(gain * bf16(x * rsqrt(mean(x^2) + eps))).
"""
import torch

from .. import _lib

#: Widest row the one-wave-per-row kernel accepts (rmsnorm.py:13 uses 8192 too).
MAX_BLOCK = 8192


def add_rms_norm(x, residual, weight, eps):
    """Return (bf16(x + residual), rms_norm of that sum); inputs are not mutated.

    Mirrors kernels/rmsnorm.py:35-54: inputs must have identical contiguous
    shape, dtype and device.
    """
    if (x.shape != residual.shape or x.dtype != residual.dtype
            or x.device != residual.device or not x.is_contiguous()
            or not residual.is_contiguous() or weight.numel() != x.shape[-1]):
        raise ValueError("expected matching contiguous residual tensors and norm gain")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("add_rms_norm expects bfloat16 tensors")
    cols = x.shape[-1]
    if cols > MAX_BLOCK:
        raise ValueError("normalization row exceeds supported width")
    _lib.require_gpu(x, residual, weight)
    summed, normalized = torch.empty_like(x), torch.empty_like(x)
    _lib.call("htn_add_rms_norm", _lib.ptr(x), _lib.ptr(residual), _lib.ptr(weight.contiguous()),
              _lib.ptr(summed), _lib.ptr(normalized), x.numel() // cols, cols, float(eps),
              _lib.stream(x.device))
    return summed, normalized


def rms_norm(x, weight, eps):
    """RMSNorm over the last dimension (kernels/rmsnorm.py:84-107)."""
    shape = x.shape
    cols = shape[-1]
    if cols > MAX_BLOCK:
        raise ValueError(f"a row must fit in one block; {cols} columns does not")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or weight.numel() != cols:
        raise ValueError("rms_norm expects bfloat16 rows and a matching gain")
    _lib.require_gpu(x, weight)
    rows = x.reshape(-1, cols)
    if rows.stride(-1) != 1:
        rows = rows.contiguous()
    out = torch.empty((rows.shape[0], cols), dtype=x.dtype, device=x.device)
    row_stride = rows.stride(0) if rows.shape[0] > 1 else cols
    _lib.call("htn_rms_norm", _lib.ptr(rows), row_stride, _lib.ptr(weight.contiguous()),
              _lib.ptr(out), rows.shape[0], cols, float(eps), _lib.stream(x.device))
    return out.reshape(shape)
