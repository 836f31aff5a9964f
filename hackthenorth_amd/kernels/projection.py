"""Batch-one projections (dryft/engine/kernels/projection.py:36,70).

One hidden row times a row-major bf16 weight [N, K] with fp32 accumulation;
the norm prologue and the SwiGLU / residual epilogues keep the reference's
bf16 rounding boundaries. Inputs and weights are never mutated.
"""
import torch

from .. import _lib


def _bf16_gpu(*tensors):
    for t in tensors:
        if t.dtype != torch.bfloat16:
            raise ValueError("projections require bfloat16 tensors")
    _lib.require_gpu(*tensors)


def norm_projection(x, gain, weight, eps=1e-6, *, swiglu=False, block_n=4, warps=8):
    """RMSNorm one hidden row, then project (optionally through packed gate/up SwiGLU).

    `block_n` and `warps` were Triton launch parameters (projection.py:36-53);
    they are accepted and ignored.
    """
    if x.numel() != x.shape[-1] or not x.is_contiguous():
        raise ValueError("the batch-one prototype requires one contiguous hidden row")
    n, k = weight.shape
    if x.shape[-1] != k or gain.numel() != k or not weight.is_contiguous():
        raise ValueError("incompatible projection dimensions or weight stride")
    if swiglu:
        if n % 2:
            raise ValueError("packed gate/up width must be even")
        n //= 2
    _bf16_gpu(x, gain, weight)
    out = torch.empty((*x.shape[:-1], n), dtype=x.dtype, device=x.device)
    _lib.call("htn_gemv_norm", _lib.ptr(x), _lib.ptr(gain.contiguous()), float(eps),
              _lib.ptr(weight), _lib.ptr(out), n, k, int(bool(swiglu)), _lib.stream(x.device))
    return out


def output_projection_residual(x, weight, residual):
    """bf16(bf16(W x) + residual) for one row (projection.py:70-83)."""
    n, k = weight.shape
    if x.numel() != k or residual.numel() != n:
        raise ValueError("output projection requires one activation and residual row")
    if any(t.dtype != torch.bfloat16 or not t.is_contiguous() for t in (x, weight, residual)):
        raise ValueError("output projection requires contiguous BF16 tensors")
    _lib.require_gpu(x, weight, residual)
    out = torch.empty_like(residual)
    _lib.call("htn_gemv_residual", _lib.ptr(x), _lib.ptr(weight), _lib.ptr(residual),
              _lib.ptr(out), n, k, _lib.stream(x.device))
    return out


def projection(x, weight):
    """bf16(W x) for one contiguous row (the plain batch-one linear)."""
    n, k = weight.shape
    if x.numel() != k or not x.is_contiguous() or not weight.is_contiguous():
        raise ValueError("projection requires one contiguous row and a row-major weight")
    _bf16_gpu(x, weight)
    out = torch.empty((*x.shape[:-1], n), dtype=x.dtype, device=x.device)
    _lib.call("htn_gemv", _lib.ptr(x), _lib.ptr(weight), _lib.ptr(out), n, k,
              _lib.stream(x.device))
    return out
