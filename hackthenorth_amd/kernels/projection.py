"""Batch-one projections (dryft/engine/kernels/projection.py:36,70).

One hidden row times a row-major bf16 weight [N, K] with fp32 accumulation;
the norm prologue and the SwiGLU / residual epilogues keep the reference's
bf16 rounding boundaries. Inputs and weights are never mutated.
"""
import torch

from .. import _lib
from ..quant import QuantizedWeight


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
    if isinstance(weight, QuantizedWeight):
        _bf16_gpu(x, gain)
        _lib.require_gpu(weight.data)
        out = torch.empty((*x.shape[:-1], n), dtype=x.dtype, device=x.device)
        _lib.call("htn_gemv_norm_w8", _lib.ptr(x), _lib.ptr(gain.contiguous()), float(eps),
                  _lib.ptr(weight.data), _lib.ptr(weight.scale), weight.code, _lib.ptr(out), n,
                  k, int(bool(swiglu)), _lib.stream(x.device))
        return out
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
    return residual_projection(x, weight, residual, "output projection")


def residual_projection(x, weight, residual, what):
    """bf16(bf16(W x) + residual) for a bf16 or 8-bit weight."""
    n, k = weight.shape
    acts = (x, residual) if isinstance(weight, QuantizedWeight) else (x, weight, residual)
    if any(t.dtype != torch.bfloat16 or not t.is_contiguous() for t in acts):
        raise ValueError(f"{what} requires contiguous BF16 tensors")
    out = torch.empty_like(residual)
    if isinstance(weight, QuantizedWeight):
        _lib.require_gpu(x, weight.data, residual)
        _lib.call("htn_gemv_residual_w8", _lib.ptr(x), _lib.ptr(weight.data),
                  _lib.ptr(weight.scale), weight.code, _lib.ptr(residual), _lib.ptr(out), n, k,
                  _lib.stream(x.device))
        return out
    _lib.require_gpu(x, weight, residual)
    _lib.call("htn_gemv_residual", _lib.ptr(x), _lib.ptr(weight), _lib.ptr(residual),
              _lib.ptr(out), n, k, _lib.stream(x.device))
    return out


def projection(x, weight):
    """bf16(W x) for one contiguous row (the plain batch-one linear)."""
    n, k = weight.shape
    if x.numel() != k or not x.is_contiguous() or not weight.is_contiguous():
        raise ValueError("projection requires one contiguous row and a row-major weight")
    out = torch.empty((*x.shape[:-1], n), dtype=x.dtype, device=x.device)
    if isinstance(weight, QuantizedWeight):
        _bf16_gpu(x)
        _lib.require_gpu(weight.data)
        _lib.call("htn_gemv_w8", _lib.ptr(x), _lib.ptr(weight.data), _lib.ptr(weight.scale),
                  weight.code, _lib.ptr(out), n, k, _lib.stream(x.device))
        return out
    _bf16_gpu(x, weight)
    _lib.call("htn_gemv", _lib.ptr(x), _lib.ptr(weight), _lib.ptr(out), n, k,
              _lib.stream(x.device))
    return out
