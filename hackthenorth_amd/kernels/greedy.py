"""Vocabulary projection with greedy selection (dryft/engine/kernels/greedy.py:45).

All vocabulary rows are evaluated; projection sums round to bf16 before the
comparison and equal maxima choose the lowest id. The decode step uses
greedy_head, which also fuses the final RMSNorm and writes the token (and
advances the position) in place on the device.
"""
import torch

from .. import _lib
from ..quant import QuantizedWeight


def greedy_head(x, gain, eps, w, out, advance=None):
    """token = argmax(bf16(W . rms_norm(x))) into out[0] (int64, device).

    gain=None skips the norm. advance, when given (int64 [1]), is incremented
    after the whole head has run -- the decode step's position.add_(1).
    """
    k = x.shape[-1]
    if x.numel() != k or not x.is_contiguous() or w.shape[1] != k or not w.is_contiguous():
        raise ValueError("greedy head expects one contiguous row and a row-major weight")
    if out.dtype != torch.int64 or (advance is not None and advance.dtype != torch.int64):
        raise ValueError("token and position buffers must be int64")
    scratch = torch.empty(_lib.HEAD_SCRATCH_BYTES, dtype=torch.uint8, device=x.device)
    if isinstance(w, QuantizedWeight):
        _lib.require_gpu(x, w.data, out)
        _lib.call("htn_lm_head_argmax_w8", _lib.ptr(x), _lib.ptr(gain), float(eps),
                  _lib.ptr(w.data), _lib.ptr(w.scale), w.code, w.shape[0], k, _lib.ptr(out),
                  _lib.ptr(advance), _lib.ptr(scratch), _lib.stream(x.device))
        return out
    _lib.require_gpu(x, w, out)
    _lib.call("htn_lm_head_argmax", _lib.ptr(x), _lib.ptr(gain), float(eps), _lib.ptr(w),
              w.shape[0], k, _lib.ptr(out), _lib.ptr(advance), _lib.ptr(scratch),
              _lib.stream(x.device))
    return out


def greedy_token(x, w):
    """argmax over bf16(x @ w.T) per row, lowest id on ties; returns x.shape[:-1] int64.

    One row takes the batch-one head; several rows read the vocabulary
    weight once per 32 rows (greedy.py:45-60 reads it once for up to 32).
    """
    k = x.shape[-1]
    if w.dim() != 2 or w.shape[1] != k or x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError("greedy_token expects bfloat16 rows and a [V, K] weight")
    _lib.require_gpu(x, w)
    rows = x.reshape(-1, k).contiguous()
    weight = w.contiguous()
    if rows.shape[0] == 1:
        out = torch.empty((1,), dtype=torch.int64, device=x.device)
        greedy_head(rows[0], None, 0.0, weight, out)
        return out.reshape(x.shape[:-1])
    from .rows import greedy_rows
    return greedy_rows(rows, weight).reshape(x.shape[:-1])


def argmax(logits):
    """Row-wise argmax over bf16 logits [..., V] (lowest id on ties)."""
    if logits.dtype != torch.bfloat16:
        raise ValueError("argmax expects bfloat16 logits")
    _lib.require_gpu(logits)
    rows = logits.reshape(-1, logits.shape[-1]).contiguous()
    out = torch.empty((rows.shape[0],), dtype=torch.int64, device=logits.device)
    _lib.call("htn_argmax_bf16", _lib.ptr(rows), rows.shape[0], rows.shape[1], _lib.ptr(out),
              _lib.stream(logits.device))
    return out.reshape(logits.shape[:-1])
