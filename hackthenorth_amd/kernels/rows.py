"""Projections of 2 to 128 rows that read each weight once (MFMA tiles).

The speculative verify pass scores k + 1 tokens in one forward; the reference
runs its multi-row projections as Triton GEMM tiles (dryft/engine/
projections.py:168-183, kernels/gateup.py:40-58, kernels/split_down.py:85-101).
Here every multi-row projection is one htn_gemm_rows launch (plus a K-split
reduction when the strips alone cannot fill the GPU) with the batch-one
GEMVs' bf16 rounding boundaries. From TILE_ROWS rows on (a prompt's
prefill) the projections run as one tiled GEMM launch each (htn_gemm_tiles,
both operands staged in LDS), an input RMSNorm as its own row-norm launch;
otherwise rows run in chunks of 128.
"""
import torch

from .. import _lib

MAX_ROWS = 128
TILE_ROWS = 256


def _tiles(x, weight, n, epilogue, residual=None, gain=None, eps=1e-6):
    """One htn_gemm_tiles launch over every row of x (after the rows' RMSNorm
    with `gain`, when given); returns the [M, n] output."""
    rows, k = x.shape
    if gain is not None:
        xn = torch.empty((rows, k), dtype=x.dtype, device=x.device)
        _lib.call("htn_rms_norm", _lib.ptr(x), x.stride(0), _lib.ptr(gain), _lib.ptr(xn), rows, k,
                  float(eps), _lib.stream(x.device))
        x = xn
    out = torch.empty((rows, n), dtype=x.dtype, device=x.device)
    nbytes = _lib.load().htn_gemm_tiles_scratch_bytes(rows, n, k, epilogue)
    scratch = torch.empty((nbytes + 15) // 16, 4, dtype=torch.float32, device=x.device) \
        if nbytes > 0 else None
    _lib.call("htn_gemm_tiles", _lib.ptr(x), x.stride(0), _lib.ptr(weight), n, k, rows, epilogue,
              _lib.ptr(residual), residual.stride(0) if residual is not None else 0,
              _lib.ptr(out), out.stride(0), _lib.ptr(scratch), _lib.stream(x.device))
    return out


def _scratch(device, rows, n, k, epilogue, norm):
    nbytes = _lib.load().htn_gemm_rows_scratch_bytes(rows, n, k, epilogue, int(norm))
    if nbytes <= 0:
        return None
    return torch.empty((nbytes + 7) // 8, dtype=torch.int64, device=device)


def _check(x, weight):
    if x.dim() != 2 or x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise ValueError("rows must be a bf16 [M, K] matrix with unit column stride")
    if weight.dim() != 2 or weight.dtype != torch.bfloat16 or not weight.is_contiguous() \
            or weight.shape[1] != x.shape[1]:
        raise ValueError("weight must be a contiguous bf16 [N, K] matrix matching x")


def _launch(x, weight, n, epilogue, gain=None, eps=1e-6, residual=None, out=None, tokens=None):
    rows, k = x.shape
    scratch = _scratch(x.device, rows, n, k, epilogue, gain is not None)
    _lib.call("htn_gemm_rows", _lib.ptr(x), x.stride(0), _lib.ptr(gain), float(eps),
              _lib.ptr(weight), n, k, rows, epilogue, _lib.ptr(residual),
              residual.stride(0) if residual is not None else 0, _lib.ptr(out),
              out.stride(0) if out is not None else 0, _lib.ptr(tokens), _lib.ptr(scratch),
              _lib.stream(x.device))


def _chunks(rows):
    return [(s, min(rows, s + MAX_ROWS)) for s in range(0, rows, MAX_ROWS)]


def projection_rows(x, weight, gain=None, eps=1e-6):
    """bf16(W x_m) for every row m of x [M, K]; gain applies RMSNorm first."""
    _check(x, weight)
    _lib.require_gpu(x, weight, gain)
    if x.shape[0] >= TILE_ROWS:
        return _tiles(x, weight, weight.shape[0], _lib.EPI_STORE, gain=gain, eps=eps)
    out = torch.empty((x.shape[0], weight.shape[0]), dtype=x.dtype, device=x.device)
    for s, e in _chunks(x.shape[0]):
        _launch(x[s:e], weight, weight.shape[0], _lib.EPI_STORE, gain, eps, out=out[s:e])
    return out


def residual_rows(x, weight, residual):
    """bf16(bf16(W x_m) + residual_m) for every row (O and down projections)."""
    _check(x, weight)
    if residual.shape != (x.shape[0], weight.shape[0]) or residual.dtype != torch.bfloat16 \
            or residual.stride(1) != 1:
        raise ValueError("residual must be bf16 [M, N] with unit column stride")
    _lib.require_gpu(x, weight, residual)
    if x.shape[0] >= TILE_ROWS:
        return _tiles(x, weight, weight.shape[0], _lib.EPI_RESIDUAL, residual=residual)
    out = torch.empty((x.shape[0], weight.shape[0]), dtype=x.dtype, device=x.device)
    for s, e in _chunks(x.shape[0]):
        _launch(x[s:e], weight, weight.shape[0], _lib.EPI_RESIDUAL, residual=residual[s:e],
                out=out[s:e])
    return out


def splits_k(n, k, rows):
    """Whether the multi-row projection of a [n, k] weight over `rows` rows
    (per launch: at most MAX_ROWS) splits K across blocks: its split finish
    can then also write the next RMSNorm at no extra launch."""
    rows = max(1, min(rows, MAX_ROWS))
    return _lib.load().htn_gemm_rows_scratch_bytes(rows, n, k, _lib.EPI_RESIDUAL, 0) > 0


def residual_norm_rows(x, weight, residual, gain, eps=1e-6):
    """(out, normed): out = residual_rows(x, weight, residual) and normed its
    RMSNorm with `gain` (the next layer's input), both written by one launch
    when the projection splits K."""
    _check(x, weight)
    n = weight.shape[0]
    if residual.shape != (x.shape[0], n) or residual.dtype != torch.bfloat16 \
            or residual.stride(1) != 1:
        raise ValueError("residual must be bf16 [M, N] with unit column stride")
    if gain is None or gain.shape != (n,) or gain.dtype != torch.bfloat16 \
            or not gain.is_contiguous():
        raise ValueError("gain must be a contiguous bf16 [N] vector")
    _lib.require_gpu(x, weight, residual, gain)
    if x.shape[0] >= TILE_ROWS:
        out = _tiles(x, weight, n, _lib.EPI_RESIDUAL, residual=residual)
        normed = torch.empty_like(out)
        _lib.call("htn_rms_norm", _lib.ptr(out), out.stride(0), _lib.ptr(gain), _lib.ptr(normed),
                  out.shape[0], n, float(eps), _lib.stream(x.device))
        return out, normed
    out = torch.empty((x.shape[0], n), dtype=x.dtype, device=x.device)
    normed = torch.empty_like(out)
    for s, e in _chunks(x.shape[0]):
        rows, k = x[s:e].shape
        scratch = _scratch(x.device, rows, n, k, _lib.EPI_RESIDUAL_NORM, False)
        _lib.call("htn_gemm_rows_residual_norm", _lib.ptr(x[s:e]), x.stride(0),
                  _lib.ptr(weight), n, k, rows, _lib.ptr(residual[s:e]), residual.stride(0),
                  _lib.ptr(out[s:e]), out.stride(0), _lib.ptr(gain), float(eps),
                  _lib.ptr(normed[s:e]), _lib.ptr(scratch), _lib.stream(x.device))
    return out, normed


def swiglu_rows(x, gate_up_weight, gain=None, eps=1e-6):
    """SwiGLU of the packed gate/up projection ([2I, K]: gate rows, then up rows)."""
    _check(x, gate_up_weight)
    if gate_up_weight.shape[0] % 2:
        raise ValueError("packed gate/up width must be even")
    _lib.require_gpu(x, gate_up_weight, gain)
    n = gate_up_weight.shape[0] // 2
    if x.shape[0] >= TILE_ROWS:
        return _tiles(x, gate_up_weight, n, _lib.EPI_SWIGLU, gain=gain, eps=eps)
    out = torch.empty((x.shape[0], n), dtype=x.dtype, device=x.device)
    for s, e in _chunks(x.shape[0]):
        _launch(x[s:e], gate_up_weight, n, _lib.EPI_SWIGLU, gain, eps, out=out[s:e])
    return out


def greedy_rows(x, weight, gain=None, eps=1e-6):
    """argmax_n bf16(W x_m) per row (lowest id on ties); gain applies RMSNorm first."""
    _check(x, weight)
    _lib.require_gpu(x, weight, gain)
    tokens = torch.empty((x.shape[0],), dtype=torch.int64, device=x.device)
    for s, e in _chunks(x.shape[0]):
        _launch(x[s:e], weight, weight.shape[0], _lib.EPI_ARGMAX, gain, eps,
                tokens=tokens[s:e])
    return tokens
