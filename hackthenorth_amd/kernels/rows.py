"""Projections of 2 to 128 rows that read each weight once (MFMA tiles).

The speculative verify pass scores k + 1 tokens in one forward; the reference
runs its multi-row projections as Triton GEMM tiles (dryft/engine/
projections.py:168-183, kernels/gateup.py:40-58, kernels/split_down.py:85-101).
Here every multi-row projection is one htn_gemm_rows launch (plus a K-split
reduction when the strips alone cannot fill the GPU) with the batch-one
GEMVs' bf16 rounding boundaries. From TILE_ROWS rows on (a prompt's
prefill) the plain product runs through hipBLASLt (htn_gemm_library) with
the epilogues as row-wise launches (RMSNorm before, SwiGLU or the residual add
with the next RMSNorm after), or, where the library has no algorithm and for
residual projections without a following norm, as one tiled GEMM launch with
the epilogue fused (htn_gemm_tiles); otherwise rows run in chunks of 128.
"""
import torch

from .. import _lib

MAX_ROWS = 128
TILE_ROWS = 256
# Plain products of TILE_ROWS rows or more through hipBLASLt (False: this
# library's tiled kernel for every prompt projection, e.g. to measure it).
LIBRARY = True


def _normed(x, gain, eps):
    """The rows' RMSNorm with `gain` (one row-norm launch), or x without one."""
    if gain is None:
        return x
    rows, k = x.shape
    xn = torch.empty((rows, k), dtype=x.dtype, device=x.device)
    _lib.call("htn_rms_norm", _lib.ptr(x), x.stride(0), _lib.ptr(gain), _lib.ptr(xn), rows, k,
              float(eps), _lib.stream(x.device))
    return xn


def _library(x, weight, width):
    """bf16(x W^T) for every row through hipBLASLt (htn_gemm_library), or
    None when the library has no algorithm for the shape."""
    if not LIBRARY:
        return None
    rows, k = x.shape
    lib = _lib.load()
    out = torch.empty((rows, width), dtype=x.dtype, device=x.device)
    workspace = torch.empty(lib.htn_gemm_library_workspace_bytes() // 16, 4, dtype=torch.float32,
                            device=x.device)
    rc = lib.htn_gemm_library(_lib.ptr(x), x.stride(0), _lib.ptr(weight), width, k, rows,
                              _lib.ptr(out), out.stride(0), _lib.ptr(workspace),
                              _lib.stream(x.device))
    if rc == _lib.HTN_EUNSUPPORTED:
        return None
    _lib.check(rc, "htn_gemm_library")
    return out


def _prefill(x, weight, n, epilogue, gain=None, eps=1e-6):
    """Store or SwiGLU epilogue over every row of a prompt: the plain product
    through the library, SwiGLU as a row-wise launch; the tiled kernel when
    the library declines the shape."""
    xn = _normed(x, gain, eps)
    width = 2 * n if epilogue == _lib.EPI_SWIGLU else n
    # A plain store of under 512 rows keeps the tiles' k split: the 8B QKV
    # projection at 256 rows takes 35.5 us there against 42.4 us through the
    # library (which wins from 512 rows on and for every other projection).
    y = _library(xn, weight, width) if epilogue != _lib.EPI_STORE or x.shape[0] >= 2 * TILE_ROWS \
        else None
    if y is None:
        return _tiles(xn, weight, n, epilogue)
    if epilogue == _lib.EPI_STORE:
        return y
    rows = x.shape[0]
    out = torch.empty((rows, n), dtype=x.dtype, device=x.device)
    _lib.call("htn_swiglu", _lib.ptr(y), y.stride(0), _lib.ptr(y[:, n:]), y.stride(0),
              _lib.ptr(out), rows, n, _lib.stream(x.device))
    return out


def _tiles(x, weight, n, epilogue, residual=None, gain=None, eps=1e-6):
    """One htn_gemm_tiles launch over every row of x (after the rows' RMSNorm
    with `gain`, when given); returns the [M, n] output."""
    rows, k = x.shape
    x = _normed(x, gain, eps)
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
        return _prefill(x, weight, weight.shape[0], _lib.EPI_STORE, gain=gain, eps=eps)
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
        rows = x.shape[0]
        y = _library(x, weight, n)
        if y is None:
            out = _tiles(x, weight, n, _lib.EPI_RESIDUAL, residual=residual)
            normed = torch.empty_like(out)
            _lib.call("htn_rms_norm", _lib.ptr(out), out.stride(0), _lib.ptr(gain),
                      _lib.ptr(normed), rows, n, float(eps), _lib.stream(x.device))
            return out, normed
        # bf16(bf16(y) + residual) and its RMSNorm in one row-wise launch.
        if not residual.is_contiguous():
            residual = residual.contiguous()
        out = torch.empty((rows, n), dtype=x.dtype, device=x.device)
        normed = torch.empty_like(out)
        _lib.call("htn_add_rms_norm", _lib.ptr(y), _lib.ptr(residual), _lib.ptr(gain),
                  _lib.ptr(out), _lib.ptr(normed), rows, n, float(eps), _lib.stream(x.device))
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
        return _prefill(x, gate_up_weight, n, _lib.EPI_SWIGLU, gain=gain, eps=eps)
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
