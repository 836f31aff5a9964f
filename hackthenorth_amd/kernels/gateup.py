"""Multi-row gate/up projection with the SwiGLU epilogue (dryft/engine/kernels/gateup.py:40).

The reference packs the weight offline as [K, I, 2] (gate, up interleaved per
column), i.e. a row-major [K, 2I] matrix. htn_gate_up_swiglu reads that
layout in place: a block streams 128 contiguous bytes (32 gate/up pairs) of
every weight row and regroups them in registers into MFMA fragments, so no
repacked copy exists and the weight is read once for all rows. Rounding is
the reference's: fp32 dot products rounded to bf16, SiLU rounded to bf16,
times up, rounded to bf16 (gateup.py:1-6).

`config` was the Triton tile (row tile, column tile, K tile, warps, stages);
only its K tile is honoured, as the reference's divisibility check
(gateup.py:50-51).
"""
import torch

from .. import _lib

LEGACY_CONFIG = (16, 128, 64, 4, 3)
MAX_ROWS = 32


def _scratch(device, rows, width, k):
    nbytes = _lib.load().htn_gate_up_swiglu_scratch_bytes(rows, width, k)
    if nbytes <= 0:
        return None
    return torch.empty((nbytes + 7) // 8, dtype=torch.int64, device=device)


def gate_up_swiglu(x, interleaved_weight, config=LEGACY_CONFIG):
    """bf16 x [..., K] and interleaved weight [K, 2I] -> [..., I].

    Decode-sized: up to 32 rows per launch (more run in chunks of 32). K must
    be a multiple of the config's K tile; inputs and weights are never
    mutated.
    """
    w = interleaved_weight
    if w.dim() != 2 or w.shape[1] % 2 or w.shape[0] != x.shape[-1]:
        raise ValueError("interleaved weight must be [K, 2I] matching x")
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError("gate_up_swiglu takes bf16 x and weight")
    if not w.is_contiguous():
        raise ValueError("interleaved weight must be contiguous")
    k = x.shape[-1]
    if k % config[2]:
        raise ValueError("K must divide the K tile")
    _lib.require_gpu(x, w)
    width = w.shape[1] // 2
    rows = x.reshape(-1, k)
    if not rows.is_contiguous():
        rows = rows.contiguous()
    m = rows.shape[0]
    out = torch.empty((m, width), dtype=x.dtype, device=x.device)
    for s in range(0, m, MAX_ROWS):
        e = min(m, s + MAX_ROWS)
        scratch = _scratch(x.device, e - s, width, k)
        _lib.call("htn_gate_up_swiglu", _lib.ptr(rows[s:e]), rows.stride(0), _lib.ptr(w), width,
                  k, e - s, _lib.ptr(out[s:e]), out.stride(0), _lib.ptr(scratch),
                  _lib.stream(x.device))
    return out.reshape(*x.shape[:-1], width)
