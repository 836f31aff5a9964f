"""Multi-row gate/up projection with the SwiGLU epilogue (dryft/engine/kernels/gateup.py:40).

The reference packs the weight offline as [K, I, 2] (gate, up interleaved per
column). The MFMA kernel streams row-major [2I, K] weights (gate rows, then up
rows), so the interleaved weight is repacked once per tensor and cached; the
input weight is never mutated. `config` was the Triton tile and is ignored.
"""
import weakref

import torch

from .rows import swiglu_rows

LEGACY_CONFIG = (16, 128, 64, 4, 3)
_packed = weakref.WeakKeyDictionary()


def pack_interleaved(interleaved_weight):
    """[K, 2I] with columns (gate_i, up_i) -> contiguous [2I, K] (gate rows, up rows)."""
    w = interleaved_weight
    return torch.cat((w[:, 0::2].t(), w[:, 1::2].t()), dim=0).contiguous()


def gate_up_swiglu(x, interleaved_weight, config=LEGACY_CONFIG):
    """x [..., K] (2 to 32 rows per chunk) and interleaved weight [K, 2I] -> [..., I]."""
    if interleaved_weight.dim() != 2 or interleaved_weight.shape[1] % 2 \
            or interleaved_weight.shape[0] != x.shape[-1]:
        raise ValueError("interleaved weight must be [K, 2I] matching x")
    packed = _packed.get(interleaved_weight)
    if packed is None:
        packed = pack_interleaved(interleaved_weight)
        _packed[interleaved_weight] = packed
    rows = x.reshape(-1, x.shape[-1])
    if not rows.is_contiguous():
        rows = rows.contiguous()
    return swiglu_rows(rows, packed).reshape(*x.shape[:-1], packed.shape[0] // 2)
