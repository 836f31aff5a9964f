"""Device-side counter-based random fills for synthetic weights and inputs.

Same generator as the numpy one the tests use (bit-identical results): a
splitmix64 hash per element, Irwin-Hall(4) normals scaled by one fp32 multiply
and rounded to bf16. The reference draws random test tensors from torch's RNG
(dryft/tests/test_fused_kernels.py:21-37), which is not reproducible across
machines.
"""
import math

import torch

from .. import _lib

IH_STD = math.sqrt(4.0 * (65536.0 ** 2 - 1.0) / 12.0)


def normal_(t, seed, stream, std=1.0, start=0):
    """Fill a contiguous bf16 tensor in place with N(0, std) (Irwin-Hall approximation)."""
    if t.dtype != torch.bfloat16 or not t.is_contiguous():
        raise ValueError("normal_ fills contiguous bfloat16 tensors")
    _lib.require_gpu(t)
    if t.numel():
        _lib.call("htn_fill_normal_bf16", _lib.ptr(t), t.numel(), seed, stream, start,
                  std / IH_STD, _lib.stream(t.device))
    return t


def randint(count, high, seed, stream, device="cuda"):
    out = torch.empty((count,), dtype=torch.int64, device=device)
    _lib.call("htn_fill_randint_i64", _lib.ptr(out), count, seed, stream, high,
              _lib.stream(out.device))
    return out
