"""Embedding-row gather (the reference calls base.embed_tokens, dryft/engine/decode.py:81)."""
import torch

from .. import _lib


def embed_gather(ids, table):
    """out[..., :] = table[ids[...], :]; ids int64 on device (read by the kernel).

    Ids outside [0, V) give a zero row (torch would raise a device assert).
    """
    if ids.dtype != torch.int64 or table.dim() != 2 or table.dtype != torch.bfloat16 \
            or not table.is_contiguous():
        raise ValueError("embed_gather expects int64 ids and a contiguous bf16 [V, H] table")
    _lib.require_gpu(ids, table)
    flat = ids.reshape(-1).contiguous()
    out = torch.empty((*ids.shape, table.shape[1]), dtype=table.dtype, device=table.device)
    _lib.call("htn_embed_gather", _lib.ptr(flat), flat.numel(), _lib.ptr(table), table.shape[0],
              table.shape[1], _lib.ptr(out), _lib.stream(table.device))
    return out
