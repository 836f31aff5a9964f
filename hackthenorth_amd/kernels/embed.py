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


def embed_gather_pair(ids_a, table_a, ids_b, table_b):
    """(embed_gather(ids_a, table_a), embed_gather(ids_b, table_b)) in one launch."""
    for ids, table in ((ids_a, table_a), (ids_b, table_b)):
        if ids.dtype != torch.int64 or table.dim() != 2 or table.dtype != torch.bfloat16 \
                or not table.is_contiguous():
            raise ValueError("embed_gather_pair expects int64 ids and contiguous bf16 [V, H] tables")
        _lib.require_gpu(ids, table)
    flat_a, flat_b = ids_a.reshape(-1).contiguous(), ids_b.reshape(-1).contiguous()
    out_a = torch.empty((*ids_a.shape, table_a.shape[1]), dtype=table_a.dtype, device=table_a.device)
    out_b = torch.empty((*ids_b.shape, table_b.shape[1]), dtype=table_b.dtype, device=table_b.device)
    _lib.call("htn_embed_gather_pair", _lib.ptr(flat_a), flat_a.numel(), _lib.ptr(table_a),
              table_a.shape[0], table_a.shape[1], _lib.ptr(out_a), _lib.ptr(flat_b), flat_b.numel(),
              _lib.ptr(table_b), table_b.shape[0], table_b.shape[1], _lib.ptr(out_b),
              _lib.stream(table_a.device))
    return out_a, out_b
