"""QK-norm + RoPE (+ KV-cache append) and SwiGLU (dryft/engine/kernels/fused.py:70,132,171).

Rounding: n = bf16(g * bf16(x * inv)) per 128-wide head, then
out = bf16(bf16(n * cos) + bf16(rotate_half(n) * sin)); v is copied unchanged.
"""
import torch

from .. import _lib


def _heads_view(t, name):
    if t.dim() != 4 or t.shape[-1] != _lib.HEAD_DIM or t.stride(-1) != 1 \
            or t.stride(-2) != _lib.HEAD_DIM:
        raise ValueError(f"{name} must be a [B, T, heads, 128] view with packed heads")
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16")


def _rope_rows(cos, sin):
    if cos.shape != sin.shape or cos.shape[-1] != _lib.HEAD_DIM or cos.stride(-1) != 1 \
            or sin.stride(-1) != 1 or cos.stride() != sin.stride():
        raise ValueError("cos/sin must be matching [..., T, 128] tables")
    rows = cos.shape[-2] if cos.dim() >= 2 else 1
    stride = cos.stride(-2) if cos.dim() >= 2 else 0
    return rows, stride


def norm_rope_cache(q, k, v, q_norm, k_norm, cos, sin, keys, values, positions):
    """Normalize/rotate q and k and write k, v into fixed cache slots.

    q/k/v are [B, T, heads, 128] views (packed projection slices allowed);
    cos/sin [1, T, 128]; keys/values [B, Hkv, capacity, 128] contiguous and
    mutated in place at slots `positions` (int64 [T], on device).
    Returns (q [B, Hq, T, 128] view, keys, values) like kernels/fused.py:70-82.
    """
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _heads_view(t, n)
    batch, tokens, q_heads, dim = q.shape
    k_heads = k.shape[2]
    if k.shape[:2] != (batch, tokens) or v.shape != k.shape:
        raise ValueError("q, k and v must share batch and token dimensions")
    if keys.shape != values.shape or keys.shape[0] != batch or keys.shape[1] != k_heads \
            or keys.shape[3] != dim or not keys.is_contiguous() or not values.is_contiguous():
        raise ValueError("caches must be contiguous [B, Hkv, capacity, 128]")
    if positions.dtype != torch.int64 or positions.numel() != tokens:
        raise ValueError("positions must be int64 with one entry per token")
    rows, stride = _rope_rows(cos, sin)
    if rows != tokens:
        raise ValueError("cos/sin need one row per token")
    _lib.require_gpu(q, k, v, keys, values, positions, cos, sin)
    out_q = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    _lib.call("htn_norm_rope_cache",
              _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
              _lib.ptr(v), v.stride(0), v.stride(1),
              _lib.ptr(q_norm.weight), _lib.ptr(k_norm.weight),
              float(q_norm.variance_epsilon), float(k_norm.variance_epsilon),
              _lib.ptr(cos), _lib.ptr(sin), stride, rows, 0,
              _lib.ptr(keys), _lib.ptr(values), keys.shape[2], _lib.ptr(positions.contiguous()),
              _lib.ptr(out_q), None, batch, tokens, q_heads, k_heads, _lib.stream(q.device))
    return out_q.transpose(1, 2), keys, values


def norm_rope(q, k, q_norm, k_norm, cos, sin, tile=True):
    """Q/K [B, T, H, 128] (packed projection views allowed) to contiguous outputs.

    `tile` selected a Triton launch shape in the reference (fused.py:132-157);
    the HIP kernel has one shape and ignores it.
    """
    _heads_view(q, "q")
    _heads_view(k, "k")
    batch, tokens, q_heads, _ = q.shape
    rows, stride = _rope_rows(cos, sin)
    if rows != tokens:
        raise ValueError("cos/sin need one row per token")
    _lib.require_gpu(q, k, cos, sin)
    out_q = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    out_k = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    _lib.call("htn_norm_rope_cache",
              _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
              None, 0, 0, _lib.ptr(q_norm.weight), _lib.ptr(k_norm.weight),
              float(q_norm.variance_epsilon), float(k_norm.variance_epsilon),
              _lib.ptr(cos), _lib.ptr(sin), stride, rows, 0, None, None, 0, None,
              _lib.ptr(out_q), _lib.ptr(out_k), batch, tokens, q_heads, k.shape[2],
              _lib.stream(q.device))
    return out_q, out_k


def swiglu(gate, up):
    """bf16(bf16(silu(gate)) * up), elementwise; gate/up may be strided row views."""
    if gate.shape != up.shape or gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
        raise ValueError("swiglu expects matching bfloat16 gate and up")
    _lib.require_gpu(gate, up)
    out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    cols = gate.shape[-1]
    g, u = gate.reshape(-1, cols), up.reshape(-1, cols)
    if g.stride(-1) != 1:
        g = g.contiguous()
    if u.stride(-1) != 1:
        u = u.contiguous()
    rows = g.shape[0]
    gs = g.stride(0) if rows > 1 else cols
    us = u.stride(0) if rows > 1 else cols
    _lib.call("htn_swiglu", _lib.ptr(g), gs, _lib.ptr(u), us, _lib.ptr(out), rows, cols,
              _lib.stream(gate.device))
    return out
