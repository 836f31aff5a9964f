"""Grouped-query decode attention over fixed KV storage (dryft/engine/kernels/attention.py).

Q is [B, Hq, Q, 128]; K/V are contiguous [B, Hkv, capacity, 128]; positions
holds one absolute cache position per query (int64, on device). Query t sees
slots <= positions[t]; slots after the largest position are never read.
Output has Q's shape, contiguous bf16. Inputs are not mutated (the prologue
variant appends the newest k/v to the cache, as the reference's does).
"""
import torch

from .. import _lib
from ..quant import QuantizedWeight


# (device index, stream handle) -> zero-initialised scratch buffers, newest last.
_SCRATCH = {}


def _scratch(device, batch, heads, queries, capacity, nbytes=None):
    """The attention scratch of the current stream. Its leading arrival
    counters must be zero before a call and every call leaves them zero, so
    one zero-filled buffer per stream is kept and reused (calls on one stream
    are ordered; buffers of different streams never meet). It only grows, and
    outgrown buffers are kept: a captured graph may still use their address.
    During capture a too-small buffer is not replaced: the call gets a fresh
    zero-filled one, whose fill the graph records ahead of the kernel.
    `nbytes` overrides the attention's own size (the fused output projection
    needs more)."""
    if nbytes is None:
        nbytes = _lib.load().htn_attention_scratch_bytes(batch, heads, queries, capacity)
    nbytes = max(nbytes, 4)
    current = torch.cuda.current_stream(device)
    buffers = _SCRATCH.setdefault((current.device_index, current.cuda_stream), [])
    if buffers and buffers[-1].numel() * 4 >= nbytes:
        return buffers[-1]
    buffer = torch.zeros((nbytes + 3) // 4, dtype=torch.float32, device=device)
    if not torch.cuda.is_current_stream_capturing():
        buffers.append(buffer)
    return buffer


def xcd_merge_mismatches(device=None, reset=False):
    """How many in-kernel split merges found a split of their (batch, kv head)
    pair on another XCD than their own, plus how many fused output-projection
    blocks could not use their pair's partials, summed over the attention
    scratch buffers kept for `device` (0 on a correct run: both rely on
    round-robin workgroup dispatch to keep a pair's partials in one L2).
    Reads device memory, so it synchronises; reset=True clears the counts."""
    index = torch.device(device).index if device is not None else torch.cuda.current_device()
    if index is None:
        index = torch.cuda.current_device()
    words = [_lib.ATTENTION_XCD_MISMATCH_BYTE // 4, _lib.ATTENTION_OUTPUT_ERROR_BYTE // 4]
    total = 0
    for (dev, _stream), buffers in _SCRATCH.items():
        if dev != index:
            continue
        for buffer in buffers:
            counts = buffer.view(torch.int32)[words[0]:words[1] + 1]
            total += int(counts.sum())
            if reset:
                counts.zero_()
    return total


class XcdMergeError(RuntimeError):
    """An in-kernel split merge found a split of its pair on another XCD."""


def check_xcd_merge(device=None):
    """Raise XcdMergeError if any in-kernel split merge on `device` has found a
    split of its (batch, kv head) pair on another XCD since the last check.

    Before raising, the device is switched to the separate merge launch, so
    states built afterwards are correct; graphs captured before keep the
    in-kernel merge and must be captured again. Reads device memory (one
    small copy per attention scratch buffer), so it synchronises.
    """
    count = xcd_merge_mismatches(device, reset=True)
    if count:
        index = torch.device(device).index if device is not None else None
        with torch.cuda.device(index if index is not None else torch.cuda.current_device()):
            _lib.call("htn_attention_disable_in_kernel_merge")
        raise XcdMergeError(
            f"{count} in-kernel attention merges saw splits from another XCD: workgroup "
            "dispatch is not round-robin on this device; the in-kernel merge is now off "
            "(separate merge launch), and states captured before must be rebuilt")


def _check_cache(keys, values, batch, kv_heads):
    if keys.shape != values.shape or keys.dim() != 4 or keys.shape[0] != batch \
            or keys.shape[1] != kv_heads or keys.shape[3] != _lib.HEAD_DIM \
            or not keys.is_contiguous() or not values.is_contiguous() \
            or keys.dtype != torch.bfloat16 or values.dtype != torch.bfloat16:
        raise ValueError("caches must be contiguous bf16 [B, Hkv, capacity, 128]")


def grouped_attention(q, k, v, positions, out=None):
    """softmax(q k^T / sqrt(128)) v per query over its visible slots (attention.py:213-237).

    `out`, when given, is a bf16 [B, Hq, Q, 128] view with unit dim stride
    (for example a transposed token-major buffer) that receives the rows."""
    batch, heads, queries, dim = q.shape
    kv_heads = k.shape[1]
    if dim != _lib.HEAD_DIM or q.stride(-1) != 1 or q.dtype != torch.bfloat16:
        raise ValueError("q must be bf16 [B, Hq, Q, 128] with unit dim stride")
    if heads % kv_heads:
        raise ValueError("query heads must be a multiple of kv heads")
    _check_cache(k, v, batch, kv_heads)
    if positions.dtype != torch.int64 or positions.numel() != queries:
        raise ValueError("positions must be int64 with one entry per query")
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise ValueError("out must be a bf16 view shaped like q with unit dim stride")
    _lib.require_gpu(q, k, v, positions, out)
    scratch = _scratch(q.device, batch, heads, queries, k.shape[2])
    _lib.call("htn_grouped_attention", _lib.ptr(q), q.stride(0), q.stride(1), q.stride(2),
              _lib.ptr(k), _lib.ptr(v), k.shape[2], _lib.ptr(positions.contiguous()),
              _lib.ptr(out), out.stride(0), out.stride(1), out.stride(2), batch, heads,
              kv_heads, queries, _lib.ptr(scratch), _lib.stream(q.device))
    return out


def _prologue(qkv, q_norm, k_norm, cos, sin, by_position, keys, values, positions, kv_heads,
              groups, k_offset, v_offset, next_weight=None):
    batch, width = qkv.shape[0], qkv.shape[-1]
    if qkv.numel() != batch * width or qkv.stride(-1) != 1 or qkv.dtype != torch.bfloat16:
        raise ValueError("qkv must be a bf16 [B, 1, width] packed projection")
    if cos.shape != sin.shape or cos.shape[-1] != _lib.HEAD_DIM or not cos.is_contiguous() \
            or not sin.is_contiguous():
        raise ValueError("cos/sin must be contiguous 128-wide rows")
    _check_cache(keys, values, batch, kv_heads)
    heads = kv_heads * groups
    if k_offset < heads * _lib.HEAD_DIM or v_offset < k_offset + kv_heads * _lib.HEAD_DIM \
            or v_offset + kv_heads * _lib.HEAD_DIM > width:
        raise ValueError("k/v offsets do not fit the packed projection")
    if positions.dtype != torch.int64:
        raise ValueError("positions must be int64")
    _lib.require_gpu(qkv, keys, values, positions, cos, sin)
    rope_rows = cos.numel() // _lib.HEAD_DIM
    out = torch.empty((batch, heads, 1, _lib.HEAD_DIM), dtype=qkv.dtype, device=qkv.device)
    scratch = _scratch(qkv.device, batch, heads, 1, keys.shape[2])
    args = (_lib.ptr(qkv), qkv.stride(0), k_offset, v_offset,
            _lib.ptr(q_norm.weight), _lib.ptr(k_norm.weight), float(q_norm.variance_epsilon),
            float(k_norm.variance_epsilon), _lib.ptr(cos), _lib.ptr(sin), _lib.HEAD_DIM,
            rope_rows, int(by_position), _lib.ptr(keys), _lib.ptr(values), keys.shape[2],
            _lib.ptr(positions), _lib.ptr(out), batch, kv_heads, groups, _lib.ptr(scratch))
    if next_weight is None:
        _lib.call("htn_prologue_attention", *args, _lib.stream(qkv.device))
        return out
    # The projection that reads this output: idle CUs load its weights into
    # the L2 of the XCDs that will multiply them while the attention runs.
    if isinstance(next_weight, QuantizedWeight):
        data, fmt = next_weight.data, next_weight.code
    else:
        data, fmt = next_weight, 0
    if data.dim() != 2 or not data.is_contiguous():
        raise ValueError("next_weight must be a contiguous [N, K] weight")
    _lib.require_gpu(data)
    _lib.call("htn_prologue_attention_prefetch", *args, _lib.ptr(data), data.shape[0],
              data.shape[1], fmt, _lib.stream(qkv.device))
    return out


def prologue_attention_output(qkv, q_norm, k_norm, cos, sin, keys, values, positions,
                              kv_heads, groups, k_offset, v_offset, o_weight, residual):
    """prologue_attention followed by output_projection_residual(a, o_weight,
    residual) (attention.py:162 then projection.py:70, as fused_layer.py:146-147
    runs them), in one library call: for one sequence the projection runs in
    the attention launch (each kv head's XCD multiplies that head group's
    columns of W_o while the attention runs) plus a small summing launch.
    Returns [batch, H] bf16, H = o_weight rows."""
    batch, width = qkv.shape[0], qkv.shape[-1]
    if qkv.numel() != batch * width or qkv.stride(-1) != 1 or qkv.dtype != torch.bfloat16:
        raise ValueError("qkv must be a bf16 [B, 1, width] packed projection")
    if cos.shape != sin.shape or cos.shape[-1] != _lib.HEAD_DIM or not cos.is_contiguous() \
            or not sin.is_contiguous():
        raise ValueError("cos/sin must be contiguous 128-wide rows")
    _check_cache(keys, values, batch, kv_heads)
    heads = kv_heads * groups
    if k_offset < heads * _lib.HEAD_DIM or v_offset < k_offset + kv_heads * _lib.HEAD_DIM \
            or v_offset + kv_heads * _lib.HEAD_DIM > width:
        raise ValueError("k/v offsets do not fit the packed projection")
    if positions.dtype != torch.int64:
        raise ValueError("positions must be int64")
    if isinstance(o_weight, QuantizedWeight):
        data, scale, fmt = o_weight.data, o_weight.scale, o_weight.code
    else:
        data, scale, fmt = o_weight, None, 0
    n = data.shape[0]
    if data.dim() != 2 or not data.is_contiguous() or data.shape[1] != heads * _lib.HEAD_DIM:
        raise ValueError("o_weight must be a contiguous [H, Hq * 128] weight")
    if residual.dtype != torch.bfloat16 or residual.numel() != batch * n \
            or not residual.is_contiguous():
        raise ValueError("residual must be a contiguous bf16 [B, H]")
    _lib.require_gpu(qkv, keys, values, positions, cos, sin, data, residual)
    rope_rows = cos.numel() // _lib.HEAD_DIM
    out = torch.empty((batch, n), dtype=qkv.dtype, device=qkv.device)
    nbytes = _lib.load().htn_attention_output_scratch_bytes(batch, heads, kv_heads,
                                                            keys.shape[2], n)
    scratch = _scratch(qkv.device, batch, heads, 1, keys.shape[2], nbytes)
    _lib.call("htn_prologue_attention_output", _lib.ptr(qkv), qkv.stride(0), k_offset, v_offset,
              _lib.ptr(q_norm.weight), _lib.ptr(k_norm.weight), float(q_norm.variance_epsilon),
              float(k_norm.variance_epsilon), _lib.ptr(cos), _lib.ptr(sin), _lib.HEAD_DIM,
              rope_rows, 0, _lib.ptr(keys), _lib.ptr(values), keys.shape[2],
              _lib.ptr(positions), batch, kv_heads, groups, _lib.ptr(data), _lib.ptr(scale),
              fmt, n, _lib.ptr(residual), _lib.ptr(out), _lib.ptr(scratch),
              _lib.stream(qkv.device))
    return out


def prologue_attention(qkv, q_norm, k_norm, cos, sin, keys, values, positions,
                       kv_heads, groups, k_offset, v_offset, next_weight=None):
    """Single-token decode attention with norm/rope/cache-write fused in (attention.py:162).

    qkv is the packed (batch, 1, width) projection; cos/sin the selected
    [1, 1, 128] rows. Writes the newest K/V into slot positions[0] and
    returns [batch, heads, 1, 128]. `next_weight`, the output projection's
    weight (bf16 or QuantizedWeight), is read into the L2 of the XCDs whose
    GEMV blocks will multiply it, by blocks on CUs the attention leaves idle;
    results are the same with or without it.
    """
    return _prologue(qkv, q_norm, k_norm, cos, sin, False, keys, values, positions, kv_heads,
                     groups, k_offset, v_offset, next_weight)


def decode_attention(qkv, q_norm, k_norm, cos_table, sin_table, keys, values, position,
                     kv_heads, groups, k_offset, v_offset):
    """prologue_attention reading the RoPE row for position[0] straight from the
    [capacity, 128] tables, so the decode step needs no index_select launch."""
    return _prologue(qkv, q_norm, k_norm, cos_table, sin_table, True, keys, values, position,
                     kv_heads, groups, k_offset, v_offset)
