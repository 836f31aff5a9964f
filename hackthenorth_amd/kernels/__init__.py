"""Fused decode ops with the reference's Python signatures (dryft/engine/kernels/*).

Every op validates its arguments like the reference wrapper (ValueError on a
contract violation), allocates its outputs with torch on the input's device,
and launches one hand-written gfx950 kernel from libhtn_decode.so on the
current stream. There is no CPU or torch fallback.
"""
