"""MI355X-native batch-one Qwen3 decode path (hand-written gfx950 HIP kernels).

Drop-in for the decode path of dryft/engine in rickytang666/hackthenorth:
  hackthenorth_amd.kernels.*   the fused-op signatures of dryft/engine/kernels
  hackthenorth_amd.decode      KVCache, RotaryTable, forward, DecodeState, stream_decode
  hackthenorth_amd.engine      Engine(model_path).generate(input_ids, max_new_tokens)
  hackthenorth_amd.speculate   prompt lookup and exact verification
The kernels live in libhtn_decode.so (C ABI: include/htn_decode.h).
"""
from . import _lib

__all__ = ["_lib"]
