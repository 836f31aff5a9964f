"""CPU oracle for the batch-one Qwen3 decode path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline);
the product package hackthenorth_amd never imports it.

  rng.py     counter-based RNG (numpy) shared bit-for-bit with the HIP generator
  qwen3.py   torch-eager Qwen3 forward with the reference's rounding boundaries
"""
