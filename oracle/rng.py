"""Counter-based RNG restated in numpy -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the checker of the HIP library: nothing in the
product path imports it.

The generator is a splitmix64 finaliser applied to (key + (i+1) * golden)
where key mixes a 64-bit seed and a 64-bit stream id. Every step is integer
arithmetic or a single correctly rounded fp32 multiply followed by
round-to-nearest-even to bfloat16, so the HIP generator in
hackthenorth_amd/csrc/rng.hip produces bit-identical tensors on any machine.
The reference draws its test tensors from torch's RNG
(dryft/tests/test_fused_kernels.py:21-37); torch streams are not stable across
machines, so the shapes and distributions are kept and the generator replaced.

Distributions:
  normal(std)   Irwin-Hall sum of four 16-bit uniforms, centred and scaled to
                unit variance (|z| <= 3.46), times std -- an approximation of
                N(0, std^2) that stays bit-reproducible.
  randint(n)    multiply-shift of the top 32 bits: floor(u32 * n / 2^32).
  uniform(a,b)  a + (b-a) * (top 24 bits / 2^24), fp32 multiply then add.
  w8 codes      randint(255) - 127 as int8 bytes, or the round-to-nearest-even
                OCP fp8 e4m3fn encoding of that integer.

Parity pinned: tests/test_oracle_rng.py checks the moments, the range
limits, and hand-computed splitmix64 values for known counters; the e4m3fn
encoder and decoder are checked against torch.float8_e4m3fn conversions over
every code and over all integers in [-127, 127].
"""
import os

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
STREAM_MUL = np.uint64(0xD1B54A32D192ED03)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

# Irwin-Hall(4) over 16-bit uniforms: mean 4*65535/2, variance 4*(65536^2-1)/12.
IH_MEAN = 131070
IH_STD = float(np.sqrt(4.0 * (65536.0 ** 2 - 1.0) / 12.0))

CHUNK = 1 << 22


def mix64(z):
    """splitmix64 finaliser on uint64 arrays (wrap-around arithmetic)."""
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_key(seed, stream):
    with np.errstate(over="ignore"):
        return mix64(np.uint64(seed) ^ (np.uint64(stream) * STREAM_MUL))


def hashes(seed, stream, start, count):
    """64-bit hash of counters start..start+count-1 for (seed, stream)."""
    key = stream_key(seed, stream)
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return mix64(key + idx * GOLDEN)


def normal_scale(std):
    """fp32 multiplier applied to the centred Irwin-Hall integer."""
    return np.float32(std / IH_STD)


def f32_to_bf16_bits(x):
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16); NaN stays NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    with np.errstate(over="ignore"):
        r = u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    out = (r >> np.uint32(16)).astype(np.uint16)
    out[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return out


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_f32(seed, stream, count, std=1.0, start=0):
    """fp32 values before the bf16 rounding (exact products, see module doc)."""
    out = np.empty(count, dtype=np.float32)
    scale = normal_scale(std)
    for lo in range(0, count, CHUNK):
        n = min(CHUNK, count - lo)
        h = hashes(seed, stream, start + lo, n)
        m = np.uint64(0xFFFF)
        s = ((h & m) + ((h >> np.uint64(16)) & m) + ((h >> np.uint64(32)) & m)
             + (h >> np.uint64(48))).astype(np.int64) - IH_MEAN
        out[lo:lo + n] = s.astype(np.float32) * scale
    return out


def _chunked(count, fill):
    """Run fill(lo, n) over CHUNK-sized pieces on a thread pool (numpy releases
    the GIL in its array loops); each piece writes its own output range."""
    pieces = [(lo, min(CHUNK, count - lo)) for lo in range(0, count, CHUNK)]
    if len(pieces) <= 1:
        for lo, n in pieces:
            fill(lo, n)
        return
    from concurrent.futures import ThreadPoolExecutor
    workers = min(16, len(pieces), len(os.sched_getaffinity(0)))
    with ThreadPoolExecutor(workers) as pool:
        list(pool.map(lambda p: fill(*p), pieces))


def normal_bf16_bits(seed, stream, count, std=1.0, start=0):
    out = np.empty(count, dtype=np.uint16)

    def fill(lo, n):
        out[lo:lo + n] = f32_to_bf16_bits(normal_f32(seed, stream, n, std, start + lo))

    _chunked(count, fill)
    return out


def randint(seed, stream, count, high, start=0):
    """Uniform integers in [0, high) as int64."""
    h = hashes(seed, stream, start, count)
    with np.errstate(over="ignore"):
        return (((h >> np.uint64(32)) * np.uint64(high)) >> np.uint64(32)).astype(np.int64)


def uniform_f32(seed, stream, count, low, high, start=0):
    h = hashes(seed, stream, start, count)
    u = (h >> np.uint64(40)).astype(np.float32) * np.float32(1.0 / (1 << 24))
    return np.float32(low) + np.float32(high - low) * u


def int8_uniform(seed, stream, count, start=0):
    """Uniform int8 in [-127, 127]."""
    out = np.empty(count, dtype=np.int8)

    def fill(lo, n):
        h = hashes(seed, stream, start + lo, n)
        with np.errstate(over="ignore"):
            v = ((h >> np.uint64(32)) * np.uint64(255)) >> np.uint64(32)
        out[lo:lo + n] = (v.astype(np.int64) - 127).astype(np.int8)

    _chunked(count, fill)
    return out


def int8_codes(seed, stream, count, start=0):
    """int8_uniform as raw two's complement bytes (uint8)."""
    return int8_uniform(seed, stream, count, start).view(np.uint8)


def e4m3_decode(codes):
    """OCP fp8 e4m3fn codes (uint8) -> float32: sign, 4-bit exponent with bias 7,
    3-bit mantissa; exponent 0 is subnormal (m * 2^-9); 0x7f / 0xff are NaN."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c >> 7, -1.0, 1.0)
    e = (c >> 3) & 15
    m = c & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e - 10.0))
    out = (sign * mag).astype(np.float32)
    out[(e == 15) & (m == 7)] = np.nan
    return out


def e4m3_encode(x):
    """float32 -> e4m3fn codes with round-to-nearest-even; |x| >= 464 saturates
    to 448 (the generator never reaches it). Exact for every value the grid
    holds; other values go to the nearer grid neighbour, ties to even mantissa."""
    x = np.asarray(x, dtype=np.float32)
    grid = e4m3_decode(np.arange(0x7f, dtype=np.uint8)).astype(np.float64)  # 0 .. 448
    a = np.abs(x).astype(np.float64)
    hi = np.clip(np.searchsorted(grid, a, side="left"), 0, len(grid) - 1)
    lo = np.clip(hi - 1, 0, len(grid) - 1)
    d_lo = a - grid[lo]
    d_hi = grid[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(a >= grid[-1], 0x7e, code)
    sign = (np.signbit(x) & (code != 0)).astype(np.int64) << 7
    return (code | sign).astype(np.uint8)


def w8_codes(seed, stream, count, fmt, start=0):
    """Synthetic 8-bit weight bytes: uniform integers in [-127, 127] stored as
    int8 ("int8") or as their e4m3fn encoding ("fp8_e4m3")."""
    v = int8_uniform(seed, stream, count, start)
    if fmt == "int8":
        return v.view(np.uint8)
    if fmt == "fp8_e4m3":
        # e4m3_encode of each of the 255 possible integers, looked up per weight.
        table = e4m3_encode(np.arange(-127, 128, dtype=np.float32))
        return table[v.astype(np.int64) + 127]
    raise ValueError(fmt)


def w8_values(codes, fmt):
    """Exact float32 values of 8-bit weight codes."""
    if fmt == "int8":
        return np.asarray(codes, dtype=np.uint8).view(np.int8).astype(np.float32)
    # e4m3_decode of each of the 256 codes, looked up per weight.
    return e4m3_decode(np.arange(256, dtype=np.uint8))[np.asarray(codes, dtype=np.uint8)]
