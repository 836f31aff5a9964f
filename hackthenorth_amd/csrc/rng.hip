// Counter-based random fills for synthetic weights, prompts and activations.
//
// splitmix64 finaliser over (stream key + (i + 1) * golden); normals are the
// centred Irwin-Hall sum of the hash's four 16-bit fields times an fp32 scale
// (one correctly rounded multiply), then round-to-nearest-even bf16. Integer
// arithmetic plus one IEEE multiply gives the same bits as the numpy
// generator on any machine.
#include "common.h"

namespace htn {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t stream_key_host(uint64_t seed, uint64_t stream) {
  uint64_t z = seed ^ (stream * 0xD1B54A32D192ED03ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

__global__ __launch_bounds__(kBlock) void fill_normal(uint32_t* __restrict__ out2, bf16_t* out1,
                                                      long count, uint64_t key, long start,
                                                      float scale) {
  // Two bf16 per thread per iteration through 32-bit stores when aligned.
  const long pairs = count >> 1;
  for (long p = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; p < pairs;
       p += static_cast<long>(gridDim.x) * kBlock) {
    float v[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint64_t h = mix64(key + static_cast<uint64_t>(start + 2 * p + j + 1) * kGolden);
      const int s = static_cast<int>((h & 0xffff) + ((h >> 16) & 0xffff) + ((h >> 32) & 0xffff) +
                                     (h >> 48)) - 131070;
      v[j] = __fmul_rn(static_cast<float>(s), scale);
    }
    if (out2) {
      out2[p] = pack_bf2(v[0], v[1]);
    } else {
      out1[2 * p] = static_cast<bf16_t>(f2bf(v[0]));
      out1[2 * p + 1] = static_cast<bf16_t>(f2bf(v[1]));
    }
  }
  if ((count & 1) && blockIdx.x == 0 && threadIdx.x == 0) {
    const long i = count - 1;
    const uint64_t h = mix64(key + static_cast<uint64_t>(start + i + 1) * kGolden);
    const int s = static_cast<int>((h & 0xffff) + ((h >> 16) & 0xffff) + ((h >> 32) & 0xffff) +
                                   (h >> 48)) - 131070;
    bf16_t* o = out2 ? reinterpret_cast<bf16_t*>(out2) : out1;
    o[i] = static_cast<bf16_t>(f2bf(__fmul_rn(static_cast<float>(s), scale)));
  }
}

__global__ __launch_bounds__(kBlock) void fill_randint(int64_t* __restrict__ out, long count,
                                                       uint64_t key, uint64_t high) {
  for (long i = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; i < count;
       i += static_cast<long>(gridDim.x) * kBlock) {
    const uint64_t h = mix64(key + static_cast<uint64_t>(i + 1) * kGolden);
    out[i] = static_cast<int64_t>(((h >> 32) * high) >> 32);
  }
}

// lo + p with p already rounded: two roundings, as numpy performs them (the
// pragma keeps the compiler from fusing the caller's multiply into an FMA).
__device__ __forceinline__ float add_no_fma(float lo, float p) {
#pragma clang fp contract(off)
  return lo + p;
}

__global__ __launch_bounds__(kBlock) void fill_uniform(float* __restrict__ out, long count,
                                                       uint64_t key, float lo, float span) {
  for (long i = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; i < count;
       i += static_cast<long>(gridDim.x) * kBlock) {
    const uint64_t h = mix64(key + static_cast<uint64_t>(i + 1) * kGolden);
    const float u = static_cast<float>(h >> 40) * (1.0f / 16777216.0f);  // exact
    out[i] = add_no_fma(lo, span * u);
  }
}

// Round-to-nearest-even fp8 e4m3fn encoding of a finite float with
// |f| < 464 (larger magnitudes saturate to 448; only integers in [-127, 127]
// are encoded here). Normals round the fp32 mantissa to 3 bits with the carry
// running into the exponent; below 2^-6 the value is a multiple of 2^-9.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const float a = fabsf(f);
  uint32_t code;
  if (a < 0.015625f) {
    code = static_cast<uint32_t>(rintf(a * 512.0f));  // 0..8; 8 is the smallest normal
  } else {
    const uint32_t au = __float_as_uint(a);
    const uint32_t r = (au + 0x7ffffu + ((au >> 20) & 1u)) >> 20;  // (exp << 3) | mantissa
    code = r - (120u << 3);
    if (code > 0x7eu) code = 0x7eu;
  }
  return sign | code;
}

__global__ __launch_bounds__(kBlock) void fill_w8(uint8_t* __restrict__ out, long count,
                                                  uint64_t key, int format) {
  for (long i = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; i < count;
       i += static_cast<long>(gridDim.x) * kBlock) {
    const uint64_t h = mix64(key + static_cast<uint64_t>(i + 1) * kGolden);
    const int v = static_cast<int>(((h >> 32) * 255u) >> 32) - 127;
    out[i] = static_cast<uint8_t>(format == HTN_WEIGHT_INT8 ? static_cast<uint32_t>(v) & 0xffu
                                                            : f32_to_e4m3(static_cast<float>(v)));
  }
}

long fill_blocks(long count) {
  long blocks = (count + kBlock - 1) / kBlock;
  const long cap = static_cast<long>(device_cus()) * 16;
  blocks = blocks < cap ? blocks : cap;
  return blocks < 1 ? 1 : blocks;
}

}  // namespace htn

using namespace htn;

extern "C" int htn_fill_uniform_f32(float* out, int64_t count, uint64_t seed, uint64_t stream,
                                    float lo, float span, htn_stream_t stream_) {
  if (!out || count <= 0) return HTN_EINVAL;
  hipLaunchKernelGGL(fill_uniform, dim3(fill_blocks(count)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream_), out, static_cast<long>(count),
                     stream_key_host(seed, stream), lo, span);
  return launch_status();
}

extern "C" int htn_fill_weights_w8(void* out, int64_t count, uint64_t seed, uint64_t stream,
                                   int format, htn_stream_t stream_) {
  if (!out || count <= 0 || (format != HTN_WEIGHT_INT8 && format != HTN_WEIGHT_FP8_E4M3))
    return HTN_EINVAL;
  hipLaunchKernelGGL(fill_w8, dim3(fill_blocks(count)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream_), static_cast<uint8_t*>(out),
                     static_cast<long>(count), stream_key_host(seed, stream), format);
  return launch_status();
}

extern "C" int htn_fill_normal_bf16(void* out, int64_t count, uint64_t seed, uint64_t stream,
                                    int64_t start, float scale, htn_stream_t stream_) {
  if (!out || count <= 0 || start < 0) return HTN_EINVAL;
  const uint64_t key = stream_key_host(seed, stream);
  long blocks = (count / 2 + kBlock - 1) / kBlock;
  const long cap = static_cast<long>(device_cus()) * 16;
  blocks = blocks < cap ? blocks : cap;
  if (blocks < 1) blocks = 1;
  const bool al = (reinterpret_cast<uintptr_t>(out) & 3u) == 0;
  hipLaunchKernelGGL(fill_normal, dim3(blocks), dim3(kBlock), 0, static_cast<hipStream_t>(stream_),
                     al ? static_cast<uint32_t*>(out) : nullptr,
                     al ? nullptr : static_cast<bf16_t*>(out), static_cast<long>(count), key,
                     static_cast<long>(start), scale);
  return launch_status();
}

extern "C" int htn_fill_randint_i64(int64_t* out, int64_t count, uint64_t seed, uint64_t stream,
                                    int64_t high, htn_stream_t stream_) {
  if (!out || count <= 0 || high <= 0 || high > (1LL << 32)) return HTN_EINVAL;
  const uint64_t key = stream_key_host(seed, stream);
  long blocks = (count + kBlock - 1) / kBlock;
  const long cap = static_cast<long>(device_cus()) * 16;
  blocks = blocks < cap ? blocks : cap;
  hipLaunchKernelGGL(fill_randint, dim3(blocks), dim3(kBlock), 0, static_cast<hipStream_t>(stream_),
                     out, static_cast<long>(count), key, static_cast<uint64_t>(high));
  return launch_status();
}
