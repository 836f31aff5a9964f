// Shared device helpers for the gfx950 decode kernels.
//
// bf16 values travel as raw 16-bit patterns; conversions are explicit so every
// rounding boundary of the decode path is visible in the kernel source.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/htn_decode.h"

namespace htn {

typedef uint16_t bf16_t;

constexpr int kWave = 64;
constexpr int kBlock = 256;  // four waves

// ------------------------------------------------------------------ bf16

__device__ __forceinline__ float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 -> bf16 (the rounding torch and the reference
// use). gfx950 converts in hardware (v_cvt_pk_bf16_f32): its results equal
// the bit formula bf16 = (u + 0x7fff + ((u >> 16) & 1)) >> 16 on every normal,
// subnormal, infinite and halfway input, and it keeps NaN payloads with the
// quiet bit set ((u >> 16) | 0x40), as measured over 524288 bit patterns.
__device__ __forceinline__ uint32_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }
// bf16(g * sigmoid(g)) from the hardware exp2 and reciprocal: with
// t = e^-|g| <= 1, sigmoid(g) = 1 / (1 + t) for g >= 0 and t / (1 + t)
// otherwise, so the reciprocal's argument stays in [1, 2] and nothing
// overflows. About 2 ulp in fp32 for |g| < 8 before the bf16 rounding (the
// exponent argument's own rounding adds |g| * 2^-24 relative beyond that).
__device__ __forceinline__ float silu_bf(float g) {
  const float t = __builtin_amdgcn_exp2f(-fabsf(g) * 1.4426950408889634f);
  const float r = __builtin_amdgcn_rcpf(1.0f + t);
  return round_bf(g * (g >= 0.f ? r : t * r));
}

// Two roundings in one v_cvt_pk_bf16_f32: lo in bits 0-15, hi in 16-31.
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
// Streaming (nontemporal) 16- and 8-byte loads, for data read exactly once.
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 load_stream16(const void* p) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
}
__device__ __forceinline__ uint2 load_stream8(const void* p) {
  return __builtin_bit_cast(uint2, __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p)));
}

// round_bf of two values through one conversion.
__device__ __forceinline__ void round_bf2(float a, float b, float& ra, float& rb) {
  const uint32_t w = pack_bf2(a, b);
  ra = bf_lo(w);
  rb = bf_hi(w);
}

// 8 bf16 in a uint4 -> fp32 dot with 8 fp32 values.
__device__ __forceinline__ float dot8(uint4 w, const float* x) {
  float s = bf_lo(w.x) * x[0];
  s = fmaf(bf_hi(w.x), x[1], s);
  s = fmaf(bf_lo(w.y), x[2], s);
  s = fmaf(bf_hi(w.y), x[3], s);
  s = fmaf(bf_lo(w.z), x[4], s);
  s = fmaf(bf_hi(w.z), x[5], s);
  s = fmaf(bf_lo(w.w), x[6], s);
  s = fmaf(bf_hi(w.w), x[7], s);
  return s;
}

__device__ __forceinline__ void unpack8(uint4 v, float* o) {
  o[0] = bf_lo(v.x); o[1] = bf_hi(v.x); o[2] = bf_lo(v.y); o[3] = bf_hi(v.y);
  o[4] = bf_lo(v.z); o[5] = bf_hi(v.z); o[6] = bf_lo(v.w); o[7] = bf_hi(v.w);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// bf16(g * bf16(x * inv)) for eight packed elements (the reference's RMSNorm
// roundings).
__device__ __forceinline__ uint4 norm8(uint4 xv, uint4 gv, float inv) {
  float f[8], g[8];
  unpack8(xv, f);
  unpack8(gv, g);
  uint4 o;
  o.x = pack_bf2(g[0] * round_bf(f[0] * inv), g[1] * round_bf(f[1] * inv));
  o.y = pack_bf2(g[2] * round_bf(f[2] * inv), g[3] * round_bf(f[3] * inv));
  o.z = pack_bf2(g[4] * round_bf(f[4] * inv), g[5] * round_bf(f[5] * inv));
  o.w = pack_bf2(g[6] * round_bf(f[6] * inv), g[7] * round_bf(f[7] * inv));
  return o;
}

// Streaming 16-byte load of weights that are read exactly once per launch.
__device__ __forceinline__ uint4 load_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// acc + a.lo * b.lo + a.hi * b.hi for two packed bf16 pairs (v_dot2c_f32_bf16:
// the bf16 products are exact in fp32, accumulation in fp32).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}

// Raw buffer descriptor over [base, base + bytes): loads at byte offsets past
// the end return zeros (hardware range check), so tile loads need no clamping.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// The same descriptor from a base and range that are uniform but that the
// compiler cannot prove so (values selected per wave): readfirstlane keeps
// them in scalar registers; a descriptor in vector registers makes every load
// through it a per-lane descriptor loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
  return buffer_rsrc(reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo),
                     __builtin_amdgcn_readfirstlane(bytes));
}

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                               uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// As buffer_load16 with the non-temporal hint (bit 1 of the cache policy):
// weights are streamed exactly once per launch.
__device__ __forceinline__ uint4 buffer_load16_stream(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                      uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                 uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

// ------------------------------------------------------------------ 8-bit weights

// Weight storage: bf16, or one byte per weight (int8 two's complement, or OCP
// fp8 e4m3fn) with an fp32 scale per output row.
enum WeightFormat { WF_BF16 = 0, WF_INT8 = HTN_WEIGHT_INT8, WF_FP8 = HTN_WEIGHT_FP8_E4M3 };

template <int WF>
struct Fmt {
  static constexpr int kBytes = WF == WF_BF16 ? 2 : 1;  // bytes per weight
  static constexpr int kPerVec = 16 / kBytes;           // weights per 16-byte load
};

// Two fp32 values that are exact in bf16 (small integers) packed as bf16.
__device__ __forceinline__ uint32_t pack_exact_bf2(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Partial dot product of one 16-byte weight vector with its activations,
// which stay packed bf16 pairs (xp[i] holds activations 2i, 2i+1). Every
// weight is first made an exact bf16 value, so each step is one bf16 dot2:
//  bf16: 8 weights, used as loaded.
//  int8: 16 weights; each byte converts to fp32 with sign extension in the
//        conversion itself (exact), two values pack into one bf16 pair.
//  fp8:  16 weights; the hardware converts two e4m3fn codes straight to a
//        bf16 pair (gfx950 decodes OCP e4m3fn; every e4m3 value is a bf16
//        value, and the unit scale leaves it unchanged).
template <int WF>
__device__ __forceinline__ float dot_vec(uint4 w, const uint32_t* xp, float s) {
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
  if constexpr (WF == WF_BF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) s = dot2(d[j], xp[j], s);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t p0, p1;
      if constexpr (WF == WF_INT8) {
        const int v = static_cast<int>(d[j]);
        p0 = pack_exact_bf2(static_cast<float>(static_cast<signed char>(v)),
                            static_cast<float>(static_cast<signed char>(v >> 8)));
        p1 = pack_exact_bf2(static_cast<float>(static_cast<signed char>(v >> 16)),
                            static_cast<float>(v >> 24));
      } else {
        p0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(
                                              static_cast<int>(d[j]), 1.0f, false));
        p1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(
                                              static_cast<int>(d[j]), 1.0f, true));
      }
      s = dot2(p0, xp[2 * j], s);
      s = dot2(p1, xp[2 * j + 1], s);
    }
  }
  return s;
}

// ------------------------------------------------------------------ wave64 reductions
// DPP row operations act on 16-lane rows; the four row results are combined
// with readlane, so the total is wave-uniform. All 64 lanes must be active.

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over each 16-lane row; every lane of the row receives the row sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x128>(v);  // row_ror:8
  return v;
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x124>(v));
  v = fmaxf(v, dpp<0x128>(v));
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    uint64_t o = __shfl_xor(v, m, kWave);
    v = o > v ? o : v;
  }
  return v;
}

// Block-wide sum for 256 threads; `red` holds at least 4 floats of LDS.
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

// Order-preserving key for (bf16 logit, vocabulary id): the larger logit wins,
// and among equal logits the lower id wins. -0 is folded into +0 so that the
// two zeros compare equal, as they do in torch.argmax.
__device__ __forceinline__ uint64_t argmax_key(uint32_t bits16, uint32_t index) {
  if (bits16 == 0x8000u) bits16 = 0;
  uint32_t ord = (bits16 & 0x8000u) ? (~bits16 & 0xffffu) : (bits16 | 0x8000u);
  return (static_cast<uint64_t>(ord) << 32) | static_cast<uint64_t>(0xffffffffu - index);
}
__device__ __forceinline__ uint32_t argmax_key_index(uint64_t key) {
  return 0xffffffffu - static_cast<uint32_t>(key & 0xffffffffu);
}

// ------------------------------------------------------------------ host helpers

int device_cus();  // compute units of the current device (cached per device)
// Grid of the one-token residual GEMV (the output projection) over n rows of k
// weights (format 0 for bf16, or HTN_WEIGHT_INT8 / HTN_WEIGHT_FP8_E4M3): its block count and
// the rows each block takes per grid step (block b multiplies rows
// [b * rows, (b + 1) * rows), then the same span blocks * rows further on).
// False when the weights take the scalar path.
bool gemv_plain_layout(long n, long k, int format, long* blocks, int* rows);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

inline int launch_status() {
  return hipGetLastError() == hipSuccess ? HTN_OK : HTN_ELAUNCH;
}

}  // namespace htn
