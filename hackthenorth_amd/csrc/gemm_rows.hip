// Multi-row projections: verify passes, batched decode steps and prefill
// chunks (2 to 128 rows).
//
// y[m, n] = sum_k x[m, k] W[n, k] for every row m < M with the weight read
// once for all rows: the rows form the A operand of gfx950's
// v_mfma_f32_16x16x32_bf16 (one to eight 16-row tiles, rows past M are zero),
// a strip of 16 weight rows the B operand. The kernel stays HBM-bound on W:
//
//  * block = W waves (4 to 16, more when strips are few) on one 16-column
//    strip (plus the matching up strip for SwiGLU); the waves take
//    interleaved 64-wide k steps and reduce through LDS, so every output is
//    finished by the block that computed it. A step's 16-row x 128-byte
//    weight tile is loaded as two instructions of 8 whole rows x 128 bytes
//    (lane l: row l / 8, bytes 16 * (l % 8)), then regrouped through the
//    wave's own LDS tile into the MFMA layout (lane (c, q): row c, bytes
//    32q .. 32q + 31). Loading the MFMA layout directly spreads each
//    instruction's 64 lanes over 16 rows, twice the cache lines per byte of
//    whole-line loads, and the vector memory path, not HBM, then limits the
//    stream; the LDS round trip costs far less. Within a step the two MFMAs
//    see k permuted identically
//    in A and B (lane quad q holds k offsets 16q .. 16q+15), which leaves
//    each dot product unchanged;
//  * only when even 16 waves per strip cannot fill the GPU is K split over
//    KS blocks, whose fp32 partials a second, stream-ordered launch sums in a
//    fixed order (deterministic) before the epilogue;
//  * the optional RMSNorm runs once, as a row-norm launch into the scratch
//    buffer (reference roundings bf16(g * bf16(x * inv))), instead of in every
//    block;
//  * epilogues keep the batch-one GEMV's bf16 boundaries: store, + residual,
//    SwiGLU over the gate and up strips, or per-row argmax (lowest id on ties).
#include "common.h"

namespace htn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kStrip = 16;     // output columns per block (MFMA N)
constexpr int kStep = 64;      // k per step: two MFMAs of 32
constexpr int kMaxRowsMT = 128; // eight 16-row tiles (prefill chunks, large batches)
constexpr int kMaxRowsI = 32;   // rows per launch of the interleaved gate/up kernel
constexpr int kU = 1;          // k steps per wave per batch (1 measured fastest of 1, 2, 4)
constexpr int kMaxWaves = 16;
constexpr int kMaxK = 16384;

struct RowsArgs {
  const bf16_t* x; long x_rs;
  const bf16_t* w;
  const bf16_t* res; long res_rs;
  bf16_t* y; long y_rs;
  float* part;          // [KS][M][Nw] fp32 (KS > 1)
  uint64_t* keys;       // argmax: [strips][M]
  int64_t* tokens;      // argmax: [M]
  int M, N, K, KS, steps_per_split;
  // Residual epilogue fused with the next RMSNorm (K-split finish only):
  // normed [M][N] = bf16(gain * bf16(y * inv)), the row-wise RMSNorm of y.
  const bf16_t* ngain; float neps;
  bf16_t* normed;
  // RMSNorm of the input rows inside the projection (NORM kernels).
  const bf16_t* xgain; float xeps;
};

constexpr int kNormVec = 16;  // 16-byte vectors per lane of a row normalised in-kernel (K <= 8192)

constexpr long kAlign = 256;
long align_up(long v) { return (v + kAlign - 1) / kAlign * kAlign; }

__device__ __forceinline__ float silu_mul_bf(float g, float u) { return silu_bf(g) * u; }

// The 16 bytes of x (row m, k .. k+7) as an A fragment; rows past M and
// invalid steps give zeros.
__device__ __forceinline__ uint4 a_fragment(const RowsArgs& a, int m, int k, bool ok) {
  const int mm = m < a.M ? m : 0;
  const uint4 v = *reinterpret_cast<const uint4*>(a.x + mm * a.x_rs + k);
  return ok && m < a.M ? v : make_uint4(0, 0, 0, 0);
}

// Epilogue for one output (row m, column n) given the fp32 dot products of
// the (gate) column and, for SwiGLU, the up column.
template <int EPI>
__device__ __forceinline__ void store_out(const RowsArgs& a, int m, int n, float t0, float t1) {
  float out;
  if (EPI == HTN_EPI_STORE) out = t0;
  else if (EPI == HTN_EPI_RESIDUAL) out = round_bf(t0) + bf2f(a.res[m * a.res_rs + n]);
  else out = silu_mul_bf(round_bf(t0), round_bf(t1));
  a.y[m * a.y_rs + n] = static_cast<bf16_t>(f2bf(out));
}

// The fields every row kernel reads early, in scalar registers at entry: one
// round of scalar loads instead of one per dependent use.
__device__ __forceinline__ void preload_rows(const RowsArgs& a) {
  asm volatile("" ::"s"(a.x), "s"(a.x_rs), "s"(a.w), "s"(a.res), "s"(a.res_rs), "s"(a.y),
               "s"(a.y_rs), "s"(a.part), "s"(a.M), "s"(a.N), "s"(a.K), "s"(a.KS),
               "s"(a.steps_per_split));
}

constexpr int kPitch = 144;  // bytes per staged 64-element weight row (+16: conflict-free reads)

// One-tile kernels that normalise their rows hold the row's first vectors
// across the first weight issue (82-92 VGPRs unbounded: 5 waves per SIMD);
// bounded to 8 (S = 1, 60 VGPRs) and 6 (S = 2, 80) waves per SIMD without
// spills (8B 16-row batched step 3634 -> 3657 tok/s, 5-row verify unchanged).
template <int MT, int S, int EPI, int W, bool NORM>
__global__ __launch_bounds__(W * 64, NORM && MT == 1 ? (S == 1 ? 8 : 6) : 1) void gemm_rows_kernel(RowsArgs a) {
  preload_rows(a);
  if constexpr (NORM) asm volatile("" ::"s"(a.xgain), "s"(a.xeps));
  __shared__ float red[W][MT][S][kStrip * 16];
  __shared__ uint64_t best[EPI == HTN_EPI_ARGMAX ? MT * 16 : 1][kStrip];
  __shared__ __align__(16) unsigned char tile[W][16 * kPitch];
  __shared__ float inv_s[NORM ? MT * 16 : 1];
  const int tid = threadIdx.x, lane = tid & 63;
  // The wave index is uniform: readfirstlane keeps step indices and buffer
  // descriptors in scalar registers (a descriptor the compiler thinks varies
  // per lane is applied through a loop over lanes).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int strip = blockIdx.x, ks = blockIdx.y;
  const int n0 = strip * kStrip;
  const int col = lane & 15, quad = lane >> 4;
  const int Nw = S * a.N;
  const int j0 = ks * a.steps_per_split;
  const int total_steps = a.K / kStep;
  const int j1 = j0 + a.steps_per_split < total_steps ? j0 + a.steps_per_split : total_steps;

  // Load mapping: lane l reads 16 bytes (chunk l & 7) of strip rows l >> 3
  // and (l >> 3) + 8, through a buffer descriptor over the strip's rows:
  // rows past N (last strip) read zeros, and a batch past the wave's last
  // step gets an empty descriptor, so the loads need neither clamping nor a
  // branch (a branch that joins with fewer loads in flight makes the
  // compiler wait for all of them).
  const int lr = lane >> 3, lc = lane & 7;
  const uint32_t strip_bytes =
      static_cast<uint32_t>(a.N - n0 < kStrip ? a.N - n0 : kStrip) * static_cast<uint32_t>(a.K) * 2u;
  const unsigned char* sbase[S];
#pragma unroll
  for (int s = 0; s < S; ++s)
    sbase[s] = reinterpret_cast<const unsigned char*>(a.w + static_cast<long>(n0 + s * a.N) * a.K);
  const uint32_t voff0 = (static_cast<uint32_t>(lr) * a.K + lc * 8) * 2u;
  const uint32_t voff1 = voff0 + 8u * static_cast<uint32_t>(a.K) * 2u;
  unsigned char* wt = tile[wave];
  u32x4* wr0 = reinterpret_cast<u32x4*>(wt + lr * kPitch + lc * 16);
  u32x4* wr1 = reinterpret_cast<u32x4*>(wt + (lr + 8) * kPitch + lc * 16);
  const u32x4* rd = reinterpret_cast<const u32x4*>(wt + col * kPitch + quad * 32);

  // Weight batches (native vectors: a struct copy into LDS would keep the
  // array in scratch memory).
  u32x4 wv[kU][S][2];
#define HTN_ISSUE(JB)                                                                      \
  {                                                                                       \
    _Pragma("unroll") for (int u = 0; u < kU; ++u) {                                      \
      const int j = (JB) + u * W;                                                         \
      const uint32_t range = j < j1 ? strip_bytes : 0u;                                   \
      const uint32_t soff = static_cast<uint32_t>(j < j1 ? j : 0) * kStep * 2u;           \
      _Pragma("unroll") for (int s = 0; s < S; ++s) {                                     \
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(sbase[s], range);                   \
        wv[u][s][0] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff0, soff, 0);         \
        wv[u][s][1] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff1, soff, 0);         \
      }                                                                                   \
    }                                                                                     \
  }
  // RMSNorm prologue (NORM): each input row's 1 / rms by one wave, in the
  // row-norm kernel's order (lane l over vectors l, l + 64, ..., element by
  // element, then one wave sum), so the normalised fragments below equal
  // the row-norm kernel's output bit for bit. A wave's first row is loaded
  // before the first weight batch: vector loads complete in issue order, so
  // the reduction waits only for the row, with the weights still in flight.
  // Registers: the first kNormHead vectors per lane (rows up to 4096) are
  // held from before the weight issue; longer rows load the rest afterwards,
  // summed in the same order.
  constexpr int kNormHead = 8;
  const int nv = a.K >> 3;
  uint4 xv[NORM ? kNormHead : 1];
  // Row m of x through a descriptor over its K elements: vectors past the
  // row read zeros, without a branch.
  auto xrow = [&](int m) { return buffer_rsrc(a.x + m * a.x_rs, static_cast<uint32_t>(a.K) * 2u); };
  if constexpr (NORM) {
    const __amdgpu_buffer_rsrc_t rs = xrow(wave < a.M ? wave : 0);
#pragma unroll
    for (int jv = 0; jv < kNormHead; ++jv) xv[jv] = buffer_load16(rs, (jv * 64 + lane) * 16u, 0);
    __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the weights
  }
  HTN_ISSUE(j0 + wave);
  if constexpr (NORM) {
    // 1 / rms of row m from its first kNormHead vectors (given) and the rest
    // (loaded here), summed in the row-norm kernel's order.
    auto row_inv = [&](int m, const uint4 (&head)[kNormHead]) {
      float ss = 0.f;
#pragma unroll
      for (int jv = 0; jv < kNormHead; ++jv) {
        float f[8];
        unpack8(head[jv], f);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = fmaf(f[i], f[i], ss);
      }
      for (int v = kNormHead * 64 + lane; v < nv; v += 64) {
        float f[8];
        unpack8(*reinterpret_cast<const uint4*>(a.x + m * a.x_rs + v * 8), f);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = fmaf(f[i], f[i], ss);
      }
      return 1.0f / sqrtf(wave_sum(ss) / static_cast<float>(a.K) + a.xeps);
    };
    // The wave's first row, preloaded (padded rows: zero fragments stay zero).
    {
      const float inv = wave < a.M ? row_inv(wave, xv) : 0.f;
      if (lane == 0) inv_s[wave] = inv;
    }
    // Rows past the first per wave (more rows than waves).
    for (int m = wave + W; m < MT * 16; m += W) {
      float inv = 0.f;
      if (m < a.M) {
        const __amdgpu_buffer_rsrc_t rs = xrow(m);
        uint4 more[kNormHead];
#pragma unroll
        for (int jv = 0; jv < kNormHead; ++jv) more[jv] = buffer_load16(rs, (jv * 64 + lane) * 16u, 0);
        inv = row_inv(m, more);
      }
      if (lane == 0) inv_s[m] = inv;
    }
    // LDS-only barrier: __syncthreads would also wait for every vector load
    // in flight, i.e. for the first weight batch, one memory round trip
    // before the loop could issue the next one.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }

  f32x4_t acc[MT][S];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int s = 0; s < S; ++s) acc[t][s] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int jb = j0 + wave; jb < j1; jb += W * kU) {
    // This batch's A fragments (x, and the gain under NORM) first: vector
    // loads complete in issue order, so the multiplies wait only for these,
    // not for the next weight batch issued below.
    uint4 av[kU][MT][2], gv[kU][NORM ? 2 : 1];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = jb + u * W;
      const bool ok = j < j1;
      const int k = (ok ? j : j1 - 1) * kStep + quad * 16;
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        av[u][t][0] = a_fragment(a, t * 16 + col, k, ok);
        av[u][t][1] = a_fragment(a, t * 16 + col, k + 8, ok);
      }
      if constexpr (NORM) {
        gv[u][0] = *reinterpret_cast<const uint4*>(a.xgain + k);
        gv[u][1] = *reinterpret_cast<const uint4*>(a.xgain + k + 8);
      }
    }
    // Each 16-row x 64-element tile goes through this wave's LDS tile. LDS
    // operations of one wave execute in issue order: the reads see the
    // writes, and the next tile's writes follow the previous reads.
    u32x4 bf[kU][S][2];
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int s = 0; s < S; ++s) {
        *wr0 = wv[u][s][0];
        *wr1 = wv[u][s][1];
        __builtin_amdgcn_wave_barrier();
        bf[u][s][0] = rd[0];
        bf[u][s][1] = rd[1];
        __builtin_amdgcn_wave_barrier();
      }
    // The next batch (empty past the wave's last step) is in flight during
    // this batch's normalisation and multiplies; the scheduling barrier keeps
    // the normalisation (which waits for the fragments) after the issue.
    HTN_ISSUE(jb + W * kU);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const float inv = inv_s[t * 16 + col];
          av[u][t][0] = norm8(av[u][t][0], gv[u][0], inv);
          av[u][t][1] = norm8(av[u][t][1], gv[u][1], inv);
        }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int s = 0; s < S; ++s) {
          acc[t][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, av[u][t][0]), __builtin_bit_cast(bf16x8_t, bf[u][s][0]),
              acc[t][s], 0, 0, 0);
          acc[t][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, av[u][t][1]), __builtin_bit_cast(bf16x8_t, bf[u][s][1]),
              acc[t][s], 0, 0, 0);
        }
  }
#undef HTN_ISSUE

  // D layout: lane holds column (lane & 15), rows 4 * (lane >> 4) + i.
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][t][s][(quad * 4 + i) * kStrip + col] = acc[t][s][i];
  __syncthreads();

  // tid -> (row, column) of the strip; MT * 16 rows x 16 columns.
  for (int o = tid; o < MT * 16 * kStrip; o += W * 64) {
    const int m = o / kStrip, c = o % kStrip;
    const int t = m / 16, r = m % 16;
    float v[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float sum = 0.f;
#pragma unroll
      for (int ww = 0; ww < W; ++ww) sum += red[ww][t][s][r * kStrip + c];
      v[s] = sum;
    }
    const int n = n0 + c;
    if (EPI == HTN_EPI_ARGMAX) {
      if (m < a.M)
        best[m][c] = n < a.N ? argmax_key(f2bf(v[0]), static_cast<uint32_t>(n)) : 0ull;
      continue;
    }
    if (m >= a.M || n >= a.N) continue;
    if (a.KS > 1) {
#pragma unroll
      for (int s = 0; s < S; ++s)
        a.part[(static_cast<long>(ks) * a.M + m) * Nw + s * a.N + n] = v[s];
    } else {
      store_out<EPI>(a, m, n, v[0], S > 1 ? v[S - 1] : 0.f);
    }
  }
  if (EPI == HTN_EPI_ARGMAX) {
    __syncthreads();
    if (tid < a.M) {
      uint64_t b = best[tid][0];
      for (int c = 1; c < kStrip; ++c) b = best[tid][c] > b ? best[tid][c] : b;
      a.keys[static_cast<long>(strip) * a.M + tid] = b;
    }
  }
}

// Sum of the K-split partials in split order, then the epilogue.
template <int S, int EPI>
__global__ __launch_bounds__(kBlock) void gemm_rows_finish(RowsArgs a) {
  preload_rows(a);
  const long o = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x;
  if (o >= static_cast<long>(a.M) * a.N) return;
  const int m = static_cast<int>(o / a.N), n = static_cast<int>(o % a.N);
  const int Nw = S * a.N;
  float v[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    float t = 0.f;
    for (int ks = 0; ks < a.KS; ++ks) t += a.part[(static_cast<long>(ks) * a.M + m) * Nw + s * a.N + n];
    v[s] = t;
  }
  store_out<EPI>(a, m, n, v[0], S > 1 ? v[S - 1] : 0.f);
}

// K-split finish of the residual epilogue fused with the next RMSNorm: one
// block per row m. Its threads sum the partials of the row's 8-element
// vectors in split order, add the residual, round, and store y to memory and
// LDS; wave 0 then forms the sum of squares in the row-wise RMSNorm's order
// (lane l over vectors l, l + 64, ..., element by element, then one wave
// reduction), so `normed` is bit-identical to running that norm on y, and
// every thread normalises its vectors from LDS.
__global__ __launch_bounds__(kBlock) void gemm_rows_finish_norm(RowsArgs a) {
  preload_rows(a);
  asm volatile("" ::"s"(a.ngain), "s"(a.neps), "s"(a.normed));
  __shared__ uint4 ys[8192 / 8];  // the row of y, up to 8192 columns
  __shared__ float inv_s;
  const int tid = threadIdx.x;
  const int m = blockIdx.x;
  const int nv = a.N >> 3;
  for (int v = tid; v < nv; v += kBlock) {
    float t[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < a.KS; ++ks) {
      const float4* p =
          reinterpret_cast<const float4*>(a.part + (static_cast<long>(ks) * a.M + m) * a.N + v * 8);
      const float4 p0 = p[0], p1 = p[1];
      t[0] += p0.x; t[1] += p0.y; t[2] += p0.z; t[3] += p0.w;
      t[4] += p1.x; t[5] += p1.y; t[6] += p1.z; t[7] += p1.w;
    }
    float r[8];
    unpack8(*reinterpret_cast<const uint4*>(a.res + m * a.res_rs + v * 8), r);
    uint4 yv;
    yv.x = pack_bf2(round_bf(t[0]) + r[0], round_bf(t[1]) + r[1]);
    yv.y = pack_bf2(round_bf(t[2]) + r[2], round_bf(t[3]) + r[3]);
    yv.z = pack_bf2(round_bf(t[4]) + r[4], round_bf(t[5]) + r[5]);
    yv.w = pack_bf2(round_bf(t[6]) + r[6], round_bf(t[7]) + r[7]);
    *reinterpret_cast<uint4*>(a.y + m * a.y_rs + v * 8) = yv;
    ys[v] = yv;
  }
  __syncthreads();
  if (tid < kWave) {
    float ss = 0.f;
    for (int v = tid; v < nv; v += kWave) {
      float f[8];
      unpack8(ys[v], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(f[i], f[i], ss);
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / static_cast<float>(a.N) + a.neps);
    if (tid == 0) inv_s = inv;
  }
  __syncthreads();
  const float inv = inv_s;
  for (int v = tid; v < nv; v += kBlock) {
    float f[8], g[8];
    unpack8(ys[v], f);
    unpack8(*reinterpret_cast<const uint4*>(a.ngain + v * 8), g);
    uint4 o;
    o.x = pack_bf2(g[0] * round_bf(f[0] * inv), g[1] * round_bf(f[1] * inv));
    o.y = pack_bf2(g[2] * round_bf(f[2] * inv), g[3] * round_bf(f[3] * inv));
    o.z = pack_bf2(g[4] * round_bf(f[4] * inv), g[5] * round_bf(f[5] * inv));
    o.w = pack_bf2(g[6] * round_bf(f[6] * inv), g[7] * round_bf(f[7] * inv));
    *reinterpret_cast<uint4*>(a.normed + static_cast<long>(m) * a.N + v * 8) = o;
  }
}

// Per-row argmax over the strips' keys.
__global__ __launch_bounds__(kBlock) void gemm_rows_argmax(const uint64_t* __restrict__ keys,
                                                          int strips, int M, int64_t* tokens) {
  asm volatile("" ::"s"(keys), "s"(strips), "s"(M), "s"(tokens));
  __shared__ uint64_t wbest[4];
  const int m = blockIdx.x;
  uint64_t b = 0;
  for (int i = threadIdx.x; i < strips; i += kBlock) {
    const uint64_t k = keys[static_cast<long>(i) * M + m];
    b = k > b ? k : b;
  }
  b = wave_max_u64(b);
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t r = wbest[0];
    for (int i = 1; i < 4; ++i) r = wbest[i] > r ? wbest[i] : r;
    tokens[m] = static_cast<int64_t>(argmax_key_index(r));
  }
}

// ------------------------------------------------------------------ interleaved gate/up
// SwiGLU of x by a K-major weight w[K, 2I] whose row k holds (gate_i, up_i)
// pairs: w[k, 2i] = gate_i[k], w[k, 2i + 1] = up_i[k] (the reference's
// offline layout). A block owns a strip of 32 outputs, i.e. 128 contiguous
// bytes of every weight row; lane (c, q) = (lane & 15, lane >> 4) loads
// 8 bytes, (gate, up) of outputs 2c and 2c + 1, from each of the rows
// q*8 .. q*8 + 7 of a 32-row step, so every load instruction reads four whole
// 128-byte row segments. The eight words per lane regroup in registers into
// the B fragments of four MFMAs (gate and up of the even outputs 2c, and of
// the odd outputs 2c + 1: output tile t holds outputs 2c + t), with k
// q*8 .. q*8 + 7 in lane quad q of both operands. Waves take interleaved
// steps, reduce through LDS and finish as gemm_rows_kernel does (K-split
// partials in its [KS][M][2I] gate-then-up layout).
constexpr int kStepI = 32;     // k per step: one MFMA depth
constexpr int kStripI = 32;    // outputs per block: two 16-output tiles
constexpr int kUI = 2;         // steps in flight per wave

template <int MT, int W>
__global__ __launch_bounds__(W * 64) void gemm_rows_interleaved(RowsArgs a) {
  preload_rows(a);
  __shared__ float red[W][MT][4][16 * 16];  // [wave][row tile][tile t, gate/up][row][col]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int strip = blockIdx.x, ks = blockIdx.y;
  const int n0 = strip * kStripI;
  const int col = lane & 15, quad = lane >> 4;
  const int j0 = ks * a.steps_per_split;
  const int total_steps = a.K / kStepI;
  const int j1 = j0 + a.steps_per_split < total_steps ? j0 + a.steps_per_split : total_steps;

  // The lane's output pair (2c, 2c + 1), clamped to the last pair (a.N is
  // even; clamped lanes compute discarded outputs).
  const int pair = n0 + 2 * col < a.N ? n0 + 2 * col : a.N - 2;
  const long row_len = 2L * a.N;
  const bf16_t* wlane = a.w + static_cast<long>(quad) * 8 * row_len + 2L * pair;

  uint2 wv[kUI][8];
  auto issue = [&](int jb) {
#pragma unroll
    for (int u = 0; u < kUI; ++u) {
      int j = jb + u * W;
      j = j < j1 ? j : j1 - 1;
      const bf16_t* p = wlane + static_cast<long>(j) * kStepI * row_len;
#pragma unroll
      for (int r = 0; r < 8; ++r) wv[u][r] = *reinterpret_cast<const uint2*>(p + r * row_len);
    }
  };
  issue(j0 + wave);

  f32x4_t acc[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int f = 0; f < 4; ++f) acc[t][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int jb = j0 + wave; jb < j1; jb += W * kUI) {
    if (jb != j0 + wave) issue(jb);
#pragma unroll
    for (int u = 0; u < kUI; ++u) {
      const int j = jb + u * W;
      const bool ok = j < j1;
      const int k = (ok ? j : j1 - 1) * kStepI + quad * 8;
      uint4 av[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) av[t] = a_fragment(a, t * 16 + col, k, ok);
      // Fragments f = 2 * tile + (0 gate, 1 up): word x of row r holds
      // (gate, up) of output 2c, word y of output 2c + 1.
      uint4 b[4];
      uint32_t* bw = reinterpret_cast<uint32_t*>(b);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint2 lo = wv[u][2 * d], hi = wv[u][2 * d + 1];
        bw[0 * 4 + d] = (lo.x & 0xffffu) | (hi.x << 16);
        bw[1 * 4 + d] = (lo.x >> 16) | (hi.x & 0xffff0000u);
        bw[2 * 4 + d] = (lo.y & 0xffffu) | (hi.y << 16);
        bw[3 * 4 + d] = (lo.y >> 16) | (hi.y & 0xffff0000u);
      }
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int f = 0; f < 4; ++f)
          acc[t][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, av[t]), __builtin_bit_cast(bf16x8_t, b[f]), acc[t][f],
              0, 0, 0);
    }
  }

  // D layout: lane holds column (lane & 15), rows 4 * (lane >> 4) + i.
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][t][f][(quad * 4 + i) * 16 + col] = acc[t][f][i];
  __syncthreads();

  // tid -> (row m, strip output o); output o is column o >> 1 of tile o & 1.
  const int Nw = 2 * a.N;
  for (int idx = tid; idx < MT * 16 * kStripI; idx += W * 64) {
    const int m = idx / kStripI, o = idx % kStripI;
    const int t = m / 16, r = m % 16, tile = o & 1, c = o >> 1;
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int ww = 0; ww < W; ++ww) {
      g += red[ww][t][2 * tile][r * 16 + c];
      u += red[ww][t][2 * tile + 1][r * 16 + c];
    }
    const int n = n0 + o;
    if (m >= a.M || n >= a.N) continue;
    if (a.KS > 1) {
      a.part[(static_cast<long>(ks) * a.M + m) * Nw + n] = g;
      a.part[(static_cast<long>(ks) * a.M + m) * Nw + a.N + n] = u;
    } else {
      store_out<HTN_EPI_SWIGLU>(a, m, n, g, u);
    }
  }
}

// Waves per strip: enough for about 16 waves per CU, 4 to 16 per block, and
// at least two k steps per wave. K splits across blocks only when 16 waves
// per strip still leave the GPU under-filled.
int choose_waves(int strips, int K) {
  const long target = 16L * device_cus();
  int w = 4;
  while (w < kMaxWaves && static_cast<long>(strips) * w < target && (K / kStep) >= 4 * w) w *= 2;
  return w;
}

int choose_splits(int strips, int waves, int K) {
  const int steps = K / kStep;
  const long target = 16L * device_cus();
  int ks = static_cast<int>((target + static_cast<long>(strips) * waves - 1) /
                            (static_cast<long>(strips) * waves));
  const int max_ks = steps / (4 * waves) > 0 ? steps / (4 * waves) : 1;  // 4 steps per wave
  if (ks > max_ks) ks = max_ks;
  if (ks > 8) ks = 8;
  return ks < 1 ? 1 : ks;
}

template <int MT, int S, int EPI, int W, bool NORM>
int launch_w(RowsArgs& a, hipStream_t st) {
  const int strips = (a.N + kStrip - 1) / kStrip;
  hipLaunchKernelGGL((gemm_rows_kernel<MT, S, EPI, W, NORM>), dim3(strips, a.KS), dim3(W * 64), 0,
                     st, a);
  if (launch_status() != HTN_OK) return HTN_ELAUNCH;
  if (EPI == HTN_EPI_ARGMAX) {
    hipLaunchKernelGGL(gemm_rows_argmax, dim3(a.M), dim3(kBlock), 0, st, a.keys, strips, a.M, a.tokens);
  } else if (a.KS > 1 && EPI == HTN_EPI_RESIDUAL && a.normed) {
    hipLaunchKernelGGL(gemm_rows_finish_norm, dim3(a.M), dim3(kBlock), 0, st, a);
  } else if (a.KS > 1) {
    const long outs = static_cast<long>(a.M) * a.N;
    hipLaunchKernelGGL((gemm_rows_finish<S, EPI>), dim3((outs + kBlock - 1) / kBlock), dim3(kBlock),
                       0, st, a);
  }
  return launch_status();
}

// Most waves per block for MT row tiles: the per-wave reduction array
// (W * MT * S KB of LDS) stays within 64 KB.
constexpr int max_waves(int mt) { return mt <= 2 ? 16 : (mt == 4 ? 8 : 4); }

template <int MT, int S, int EPI, bool NORM = false>
int launch(RowsArgs& a, int waves, hipStream_t st) {
  if constexpr (max_waves(MT) >= 16) {
    if (waves >= 16) return launch_w<MT, S, EPI, 16, NORM>(a, st);
  }
  if constexpr (max_waves(MT) >= 8) {
    if (waves >= 8) return launch_w<MT, S, EPI, 8, NORM>(a, st);
  }
  return launch_w<MT, S, EPI, 4, NORM>(a, st);
}

// `norm`: the input rows are normalised inside the projection (store and
// SwiGLU epilogues only).
template <int MT>
int dispatch_epi(RowsArgs& a, int epi, bool norm, int waves, hipStream_t st) {
  if constexpr (MT <= 2) {  // the in-kernel norm covers at most 32 rows
    if (norm && epi == HTN_EPI_STORE) return launch<MT, 1, HTN_EPI_STORE, true>(a, waves, st);
    if (norm && epi == HTN_EPI_SWIGLU) return launch<MT, 2, HTN_EPI_SWIGLU, true>(a, waves, st);
  }
  switch (epi) {
    case HTN_EPI_STORE: return launch<MT, 1, HTN_EPI_STORE>(a, waves, st);
    case HTN_EPI_RESIDUAL: return launch<MT, 1, HTN_EPI_RESIDUAL>(a, waves, st);
    case HTN_EPI_SWIGLU: return launch<MT, 2, HTN_EPI_SWIGLU>(a, waves, st);
    default: return launch<MT, 1, HTN_EPI_ARGMAX>(a, waves, st);
  }
}

// Row tiles per block for `rows` activation rows.
int row_tiles(long rows) { return rows <= 16 ? 1 : (rows <= 32 ? 2 : (rows <= 64 ? 4 : 8)); }

// Input RMSNorm inside the projection: store and SwiGLU epilogues, at most 32
// rows (one or two per wave) of at most kNormVec * 512 elements. The greedy
// head keeps the one-launch pre-pass: its thousands of strips would each
// re-read every row.
bool norm_in_kernel(int epilogue, long rows, long k) {
  return (epilogue == HTN_EPI_STORE || epilogue == HTN_EPI_SWIGLU) && rows <= 32 &&
         k <= kNormVec * 512;
}

struct Plan {
  int waves, ks;
  long norm_bytes, tail_bytes;
};

Plan plan(long M, long N, long K, int epilogue, bool norm) {
  Plan p{};
  const int strips = static_cast<int>((N + kStrip - 1) / kStrip);
  p.waves = choose_waves(strips, static_cast<int>(K));
  const int mt = row_tiles(M);
  if (p.waves > max_waves(mt)) p.waves = max_waves(mt);
  p.ks = epilogue == HTN_EPI_ARGMAX ? 1 : choose_splits(strips, p.waves, static_cast<int>(K));
  // Residual projections of up to 32 rows keep K whole: without a split
  // finish the next projection normalises its rows in-kernel, one launch
  // fewer per layer (4B 5-row verify, down [2560, 9728]: 2.91 -> 2.81 ms).
  if (epilogue == HTN_EPI_RESIDUAL && mt <= 2) p.ks = 1;
  // Plain stores of up to 32 rows (the QKV projection of verify passes and
  // batched steps) run faster on 8 waves per strip than on 16, the K split
  // left as planned (8B QKV, 5 rows: 16.9 -> 15.6 us with the rows
  // normalised in-kernel, 13.4 -> 12.4 us without; 4B within 1%); four
  // waves were slower again (4B 5-row verify 2.80 -> 2.85 ms).
  if (epilogue == HTN_EPI_STORE && mt <= 2 && p.waves > 8) p.waves = 8;
  p.norm_bytes = norm && !norm_in_kernel(epilogue, M, K) ? align_up(M * K * 2) : 0;
  if (epilogue == HTN_EPI_ARGMAX) p.tail_bytes = static_cast<long>(strips) * M * 8;
  else if (p.ks > 1) p.tail_bytes = static_cast<long>(p.ks) * M * N * (epilogue == HTN_EPI_SWIGLU ? 2 : 1) * 4;
  return p;
}

// The fused residual + RMSNorm keeps the projection's own plan and fuses the
// norm into its K-split finish when it has one. Splitting K only to get a
// finish was measured slower (4B verify pass 3.79 -> 3.89 ms, 8B at 4 and 16
// rows 6-7% slower): the split projection loses more than the norm launch
// costs, and a 4096-wide row is too long for one wave's finish.
Plan plan_residual_norm(long M, long N, long K) { return plan(M, N, K, HTN_EPI_RESIDUAL, false); }

// The interleaved gate/up kernel's plan, by the same rule over 32-row steps
// and 32-output strips; two row tiles keep to 8 waves (64 KB of LDS).
Plan plan_interleaved(long M, long N, long K) {
  Plan p{};
  const long strips = (N + kStripI - 1) / kStripI;
  const long steps = K / kStepI;
  const long target = 16L * device_cus();
  const int max_w = M > 16 ? 8 : kMaxWaves;
  int w = 4;
  while (w < max_w && strips * w < target && steps >= 4L * w) w *= 2;
  long ks = (target + strips * w - 1) / (strips * w);
  const long max_ks = steps / (4L * w) > 0 ? steps / (4L * w) : 1;
  if (ks > max_ks) ks = max_ks;
  if (ks > 8) ks = 8;
  p.waves = w;
  p.ks = static_cast<int>(ks < 1 ? 1 : ks);
  p.tail_bytes = p.ks > 1 ? static_cast<long>(p.ks) * M * N * 2 * 4 : 0;
  return p;
}

template <int MT, int W>
int launch_interleaved_w(RowsArgs& a, hipStream_t st) {
  const int strips = (a.N + kStripI - 1) / kStripI;
  hipLaunchKernelGGL((gemm_rows_interleaved<MT, W>), dim3(strips, a.KS), dim3(W * 64), 0, st, a);
  if (launch_status() != HTN_OK) return HTN_ELAUNCH;
  if (a.KS > 1) {
    const long outs = static_cast<long>(a.M) * a.N;
    hipLaunchKernelGGL((gemm_rows_finish<2, HTN_EPI_SWIGLU>),
                       dim3((outs + kBlock - 1) / kBlock), dim3(kBlock), 0, st, a);
  }
  return launch_status();
}

template <int MT>
int launch_interleaved(RowsArgs& a, int waves, hipStream_t st) {
  if constexpr (MT == 1) {
    if (waves >= 16) return launch_interleaved_w<MT, 16>(a, st);
  }
  if (waves >= 8) return launch_interleaved_w<MT, 8>(a, st);
  return launch_interleaved_w<MT, 4>(a, st);
}

}  // namespace
}  // namespace htn

using namespace htn;

extern "C" int64_t htn_gemm_rows_scratch_bytes(int64_t rows, int64_t n, int64_t k, int epilogue,
                                               int norm) {
  if (rows <= 0 || rows > kMaxRowsMT || n <= 0 || k <= 0 || k % kStep || k > kMaxK) return 0;
  const Plan p = epilogue == HTN_EPI_RESIDUAL_NORM ? plan_residual_norm(rows, n, k)
                                                    : plan(rows, n, k, epilogue, norm != 0);
  return p.norm_bytes + p.tail_bytes;
}

extern "C" int htn_rms_norm(const void* x, int64_t x_row_stride, const void* gain, void* out,
                            int64_t rows, int64_t cols, float eps, htn_stream_t stream);

extern "C" int htn_gemm_rows(const void* x, int64_t x_stride, const void* gain, float eps,
                             const void* w, int64_t n, int64_t k, int64_t rows, int epilogue,
                             const void* residual, int64_t res_stride, void* y, int64_t y_stride,
                             int64_t* tokens, void* scratch, htn_stream_t stream) {
  if (!x || !w || rows <= 0 || rows > kMaxRowsMT || n <= 0 || k <= 0 || n > (1L << 31))
    return HTN_EINVAL;
  if (epilogue < HTN_EPI_STORE || epilogue > HTN_EPI_ARGMAX) return HTN_EINVAL;
  if (epilogue == HTN_EPI_ARGMAX ? !tokens : !y) return HTN_EINVAL;
  if (epilogue == HTN_EPI_RESIDUAL && !residual) return HTN_EINVAL;
  // Output and residual rows must not overlap.
  if (y && (y_stride < n || (epilogue == HTN_EPI_RESIDUAL && res_stride < n))) return HTN_EINVAL;
  // 16-byte fragments of x, gain and W rows.
  if (k % kStep || k > kMaxK || x_stride % 8 || !aligned16(x) || !aligned16(w) ||
      (gain && !aligned16(gain)))
    return HTN_EUNSUPPORTED;
  const Plan p = plan(rows, n, k, epilogue, gain != nullptr);
  if ((p.norm_bytes + p.tail_bytes) > 0 && !scratch) return HTN_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  RowsArgs a{};
  a.x = static_cast<const bf16_t*>(x); a.x_rs = x_stride;
  const bool inorm = gain && norm_in_kernel(epilogue, rows, k);
  if (inorm) {
    a.xgain = static_cast<const bf16_t*>(gain);
    a.xeps = eps;
  } else if (gain) {
    // Rows normalised once into the scratch buffer.
    bf16_t* xn = static_cast<bf16_t*>(scratch);
    const int rc = htn_rms_norm(x, x_stride, gain, xn, rows, k, eps, stream);
    if (rc != HTN_OK) return rc;
    a.x = xn;
    a.x_rs = k;
  }
  a.w = static_cast<const bf16_t*>(w);
  a.res = static_cast<const bf16_t*>(residual); a.res_rs = res_stride;
  a.y = static_cast<bf16_t*>(y); a.y_rs = y_stride;
  a.M = static_cast<int>(rows); a.N = static_cast<int>(n); a.K = static_cast<int>(k);
  a.KS = p.ks;
  const int steps = a.K / kStep;
  a.steps_per_split = (steps + a.KS - 1) / a.KS;
  void* tail = static_cast<char*>(scratch) + p.norm_bytes;
  a.part = static_cast<float*>(tail);
  a.keys = static_cast<uint64_t*>(tail);
  a.tokens = tokens;
  switch (row_tiles(rows)) {
    case 1: return dispatch_epi<1>(a, epilogue, inorm, p.waves, st);
    case 2: return dispatch_epi<2>(a, epilogue, inorm, p.waves, st);
    case 4: return dispatch_epi<4>(a, epilogue, inorm, p.waves, st);
    default: return dispatch_epi<8>(a, epilogue, inorm, p.waves, st);
  }
}

extern "C" int htn_gemm_rows_residual_norm(const void* x, int64_t x_stride, const void* w,
                                           int64_t n, int64_t k, int64_t rows,
                                           const void* residual, int64_t res_stride, void* y,
                                           int64_t y_stride, const void* gain, float eps,
                                           void* normed, void* scratch, htn_stream_t stream) {
  if (!x || !w || !residual || !y || !gain || !normed || rows <= 0 || rows > kMaxRowsMT ||
      n <= 0 || k <= 0 || n > (1L << 31))
    return HTN_EINVAL;
  if (y_stride < n || res_stride < n) return HTN_EINVAL;  // rows must not overlap
  if (k % kStep || k > kMaxK) return HTN_EUNSUPPORTED;
  const Plan p = plan_residual_norm(rows, n, k);
  // The finish holds a row of y in LDS: 8-element vectors, at most 8192 columns.
  const bool fused = p.ks > 1 && n % 8 == 0 && n <= 8192 && res_stride % 8 == 0 &&
                     y_stride % 8 == 0 && aligned16(residual) && aligned16(y) &&
                     aligned16(gain) && aligned16(normed);
  if (!fused) {
    // No K split to finish (or unaligned rows): the residual projection, then
    // the row-wise RMSNorm of its output.
    const int rc = htn_gemm_rows(x, x_stride, nullptr, 0.f, w, n, k, rows, HTN_EPI_RESIDUAL,
                                 residual, res_stride, y, y_stride, nullptr, scratch, stream);
    if (rc != HTN_OK) return rc;
    return htn_rms_norm(y, y_stride, gain, normed, rows, n, eps, stream);
  }
  if (k % kStep || k > kMaxK || x_stride % 8 || !aligned16(x) || !aligned16(w))
    return HTN_EUNSUPPORTED;
  if (!scratch) return HTN_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  RowsArgs a{};
  a.x = static_cast<const bf16_t*>(x); a.x_rs = x_stride;
  a.w = static_cast<const bf16_t*>(w);
  a.res = static_cast<const bf16_t*>(residual); a.res_rs = res_stride;
  a.y = static_cast<bf16_t*>(y); a.y_rs = y_stride;
  a.M = static_cast<int>(rows); a.N = static_cast<int>(n); a.K = static_cast<int>(k);
  a.KS = p.ks;
  a.steps_per_split = (a.K / kStep + a.KS - 1) / a.KS;
  a.part = static_cast<float*>(scratch);
  a.ngain = static_cast<const bf16_t*>(gain);
  a.neps = eps;
  a.normed = static_cast<bf16_t*>(normed);
  switch (row_tiles(rows)) {
    case 1: return launch<1, 1, HTN_EPI_RESIDUAL>(a, p.waves, st);
    case 2: return launch<2, 1, HTN_EPI_RESIDUAL>(a, p.waves, st);
    case 4: return launch<4, 1, HTN_EPI_RESIDUAL>(a, p.waves, st);
    default: return launch<8, 1, HTN_EPI_RESIDUAL>(a, p.waves, st);
  }
}

extern "C" int64_t htn_gate_up_swiglu_scratch_bytes(int64_t rows, int64_t width, int64_t k) {
  if (rows <= 0 || rows > kMaxRowsI || width <= 0 || width % 2 || k <= 0 || k % kStepI) return 0;
  return plan_interleaved(rows, width, k).tail_bytes;
}

extern "C" int htn_gate_up_swiglu(const void* x, int64_t x_stride, const void* w, int64_t width,
                                  int64_t k, int64_t rows, void* y, int64_t y_stride,
                                  void* scratch, htn_stream_t stream) {
  if (!x || !w || !y || rows <= 0 || rows > kMaxRowsI || width <= 0 || k <= 0 ||
      width > (1L << 30) || y_stride < width)
    return HTN_EINVAL;
  // 16-byte rows of x, 8-byte (gate, up) pairs of w; every step 32 rows of w.
  if (width % 2 || k % kStepI || k > (1L << 24) || x_stride % 8 || x_stride < k ||
      !aligned16(x) || !aligned8(w))
    return HTN_EUNSUPPORTED;
  const Plan p = plan_interleaved(rows, width, k);
  if (p.tail_bytes > 0 && !scratch) return HTN_EINVAL;
  RowsArgs a{};
  a.x = static_cast<const bf16_t*>(x); a.x_rs = x_stride;
  a.w = static_cast<const bf16_t*>(w);
  a.y = static_cast<bf16_t*>(y); a.y_rs = y_stride;
  a.M = static_cast<int>(rows); a.N = static_cast<int>(width); a.K = static_cast<int>(k);
  a.KS = p.ks;
  a.steps_per_split = (a.K / kStepI + a.KS - 1) / a.KS;
  a.part = static_cast<float*>(scratch);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows <= 16) return launch_interleaved<1>(a, p.waves, st);
  return launch_interleaved<2>(a, p.waves, st);
}
