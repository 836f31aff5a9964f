// Batch-one GEMV family for gfx950: norm/QKV, norm/gate-up/SwiGLU, O/down +
// residual, and the fused final-norm/LM-head/argmax greedy head.
//
// Design (HBM-bound, ~1 FLOP per weight byte):
//  * one wave64 owns R output rows (R gate/up row pairs for SwiGLU) and walks
//    the whole K extent, so the dot product finishes with one in-wave DPP
//    reduction and no LDS traffic;
//  * every lane issues 16-byte non-temporal loads, U chunks of 1 KB per row
//    in flight per wave (U * R * S loads per lane), so a CU holds tens of KB
//    of outstanding HBM reads;
//  * the activation row (optionally RMS-normalised, rounded exactly as the
//    reference) is staged once per block in LDS and read back with 16-byte
//    LDS reads;
//  * blocks grid-stride over row groups, so the prologue is paid once per
//    block and the grid is sized to the CU count;
//  * weight-only 8-bit variants (int8, fp8 e4m3fn) keep the same schedule with
//    16 weights per 16-byte load and apply the per-output-channel fp32 scale
//    to the fp32 dot product before the bf16 rounding.
#include "common.h"

namespace htn {

enum Epilogue { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };

// LDS layout: [0, 64) argmax keys of the four waves, [64, 128) reduction
// scratch, then the staged activation row.
constexpr int kLdsHead = 128;

struct GemvArgs {
  const bf16_t* x;
  const bf16_t* gain;
  const bf16_t* w;     // bf16 weights, or the bytes of an 8-bit format
  const float* scale;  // 8-bit formats: one fp32 scale per weight row
  const bf16_t* res;
  bf16_t* y;
  int64_t* token_out;
  int64_t* position_inc;
  uint64_t* partial;   // argmax: one key per block
  long n;              // output rows (gate rows for SwiGLU)
  int k;
  float eps;
};

__device__ __forceinline__ float silu_mul(float g, float u) {
  return silu_bf(g) * u;  // bf16(silu(g)) * u; the caller rounds the product
}

// Greedy head, stage 1: the block's best (logit, id) key goes to its own slot
// of the partial array. A separate one-block kernel reduces the slots: an
// in-kernel cross-block completion would need an agent-scope release per
// block, which writes back L2 and costs far more than one extra launch.
__device__ __forceinline__ void argmax_block(const GemvArgs& a, uint64_t best, uint64_t* keys) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) keys[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = keys[0];
    for (int i = 1; i < kBlock / kWave; ++i) b = keys[i] > b ? keys[i] : b;
    a.partial[blockIdx.x] = b;
  }
}

// Greedy head, stage 2: one block reduces the per-block keys, publishes the
// token and (decode step) advances the position.
__global__ __launch_bounds__(kBlock) void argmax_finish(const uint64_t* __restrict__ partial, int n,
                                                       int64_t* token_out, int64_t* position_inc) {
  asm volatile("" ::"s"(partial), "s"(n), "s"(token_out), "s"(position_inc));
  __shared__ uint64_t keys[4];
  uint64_t best = 0;
  for (int i = threadIdx.x; i < n; i += kBlock) best = partial[i] > best ? partial[i] : best;
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) keys[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = keys[0];
    for (int i = 1; i < 4; ++i) b = keys[i] > b ? keys[i] : b;
    token_out[0] = static_cast<int64_t>(argmax_key_index(b));
    if (position_inc) position_inc[0] += 1;
  }
}

// Weight batch: chunks c0 .. c0+U-1 of output rows n0 .. n0+R-1 (for SwiGLU
// each is the pair gate row n, up row n + N). Lane l reads 16 bytes at vector
// c*64 + l of each row through a buffer descriptor over that row, so vectors
// past the row's end read zeros without a per-lane branch; rows past the end
// re-read the last row (discarded). n0 is wave-uniform. A batch that is not
// `live` (past the wave's last row) gets empty descriptors: its loads return
// zeros without touching memory, so the issue needs no branch.
template <int R, int S, int U, int WF>
__device__ __forceinline__ void issue_batch(const GemvArgs& a, long n0, int c0, int lane,
                                            bool live, uint4 (&wv)[U][R][S]) {
  const unsigned char* base = reinterpret_cast<const unsigned char*>(a.w);
  const uint32_t row_bytes = static_cast<uint32_t>(a.k) * Fmt<WF>::kBytes;
  const uint32_t range = live ? row_bytes : 0u;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long n = n0 + r < a.n ? n0 + r : a.n - 1;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const __amdgpu_buffer_rsrc_t rs =
          buffer_rsrc(base + (n + s * a.n) * static_cast<long>(row_bytes), range);
#pragma unroll
      for (int u = 0; u < U; ++u)
        wv[u][r][s] = buffer_load16_stream(rs, static_cast<uint32_t>(lane) * 16,
                                           static_cast<uint32_t>(c0 + u) * 64 * 16);
    }
  }
}

// Per-row epilogue operands (8-bit row scales, the residual), loaded with the
// row's first weight batch so the epilogue never waits on a fresh load.
template <int R, int S, int EPI, int WF>
__device__ __forceinline__ void issue_epilogue(const GemvArgs& a, long n0, float (&sc)[R][S],
                                               float (&rs)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long n = n0 + r < a.n ? n0 + r : a.n - 1;
    if constexpr (WF != WF_BF16) {
      sc[r][0] = a.scale[n];
      if (S > 1) sc[r][S - 1] = a.scale[n + a.n];
    }
    if constexpr (EPI == EPI_RESIDUAL) rs[r] = bf2f(a.res[n]);
  }
}

// RMSNorm operands held in registers for rows up to kNormVecs * 8 * kBlock
// elements (8192): each thread loads its x and gain vectors once.
constexpr int kNormVecs = 4;

__device__ __forceinline__ void pin4(uint4& v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}

// One wave per output row (row pair for SwiGLU), rows grid-strided over
// persistent blocks. Lane l only ever multiplies activation vectors c*64 + l:
// without the RMSNorm prologue they are loaded next to each weight batch (L1
// hits after the CU's first wave) and the waves never synchronise; with it the
// block normalises x once into LDS, amortised over all rows the block streams.
template <int R, int S, int U, bool NORM, int EPI, int WF>
__global__ __launch_bounds__(kBlock) void gemv_vec(GemvArgs a) {
  constexpr int EPV = Fmt<WF>::kPerVec;  // weights (and activations) per lane per vector
  __shared__ uint64_t keys[kBlock / kWave];
  __shared__ float red[kBlock / kWave];
  extern __shared__ __align__(16) unsigned char smem[];
  bf16_t* xs = reinterpret_cast<bf16_t*>(smem);   // normalised x (NORM only)
  // The wave index is uniform: readfirstlane keeps row addresses in SGPRs.
  const int lane = threadIdx.x & 63;
  // Every kernel argument (and the grid size, a hidden argument) in scalar
  // registers before anything uses them: one round of scalar loads instead
  // of two.
  asm volatile("" ::"s"(a.w), "s"(a.x), "s"(a.y), "s"(a.n), "s"(a.k), "s"(gridDim.x));
  if constexpr (NORM) asm volatile("" ::"s"(a.gain), "s"(a.eps));
  if constexpr (EPI == EPI_RESIDUAL) asm volatile("" ::"s"(a.res));
  if constexpr (WF != WF_BF16) asm volatile("" ::"s"(a.scale));
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kv = a.k / EPV;
  const int chunks = (kv + 63) >> 6;
  const long groups = (a.n + R - 1) / R;
  const long stride = static_cast<long>(gridDim.x) * 4;
  long grp = static_cast<long>(blockIdx.x) * 4 + wave;
  const int kv8 = a.k >> 3;

  // RMSNorm operands first: vector loads complete in issue order, so loading
  // x and the gain ahead of the weights lets the prologue start as soon as
  // they arrive instead of after the first weight batch.
  // Every load before the first wait is unconditional: a branch that joins
  // with fewer loads in flight makes the compiler wait for all of them.
  uint4 xr[NORM ? kNormVecs : 1], gr[NORM ? kNormVecs : 1];
  const bool norm_regs = NORM && a.k <= kNormVecs * 8 * kBlock;
  if constexpr (NORM) {
    const uint32_t bytes = static_cast<uint32_t>(a.k) * 2;
    const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(a.x, bytes), grs = buffer_rsrc(a.gain, bytes);
#pragma unroll
    for (int i = 0; i < kNormVecs; ++i) {
      xr[i] = buffer_load16(xrs, (threadIdx.x + i * kBlock) * 16, 0);
      gr[i] = buffer_load16(grs, (threadIdx.x + i * kBlock) * 16, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the weights
  }

  // First weight batch before anything that waits on memory.
  uint4 wv[U][R][S];
  issue_batch<R, S, U, WF>(a, grp * R, 0, lane, grp < groups, wv);

  // RMSNorm prologue: the block normalises x once into LDS (bf16, rounded as
  // the reference rounds) and its waves then stream many rows against it.
  if constexpr (NORM) {
    float ss = 0.f;
    if (norm_regs) {
      // The empty volatile asm keeps the arithmetic (and its wait) after the
      // weight loads above.
#pragma unroll
      for (int i = 0; i < kNormVecs; ++i) {
        pin4(xr[i]);
        pin4(gr[i]);
        float f[8];
        unpack8(xr[i], f);  // vectors past the row read as zeros
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fmaf(f[j], f[j], ss);
      }
    } else {
      for (int v = threadIdx.x; v < kv8; v += kBlock) {
        float f[8];
        unpack8(*reinterpret_cast<const uint4*>(a.x + v * 8), f);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = fmaf(f[i], f[i], ss);
      }
    }
    const float inv = 1.0f / sqrtf(block_sum(ss, red) / static_cast<float>(a.k) + a.eps);
    if (norm_regs) {
#pragma unroll
      for (int i = 0; i < kNormVecs; ++i) {
        const int v = threadIdx.x + i * kBlock;
        if (v < kv8) *reinterpret_cast<uint4*>(xs + v * 8) = norm8(xr[i], gr[i], inv);
      }
    } else {
      for (int v = threadIdx.x; v < kv8; v += kBlock)
        *reinterpret_cast<uint4*>(xs + v * 8) =
            norm8(*reinterpret_cast<const uint4*>(a.x + v * 8),
                  *reinterpret_cast<const uint4*>(a.gain + v * 8), inv);
    }
    __syncthreads();
  }

  // Software pipeline: each wave keeps exactly one weight batch in flight.
  // The batch after the one being multiplied (the row's next chunks, or the
  // first chunks of the wave's next row) is issued right after the
  // multiply, so it is in flight during the row's reduction and epilogue.
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(a.x, static_cast<uint32_t>(a.k) * 2);
  uint64_t best = 0;
  for (; grp < groups; grp += stride) {
    const long n0 = grp * R;
    const long next = grp + stride;
    // The row's epilogue operands, behind its first weight batch and ahead
    // of the activations the multiply waits for.
    float sc[R][S], rs[R];
    issue_epilogue<R, S, EPI, WF>(a, n0, sc, rs);
    float acc[R][S];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int s = 0; s < S; ++s) acc[r][s] = 0.f;
    // do-while: the compiler then knows a row issues loads after its
    // epilogue operands, so the epilogue waits for those operands only.
    int c0 = 0;
    do {
      uint4 xv[U][EPV / 8];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int v = (c0 + u) * 64 + lane;
        if constexpr (NORM) {
#pragma unroll
          for (int h = 0; h < EPV / 8; ++h)
            xv[u][h] = v < kv ? *reinterpret_cast<const uint4*>(xs + v * EPV + 8 * h)
                              : make_uint4(0, 0, 0, 0);
        } else {
          // Activations through a descriptor over x: vectors past the row
          // read zeros (no per-lane branch).
#pragma unroll
          for (int h = 0; h < EPV / 8; ++h)
            xv[u][h] = buffer_load16(xrs, static_cast<uint32_t>(v) * EPV * 2 + 16 * h, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        uint32_t xp[EPV / 2];
#pragma unroll
        for (int h = 0; h < EPV / 8; ++h) {
          xp[4 * h] = xv[u][h].x;
          xp[4 * h + 1] = xv[u][h].y;
          xp[4 * h + 2] = xv[u][h].z;
          xp[4 * h + 3] = xv[u][h].w;
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int s = 0; s < S; ++s) acc[r][s] = dot_vec<WF>(wv[u][r][s], xp, acc[r][s]);
      }
      const bool last = c0 + U >= chunks;
      const long ng = last ? next : grp;
      issue_batch<R, S, U, WF>(a, ng * R, last ? 0 : c0 + U, lane, ng < groups, wv);
      c0 += U;
    } while (c0 < chunks);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const long n = n0 + r;
      float t0 = wave_sum(acc[r][0]);
      float t1 = S > 1 ? wave_sum(acc[r][S - 1]) : 0.f;
      if (n < a.n) {
        if (WF != WF_BF16) {
          t0 *= sc[r][0];
          if (S > 1) t1 *= sc[r][S - 1];
        }
        if (EPI == EPI_ARGMAX) {
          const uint64_t key = argmax_key(f2bf(t0), static_cast<uint32_t>(n));
          best = key > best ? key : best;
        } else if (lane == 0) {
          float out;
          if (EPI == EPI_STORE) {
            out = t0;
          } else if (EPI == EPI_RESIDUAL) {
            out = round_bf(t0) + rs[r];
          } else {
            out = silu_mul(round_bf(t0), round_bf(t1));
          }
          a.y[n] = static_cast<bf16_t>(f2bf(out));
        }
      }
    }
  }
  if (EPI == EPI_ARGMAX) argmax_block(a, best, keys);
}

// Generic fallback for row lengths that are not a multiple of 8 or unaligned
// pointers: scalar loads, one wave per row. Same epilogues and rounding.
template <bool NORM, int EPI>
__global__ __launch_bounds__(kBlock) void gemv_scalar(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* keys = reinterpret_cast<uint64_t*>(smem);
  float* red = reinterpret_cast<float*>(smem + 64);
  float* xs = reinterpret_cast<float*>(smem + kLdsHead);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float ss = 0.f;
  for (int i = tid; i < a.k; i += kBlock) {
    const float f = bf2f(a.x[i]);
    xs[i] = f;
    ss = fmaf(f, f, ss);
  }
  if (NORM) {
    const float total = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(total / static_cast<float>(a.k) + a.eps);
    for (int i = tid; i < a.k; i += kBlock) xs[i] = round_bf(bf2f(a.gain[i]) * round_bf(xs[i] * inv));
  }
  __syncthreads();
  uint64_t best = 0;
  const int S = EPI == EPI_SWIGLU ? 2 : 1;
  for (long n = static_cast<long>(blockIdx.x) * 4 + wave; n < a.n; n += static_cast<long>(gridDim.x) * 4) {
    float acc0 = 0.f, acc1 = 0.f;
    const bf16_t* r0 = a.w + n * static_cast<long>(a.k);
    const bf16_t* r1 = a.w + (n + a.n) * static_cast<long>(a.k);
    for (int i = lane; i < a.k; i += kWave) {
      acc0 = fmaf(bf2f(r0[i]), xs[i], acc0);
      if (S > 1) acc1 = fmaf(bf2f(r1[i]), xs[i], acc1);
    }
    const float t0 = wave_sum(acc0);
    const float t1 = wave_sum(acc1);
    if (EPI == EPI_ARGMAX) {
      const uint64_t key = argmax_key(f2bf(t0), static_cast<uint32_t>(n));
      best = key > best ? key : best;
    } else if (lane == 0) {
      float out;
      if (EPI == EPI_STORE) out = t0;
      else if (EPI == EPI_RESIDUAL) out = round_bf(t0) + bf2f(a.res[n]);
      else out = silu_mul(round_bf(t0), round_bf(t1));
      a.y[n] = static_cast<bf16_t>(f2bf(out));
    }
  }
  if (EPI == EPI_ARGMAX) argmax_block(a, best, keys);
}

// Row-wise argmax over materialised bf16 logits: one block per row.
__global__ __launch_bounds__(kBlock) void argmax_rows(const bf16_t* logits, long n, int64_t* out) {
  __shared__ uint64_t keys[4];
  const long row = blockIdx.x;
  const bf16_t* p = logits + row * n;
  uint64_t best = 0;
  for (long i = threadIdx.x; i < n; i += kBlock) {
    const uint64_t key = argmax_key(p[i], static_cast<uint32_t>(i));
    best = key > best ? key : best;
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) keys[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = keys[0];
    for (int i = 1; i < 4; ++i) b = keys[i] > b ? keys[i] : b;
    out[row] = static_cast<int64_t>(argmax_key_index(b));
  }
}

// ------------------------------------------------------------------ host dispatch

namespace {

constexpr int kMaxK = 16384;

constexpr long kMaxBlocks = HTN_HEAD_SCRATCH_BYTES / 8;

long grid_for(long groups, long per_cu) {
  long blocks = (groups + 3) / 4;
  long cap = static_cast<long>(device_cus()) * per_cu;
  if (cap > kMaxBlocks) cap = kMaxBlocks;
  blocks = blocks < cap ? blocks : cap;
  return blocks < 1 ? 1 : blocks;
}

int finish_argmax(const GemvArgs& a, long blocks, hipStream_t st) {
  if (launch_status() != HTN_OK) return HTN_ELAUNCH;
  hipLaunchKernelGGL(argmax_finish, dim3(1), dim3(kBlock), 0, st, a.partial,
                     static_cast<int>(blocks), a.token_out, a.position_inc);
  return launch_status();
}

// Waves resident per CU at full occupancy of 4 blocks (16 waves).
constexpr long kWavesPerCu = 16;

// Blocks per CU for a grid-stride GEMV over `groups` row groups (four waves
// a block). bf16 residual projections and RMSNorm + gate/up whose row
// groups divide evenly over the CUs take the blocks per CU that give every
// wave the same whole number of groups, two for the residual projections
// (each wave's second row issued while the first is reduced) and three for
// gate/up: the 8B decode step's O, down and gate/up (4096, 4096 and 12288
// groups on 256 CUs) measured 2.89 -> 2.85 ms per step against four, four
// and two blocks per CU. Other shapes keep the defaults: plain and residual
// kernels fill the CU (eight blocks); RMSNorm kernels pay their prologue
// once per block, so two longer-lived blocks per CU beat four (measured from
// 3072 to 151936 row groups: e.g. the 6144-row, K = 4096 QKV projection
// takes 9.9 us at two, 10.6 us at four, and three, two rows per wave, made
// the 8B step 2.831 -> 2.847 ms); 8-bit rows are half as long, so a
// wave holds half the bytes in flight: their norm kernels keep four blocks
// per CU (eight for 1 KB rows).
long blocks_per_cu(long groups, bool norm, int epi, int wf, long k) {
  if (wf == WF_BF16 && (epi == EPI_RESIDUAL ? !norm : (norm && epi == EPI_SWIGLU))) {
    const long want = epi == EPI_RESIDUAL ? 2 : 3;
    const long cus = device_cus();
    for (long pc = 1; pc <= 8; pc *= 2)
      if (groups == pc * 4 * cus * want) return pc;
  }
  if (norm) return wf == WF_BF16 ? 2 : (k > 1024 ? 4 : 8);
  return 8;
}

template <int R, int S, int U, bool NORM, int EPI, int WF>
int launch_vec(const GemvArgs& a, hipStream_t st) {
  const long groups = (a.n + R - 1) / R;
  const long blocks = grid_for(groups, blocks_per_cu(groups, NORM, EPI, WF, a.k));
  const size_t lds = NORM ? static_cast<size_t>(a.k) * 2 : 0;
  hipLaunchKernelGGL((gemv_vec<R, S, U, NORM, EPI, WF>), dim3(blocks), dim3(kBlock), lds, st, a);
  if (EPI == EPI_ARGMAX) return finish_argmax(a, blocks, st);
  return launch_status();
}

template <bool NORM, int EPI>
int launch_scalar(const GemvArgs& a, hipStream_t st) {
  const long blocks = grid_for(a.n, 4);
  const size_t lds = static_cast<size_t>(a.k) * 4 + kLdsHead;
  hipLaunchKernelGGL((gemv_scalar<NORM, EPI>), dim3(blocks), dim3(kBlock), lds, st, a);
  if (EPI == EPI_ARGMAX) return finish_argmax(a, blocks, st);
  return launch_status();
}

// One output row (gate/up pair for SwiGLU) per wave by default, so even
// 1024-row projections spread over every CU, with U 1 KB chunks per row in
// flight. Short rows (K <= 1024 bf16 weights) over many rows take four rows
// per wave so a wave still keeps 8 KB of loads in flight. 8-bit weights need
// 16-weight-aligned rows and have no scalar fallback.
template <bool NORM, int EPI, int WF>
int dispatch(GemvArgs& a, hipStream_t st) {
  constexpr int EPV = Fmt<WF>::kPerVec;
  const bool vec = (a.k % EPV == 0) && aligned16(a.x) && aligned16(a.w) &&
                   (!NORM || aligned16(a.gain));
  if (!vec) {
    if constexpr (WF == WF_BF16) return launch_scalar<NORM, EPI>(a, st);
    else return HTN_EUNSUPPORTED;
  }
  const int chunks = (a.k / EPV + 63) / 64;
  constexpr int S = EPI == EPI_SWIGLU ? 2 : 1;
  const bool many_rows = a.n >= 4 * kWavesPerCu * device_cus();
  if constexpr (WF != WF_BF16) {
    // 8-bit rows of one 1 KB chunk take one load per row, four rows per wave
    // when there are rows enough; rows longer than 8 KB stream two at a time,
    // 12 KB rows (the 8B down projection) in one batch per row pair (int8
    // 13.95 -> 12.71 us, fp8 12.50 -> 12.02 us: two batches per wave left the
    // second one's latency exposed).
    if (chunks == 1) {
      if (S == 1 && many_rows) return launch_vec<4, S, 1, NORM, EPI, WF>(a, st);
      return launch_vec<1, S, 1, NORM, EPI, WF>(a, st);
    }
    if constexpr (S == 1 && !NORM) {
      if (chunks == 12) return launch_vec<2, S, 12, NORM, EPI, WF>(a, st);
      if (chunks > 8) return launch_vec<2, S, 8, NORM, EPI, WF>(a, st);
    }
  }
  if (chunks <= 2) {
    if (S == 1 && many_rows) return launch_vec<4, S, 2, NORM, EPI, WF>(a, st);
    if constexpr (NORM && WF == WF_BF16) {
      // RMSNorm projections of rows this short (the 0.6B QKV and gate/up,
      // 2 KB rows) take four rows or row pairs per wave whenever every CU
      // still gets a block, so a CU keeps 64 KB in flight instead of 16
      // (0.6B step 0.662 -> 0.643 ms; one row pair more or fewer, or eight
      // rows, measured slower).
      if (a.n >= 4L * device_cus()) return launch_vec<4, S, 2, NORM, EPI, WF>(a, st);
    }
    return launch_vec<1, S, 2, NORM, EPI, WF>(a, st);
  }
  if (chunks <= 4) return launch_vec<1, S, 4, NORM, EPI, WF>(a, st);
  return launch_vec<1, S, 8, NORM, EPI, WF>(a, st);
}

}  // namespace

bool gemv_plain_layout(long n, long k, int format, long* blocks, int* rows) {
  const int epv = format == WF_BF16 ? Fmt<WF_BF16>::kPerVec : Fmt<WF_INT8>::kPerVec;
  if (n <= 0 || k <= 0 || k > kMaxK || k % epv != 0) return false;
  // Mirrors dispatch() for the residual epilogue (S = 1, no prologue).
  const int chunks = static_cast<int>((k / epv + 63) / 64);
  const bool many_rows = n >= 4 * kWavesPerCu * device_cus();
  int r = 1;
  if (format != WF_BF16 && chunks == 1) r = many_rows ? 4 : 1;
  else if (format != WF_BF16 && chunks > 8) r = 2;
  else if (chunks <= 2) r = many_rows ? 4 : 1;
  *blocks = grid_for((n + r - 1) / r, blocks_per_cu((n + r - 1) / r, false, EPI_RESIDUAL, format, k));
  *rows = 4 * r;
  return true;
}

namespace {

bool bad_sizes(int64_t n, int64_t k) { return n <= 0 || k <= 0 || k > kMaxK || n > (1L << 31); }

bool bad_format(int format) { return format != WF_INT8 && format != WF_FP8; }

// Runs dispatch<NORM, EPI, WF> for the runtime weight format.
template <bool NORM, int EPI>
int dispatch_w8(GemvArgs& a, int format, hipStream_t st) {
  return format == WF_INT8 ? dispatch<NORM, EPI, WF_INT8>(a, st) : dispatch<NORM, EPI, WF_FP8>(a, st);
}

}  // namespace
}  // namespace htn

using namespace htn;

extern "C" int htn_gemv(const void* x, const void* w, void* y, int64_t rows, int64_t k,
                        htn_stream_t stream) {
  if (!x || !w || !y || bad_sizes(rows, k)) return HTN_EINVAL;
  GemvArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.w = static_cast<const bf16_t*>(w);
  a.y = static_cast<bf16_t*>(y);
  a.n = rows;
  a.k = static_cast<int>(k);
  return dispatch<false, EPI_STORE, WF_BF16>(a, static_cast<hipStream_t>(stream));
}

extern "C" int htn_gemv_norm(const void* x, const void* gain, float eps, const void* w,
                             void* y, int64_t rows, int64_t k, int swiglu,
                             htn_stream_t stream) {
  if (!x || !gain || !w || !y || bad_sizes(rows, k)) return HTN_EINVAL;
  GemvArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.gain = static_cast<const bf16_t*>(gain);
  a.w = static_cast<const bf16_t*>(w);
  a.y = static_cast<bf16_t*>(y);
  a.n = rows;
  a.k = static_cast<int>(k);
  a.eps = eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return swiglu ? dispatch<true, EPI_SWIGLU, WF_BF16>(a, st) : dispatch<true, EPI_STORE, WF_BF16>(a, st);
}

extern "C" int htn_gemv_residual(const void* x, const void* w, const void* residual, void* y,
                                 int64_t rows, int64_t k, htn_stream_t stream) {
  if (!x || !w || !residual || !y || bad_sizes(rows, k)) return HTN_EINVAL;
  GemvArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.w = static_cast<const bf16_t*>(w);
  a.res = static_cast<const bf16_t*>(residual);
  a.y = static_cast<bf16_t*>(y);
  a.n = rows;
  a.k = static_cast<int>(k);
  return dispatch<false, EPI_RESIDUAL, WF_BF16>(a, static_cast<hipStream_t>(stream));
}

extern "C" int htn_lm_head_argmax(const void* x, const void* gain, float eps, const void* w,
                                  int64_t vocab, int64_t k, int64_t* token_out,
                                  int64_t* position_inc, void* scratch, htn_stream_t stream) {
  if (!x || !w || !token_out || !scratch || bad_sizes(vocab, k)) return HTN_EINVAL;
  GemvArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.gain = static_cast<const bf16_t*>(gain);
  a.w = static_cast<const bf16_t*>(w);
  a.n = vocab;
  a.k = static_cast<int>(k);
  a.eps = eps;
  a.token_out = token_out;
  a.position_inc = position_inc;
  a.partial = static_cast<uint64_t*>(scratch);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return gain ? dispatch<true, EPI_ARGMAX, WF_BF16>(a, st) : dispatch<false, EPI_ARGMAX, WF_BF16>(a, st);
}

extern "C" int htn_gemv_w8(const void* x, const void* w, const float* scales, int format,
                           void* y, int64_t rows, int64_t k, htn_stream_t stream) {
  if (!x || !w || !scales || !y || bad_sizes(rows, k) || bad_format(format)) return HTN_EINVAL;
  GemvArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.w = static_cast<const bf16_t*>(w);
  a.scale = scales;
  a.y = static_cast<bf16_t*>(y);
  a.n = rows;
  a.k = static_cast<int>(k);
  return dispatch_w8<false, EPI_STORE>(a, format, static_cast<hipStream_t>(stream));
}

extern "C" int htn_gemv_norm_w8(const void* x, const void* gain, float eps, const void* w,
                                const float* scales, int format, void* y, int64_t rows,
                                int64_t k, int swiglu, htn_stream_t stream) {
  if (!x || !gain || !w || !scales || !y || bad_sizes(rows, k) || bad_format(format))
    return HTN_EINVAL;
  GemvArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.gain = static_cast<const bf16_t*>(gain);
  a.w = static_cast<const bf16_t*>(w);
  a.scale = scales;
  a.y = static_cast<bf16_t*>(y);
  a.n = rows;
  a.k = static_cast<int>(k);
  a.eps = eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return swiglu ? dispatch_w8<true, EPI_SWIGLU>(a, format, st)
                : dispatch_w8<true, EPI_STORE>(a, format, st);
}

extern "C" int htn_gemv_residual_w8(const void* x, const void* w, const float* scales, int format,
                                    const void* residual, void* y, int64_t rows, int64_t k,
                                    htn_stream_t stream) {
  if (!x || !w || !scales || !residual || !y || bad_sizes(rows, k) || bad_format(format))
    return HTN_EINVAL;
  GemvArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.w = static_cast<const bf16_t*>(w);
  a.scale = scales;
  a.res = static_cast<const bf16_t*>(residual);
  a.y = static_cast<bf16_t*>(y);
  a.n = rows;
  a.k = static_cast<int>(k);
  return dispatch_w8<false, EPI_RESIDUAL>(a, format, static_cast<hipStream_t>(stream));
}

extern "C" int htn_lm_head_argmax_w8(const void* x, const void* gain, float eps, const void* w,
                                     const float* scales, int format, int64_t vocab, int64_t k,
                                     int64_t* token_out, int64_t* position_inc, void* scratch,
                                     htn_stream_t stream) {
  if (!x || !w || !scales || !token_out || !scratch || bad_sizes(vocab, k) || bad_format(format))
    return HTN_EINVAL;
  GemvArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.gain = static_cast<const bf16_t*>(gain);
  a.w = static_cast<const bf16_t*>(w);
  a.scale = scales;
  a.n = vocab;
  a.k = static_cast<int>(k);
  a.eps = eps;
  a.token_out = token_out;
  a.position_inc = position_inc;
  a.partial = static_cast<uint64_t*>(scratch);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return gain ? dispatch_w8<true, EPI_ARGMAX>(a, format, st)
              : dispatch_w8<false, EPI_ARGMAX>(a, format, st);
}

extern "C" int htn_argmax_bf16(const void* logits, int64_t rows, int64_t n, int64_t* out,
                               htn_stream_t stream) {
  if (!logits || !out || rows <= 0 || n <= 0 || rows > (1L << 31) || n > (1L << 31))
    return HTN_EINVAL;
  hipLaunchKernelGGL(argmax_rows, dim3(rows), dim3(kBlock), 0, static_cast<hipStream_t>(stream),
                     static_cast<const bf16_t*>(logits), static_cast<long>(n), out);
  return launch_status();
}

// ------------------------------------------------------------------ allocation-free greedy head
//
// htn_lm_head_argmax_noalloc: htn_lm_head_argmax with its per-block keys in a
// fixed device array instead of a caller buffer, for callers that cannot
// allocate device memory. Every GPU the library runs on holds its own copy of
// the array (HTN_HEAD_SCRATCH_BYTES, the most keys the head's grid writes)
// until the process ends. Host code never passes the array's name to a
// kernel: on the host it is only a stand-in for the symbol, so the device
// address is looked up once per device with hipGetSymbolAddress and kept.

static __device__ __align__(256) uint64_t htn_head_scratch[HTN_HEAD_SCRATCH_BYTES / 8];

#include <mutex>

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_head_scratch_mu;
void* g_head_scratch_ptr[kMaxDevices] = {};

// Device address of htn_head_scratch on `device`, resolved on the first call
// for that device with the device current; nullptr on failure.
void* head_scratch_on(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_head_scratch_mu);
  if (!g_head_scratch_ptr[device]) {
    int current = -1;
    if (hipGetDevice(&current) != hipSuccess) return nullptr;
    if (current != device && hipSetDevice(device) != hipSuccess) return nullptr;
    void* p = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(htn_head_scratch));
    const bool restored = current == device || hipSetDevice(current) == hipSuccess;
    if (rc != hipSuccess || !p || !restored) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_head_scratch_ptr[device] = p;
  }
  return g_head_scratch_ptr[device];
}

}  // namespace

extern "C" int64_t htn_head_scratch_capacity(void) { return HTN_HEAD_SCRATCH_BYTES; }

extern "C" int htn_lm_head_argmax_noalloc(const void* x, const void* gain, float eps,
                                          const void* w, int64_t vocab, int64_t k,
                                          int64_t* token_out, int64_t* position_inc,
                                          htn_stream_t stream) {
  if (!x || !w || !token_out || bad_sizes(vocab, k)) return HTN_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int device = -1;
  if (st) {
    if (hipStreamGetDevice(st, &device) != hipSuccess) return HTN_EINVAL;
  } else if (hipGetDevice(&device) != hipSuccess) {
    return HTN_ELAUNCH;
  }
  void* scratch = head_scratch_on(device);
  if (!scratch) return HTN_ELAUNCH;
  // The head's grid never exceeds kMaxBlocks keys (grid_for caps it), which
  // is exactly the array's size; the check keeps that bound explicit.
  static_assert(kMaxBlocks * 8 <= static_cast<long>(sizeof(htn_head_scratch)),
                "greedy-head grid exceeds the fixed key array");
  GemvArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.gain = static_cast<const bf16_t*>(gain);
  a.w = static_cast<const bf16_t*>(w);
  a.n = vocab;
  a.k = static_cast<int>(k);
  a.eps = eps;
  a.token_out = token_out;
  a.position_inc = position_inc;
  a.partial = static_cast<uint64_t*>(scratch);
  return gain ? dispatch<true, EPI_ARGMAX, WF_BF16>(a, st) : dispatch<false, EPI_ARGMAX, WF_BF16>(a, st);
}
