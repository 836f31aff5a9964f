// Projections of many rows at once (a prompt's prefill): y = x W^T over M
// rows as a tiled GEMM on the matrix cores, one launch per projection.
//
// The multi-row kernel of gemm_rows.hip streams each weight once for up to
// 128 rows and re-reads the rows' fragments per 16-column strip; past a few
// hundred rows the arithmetic, not the weight stream, is the work, and a
// 2-D tiling that reuses both operands from LDS does it with far fewer
// instructions per multiply:
//
//  * block = 256 threads (2 x 2 waves) on a 128-row x 128-column output tile;
//    each 64-deep k step stages the x tile (128 rows x 128 bytes) and the
//    weight tile (128 rows x 128 bytes) into LDS with LDS-direct loads
//    (16 KB each; chunk c of row r at column c ^ (r & 7), so the fragment
//    reads of eight consecutive lanes hit eight different column groups),
//    the next step's loads in flight during this step's multiplies, one
//    barrier per step;
//  * each wave multiplies a 64 x 64 quarter: D^T = W X^T on
//    v_mfma_f32_16x16x32_bf16 (weight rows as M, x rows as N), so a lane
//    ends with four consecutive output columns of one row (8-byte stores);
//  * SwiGLU tiles interleave gate and up rows (32 of each per wave), so a
//    lane holds the gate and up dot products of the same outputs;
//  * when the 128-row grid would leave CUs without a block (short prompts),
//    tiles take 64 x rows (each wave a 32 x 64 part), twice the blocks over
//    the same weight tiles;
//  * when the tiles fill at most half of the blocks the CUs hold at once
//    (prompts of a few hundred rows; the K-long down projection most of
//    all), each tile's k range splits over up to 8 blocks, as many as fit in
//    one round of resident blocks; they store fp32 partial sums and a second
//    launch adds them in split order and applies the epilogue;
//  * blocks are laid out XCD-major: the blocks of one weight tile share an
//    XCD (block L runs on XCD L % 8), so its L2 serves the tile to all of them.
//
// Epilogues keep the batch-one GEMV's bf16 boundaries (store, + residual,
// SwiGLU); fp32 accumulation over k in 64-wide steps.
#include "common.h"

namespace htn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_ptr_t;

constexpr int kTm = 128;                  // x rows per block (64 for short prompts)
constexpr int kTn = 128;                  // weight rows per block
constexpr int kTk = 64;                   // k per staged step

struct TileArgs {
  const bf16_t* x; long x_rs;
  const bf16_t* w;
  const bf16_t* res; long res_rs;
  bf16_t* y; long y_rs;
  int M, N, K;        // N: output columns (gate columns for SwiGLU)
  int mtiles, ntiles; // output tiles along M and N
  int ksplit, steps;  // k splits per tile, 64-wide k steps per split
  float* part;        // K-split partial sums [ksplit][M][part_rs]
  long part_rs;       // round4(N), twice that for SwiGLU (gate, then up sums)
};

constexpr int kMinSplitSteps = 16;    // k steps each split keeps at least
constexpr int kMaxSplit = 8;

// Eight 16-byte operand fragments in one asm block: LDS-direct data is read by
// inline asm (the compiler would wait for every load in flight before an
// ordinary LDS read of such a buffer). The reads of the next k half are issued
// before the multiplies of this one; the wait names the fragments as
// operands, so no use of them moves above it.
__device__ __forceinline__ void issue_frag8(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3,
                                            uint32_t a4, uint32_t a5, uint32_t a6, uint32_t a7,
                                            u32x4 (&f)[8]) {
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %9\n\t"
      "ds_read_b128 %2, %10\n\t"
      "ds_read_b128 %3, %11\n\t"
      "ds_read_b128 %4, %12\n\t"
      "ds_read_b128 %5, %13\n\t"
      "ds_read_b128 %6, %14\n\t"
      "ds_read_b128 %7, %15"
      : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]),
        "=&v"(f[6]), "=&v"(f[7])
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "v"(a4), "v"(a5), "v"(a6), "v"(a7)
      : "memory");
}

__device__ __forceinline__ void wait_frag8(u32x4 (&f)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]),
                 "+v"(f[6]), "+v"(f[7])
               :
               : "memory");
}

// Six fragments (64-row tiles: four weight, two x), as issue_frag8 / wait_frag8.
__device__ __forceinline__ void issue_frag6(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3,
                                            uint32_t a4, uint32_t a5, u32x4 (&f)[6]) {
  asm volatile(
      "ds_read_b128 %0, %6\n\t"
      "ds_read_b128 %1, %7\n\t"
      "ds_read_b128 %2, %8\n\t"
      "ds_read_b128 %3, %9\n\t"
      "ds_read_b128 %4, %10\n\t"
      "ds_read_b128 %5, %11"
      : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5])
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "v"(a4), "v"(a5)
      : "memory");
}

__device__ __forceinline__ void wait_frag6(u32x4 (&f)[6]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5])
               :
               : "memory");
}

// 4 x NT multiplies of one k half: weight fragments f[0..3] x x fragments
// f[4 .. 4 + NT - 1].
template <int NT, int NF>
__device__ __forceinline__ void mfma_half(const u32x4 (&f)[NF], f32x4_t (&acc)[4][NT]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t)
      acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8_t, f[i]), __builtin_bit_cast(bf16x8_t, f[4 + t]), acc[i][t], 0,
          0, 0);
}

__device__ __forceinline__ void lds_barrier_t() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Epilogue of one wave's 64 x 64 quarter. Lane (col, quad) holds, per weight
// tile i and x tile t, the outputs of x row mb + 16 t + col and weight rows
// (output columns) nb + 16 i + 4 quad + (0..3); for SwiGLU tiles 0, 1 are the
// gate and 2, 3 the up rows of output columns nb .. nb + 31.
template <int EPI, int NT>
__device__ __forceinline__ void store_tile(const TileArgs& a, const f32x4_t (&acc)[4][NT], int mb,
                                           int nb, int col, int quad) {
  constexpr bool SW = EPI == HTN_EPI_SWIGLU;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int m = mb + 16 * t + col;
    if (m >= a.M) continue;
    if constexpr (SW) {
      // Weight tiles 0, 1 are gate columns nb .. nb + 31 and 2, 3 the up
      // columns of the same outputs.
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int n = nb + 16 * i + 4 * quad;
        if (n >= a.N) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = silu_bf(round_bf(acc[i][t][e])) * round_bf(acc[i + 2][t][e]);
        bf16_t* dst = a.y + static_cast<long>(m) * a.y_rs + n;
        if (n + 4 <= a.N) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
        } else {
          for (int e = 0; e < 4 && n + e < a.N; ++e) dst[e] = static_cast<bf16_t>(f2bf(o[e]));
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = nb + 16 * i + 4 * quad;
        if (n >= a.N) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] = acc[i][t][e];
          if (EPI == HTN_EPI_RESIDUAL)
            o[e] = round_bf(o[e]) + (n + e < a.N ? bf2f(a.res[static_cast<long>(m) * a.res_rs + n + e]) : 0.f);
        }
        bf16_t* dst = a.y + static_cast<long>(m) * a.y_rs + n;
        if (n + 4 <= a.N) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
        } else {
          for (int e = 0; e < 4 && n + e < a.N; ++e) dst[e] = static_cast<bf16_t>(f2bf(o[e]));
        }
      }
    }
  }
}

// K-split epilogue: the block's fp32 sums of its k range, unrounded, at
// part[(s M + m) part_rs + c], c = the output column, or for SwiGLU c = n for
// the gate sums and part_rs / 2 + n for the up sums of output column n. The
// four columns of a lane end before round4(N), so every store is whole.
template <bool SW, int NT>
__device__ __forceinline__ void store_part(const TileArgs& a, const f32x4_t (&acc)[4][NT], int s,
                                           int mb, int nb, int col, int quad) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int m = mb + 16 * t + col;
    if (m >= a.M) continue;
    float* row = a.part + (static_cast<long>(s) * a.M + m) * a.part_rs;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = nb + 16 * (SW ? (i & 1) : i) + 4 * quad;
      if (n >= a.N) continue;
      *reinterpret_cast<f32x4_t*>(row + (SW && i >= 2 ? a.part_rs / 2 : 0) + n) = acc[i][t];
    }
  }
}

// Bytes of one staged k step: the x tile (TM rows) and the weight tile (128
// rows), 128 bytes per row.
template <int TM>
struct Stage {
  static constexpr int kBytes = (TM + kTn) * kTk * 2;
};

// One k step into its stage: wave w's x rows (TM / 4 of them) and weight rows
// (32), eight rows (1 KB) per LDS-direct load.
template <int TM>
__device__ __forceinline__ void stage_tiles(unsigned char* lds, int ks, int wave,
                                            __amdgpu_buffer_rsrc_t xrs, __amdgpu_buffer_rsrc_t wrs,
                                            const uint32_t (&xoff)[4],
                                            const uint32_t (&woff)[4]) {
  unsigned char* st = lds + (ks & 1) * Stage<TM>::kBytes;
  const uint32_t ko = static_cast<uint32_t>(ks) * kTk * 2u;
#pragma unroll
  for (int u = 0; u < TM / 32; ++u)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (lds_ptr_t*)(st + ((TM / 4) * wave + 8 * u) * 128),
                                             16, xoff[u], ko, 0, 0);
#pragma unroll
  for (int u = 0; u < 4; ++u)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        wrs, (lds_ptr_t*)(st + TM * kTk * 2 + (32 * wave + 8 * u) * 128), 16, woff[u], ko, 0, 0);
}

template <int EPI, int TM>
__global__ __launch_bounds__(256) void gemm_tiles_kernel(TileArgs a) {
  // Arguments in scalar registers at entry: one round of scalar loads.
  asm volatile("" ::"s"(a.x), "s"(a.x_rs), "s"(a.w), "s"(a.res), "s"(a.res_rs), "s"(a.y),
               "s"(a.y_rs), "s"(a.M), "s"(a.N), "s"(a.K), "s"(a.mtiles), "s"(a.ntiles),
               "s"(a.ksplit), "s"(a.steps), "s"(a.part), "s"(a.part_rs));
  extern __shared__ __align__(16) unsigned char lds[];  // two stages of x and weight tiles
  constexpr int NT = TM / 32;        // 16-row x tiles per wave (4 or 2)
  constexpr int XR = TM / 4;         // x rows each wave stages (32 or 16)
  constexpr int kStage = Stage<TM>::kBytes;
  constexpr int kXBytes = TM * kTk * 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;  // this wave's TM / 2 x rows, 64 weight rows
  const int col = lane & 15, quad = lane >> 4;
  // XCD-major layout: block L on XCD L % 8 takes weight tile
  // nt = (L / 8 / (mtiles ksplit)) * 8 + L % 8, row tile (L / 8) % mtiles and
  // k split (L / 8 / mtiles) % ksplit.
  const int L = blockIdx.x, j = L >> 3, per = a.mtiles * a.ksplit;
  const int g = j / per, q = j - g * per, s = q / a.mtiles;
  const int nt = g * 8 + (L & 7), mt = q - s * a.mtiles;
  if (nt >= a.ntiles) return;
  const int m0 = mt * TM;
  // Weight rows of the tile: rows n0 .. n0 + 127, or for SwiGLU 64 output
  // columns c0 .. c0 + 63 as four 32-row groups gate, up, gate, up.
  constexpr bool SW = EPI == HTN_EPI_SWIGLU;
  const int n0 = SW ? nt * 64 : nt * kTn;

  // Staging: wave w loads x rows XR w .. XR w + XR - 1 and weight rows 32 w ..
  // 32 w + 31 of the tile, eight rows (1 KB) per instruction; lane l takes
  // row 8 u + l / 8 of the wave's rows and writes position l % 8 of it,
  // loading source chunk (l % 8) ^ (row & 7). Both operands go through one
  // descriptor per wave whose range ends at the last real row, so rows past
  // M or past the weight's end read as zeros. For SwiGLU, wave w's 32 weight
  // rows are group w: gate, up, gate, up rows of columns n0 + 32 (w / 2) ...
  const int lr = lane >> 3, lp = lane & 7;
  const long mrows = a.M - m0 < TM ? a.M - m0 : TM;
  const __amdgpu_buffer_rsrc_t xrs =
      buffer_rsrc(a.x + static_cast<long>(m0) * a.x_rs,
                  static_cast<uint32_t>(mrows * a.x_rs * 2));
  long wbase, wrows;
  if (SW) {
    const int c0 = n0 + (wave >> 1) * 32;
    wbase = static_cast<long>((wave & 1) ? a.N : 0) + c0;
    wrows = a.N - c0 < 32 ? (a.N - c0 > 0 ? a.N - c0 : 0) : 32;
  } else {
    wbase = n0 + 32 * wave;
    wrows = a.N - wbase < 32 ? (a.N - wbase > 0 ? a.N - wbase : 0) : 32;
  }
  const __amdgpu_buffer_rsrc_t wrs = uniform_rsrc(a.w + (wrows > 0 ? wbase : 0) * a.K,
                                                  static_cast<uint32_t>(wrows * a.K * 2));
  uint32_t xoff[4], woff[4];  // x offsets: the first TM / 32 are used
#pragma unroll
  for (int u = 0; u < XR / 8; ++u) {
    const int r = XR * wave + 8 * u + lr;  // x tile row
    xoff[u] = static_cast<uint32_t>(r) * static_cast<uint32_t>(a.x_rs) * 2u + (lp ^ (r & 7)) * 16;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = 8 * u + lr;     // row within the wave's 32
    const int r = 32 * wave + c;  // weight tile row
    woff[u] = static_cast<uint32_t>(c) * static_cast<uint32_t>(a.K) * 2u + (lp ^ (r & 7)) * 16;
  }

  // Fragment addresses in stage 0 (stage 1 is kStage further): k chunk
  // 4 h + quad of row 16 t + col, un-swizzled.
  const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t*)lds));
  uint32_t wa[2][4], xa[2][NT];  // [k half][tile]
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int rw = 64 * wn + 16 * t + col;
      wa[h][t] = base + kXBytes + static_cast<uint32_t>(rw * 128 + ((((4 * h + quad) ^ (rw & 7))) * 16));
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int rx = (TM / 2) * wm + 16 * t + col;
      xa[h][t] = base + static_cast<uint32_t>(rx * 128 + ((((4 * h + quad) ^ (rx & 7))) * 16));
    }
  }

  f32x4_t acc[4][NT];  // [weight tile][x tile]: D^T rows = weight rows, columns = x rows
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[i][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = a.K / kTk;
  const int k0 = s * a.steps, k1 = nk < k0 + a.steps ? nk : k0 + a.steps;
  stage_tiles<TM>(lds, k0, wave, xrs, wrs, xoff, woff);
  for (int ks = k0; ks < k1; ++ks) {
    // This wave's part of step ks has landed; after the barrier everyone's
    // has, and every wave has finished step ks - 1, whose stage step ks + 1
    // now takes (in flight during this step's multiplies).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier_t();
    if (ks + 1 < k1) stage_tiles<TM>(lds, ks + 1, wave, xrs, wrs, xoff, woff);
    const uint32_t so = static_cast<uint32_t>((ks & 1) * kStage);
    if constexpr (NT == 4) {
      u32x4 f0[8], f1[8];
      issue_frag8(wa[0][0] + so, wa[0][1] + so, wa[0][2] + so, wa[0][3] + so, xa[0][0] + so,
                  xa[0][1] + so, xa[0][2] + so, xa[0][3] + so, f0);
      wait_frag8(f0);
      issue_frag8(wa[1][0] + so, wa[1][1] + so, wa[1][2] + so, wa[1][3] + so, xa[1][0] + so,
                  xa[1][1] + so, xa[1][2] + so, xa[1][3] + so, f1);
      __builtin_amdgcn_sched_barrier(0);
      mfma_half<NT>(f0, acc);
      __builtin_amdgcn_sched_barrier(0);
      wait_frag8(f1);
      mfma_half<NT>(f1, acc);
    } else {
      u32x4 f0[6], f1[6];
      issue_frag6(wa[0][0] + so, wa[0][1] + so, wa[0][2] + so, wa[0][3] + so, xa[0][0] + so,
                  xa[0][1] + so, f0);
      wait_frag6(f0);
      issue_frag6(wa[1][0] + so, wa[1][1] + so, wa[1][2] + so, wa[1][3] + so, xa[1][0] + so,
                  xa[1][1] + so, f1);
      __builtin_amdgcn_sched_barrier(0);
      mfma_half<NT>(f0, acc);
      __builtin_amdgcn_sched_barrier(0);
      wait_frag6(f1);
      mfma_half<NT>(f1, acc);
    }
  }

  const int mb = m0 + (TM / 2) * wm, nb = SW ? n0 + 32 * wn : n0 + 64 * wn;
  if (a.ksplit > 1)
    store_part<SW, NT>(a, acc, s, mb, nb, col, quad);
  else
    store_tile<EPI, NT>(a, acc, mb, nb, col, quad);
}

// K-split sum + epilogue: thread i takes output columns 4 (i % (part_rs' / 4))
// .. + 3 of row i / (part_rs' / 4) (part_rs' = round4(N)), adds the splits'
// partials in split order and rounds as store_tile does.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_tiles_finish(TileArgs a) {
  asm volatile("" ::"s"(a.res), "s"(a.res_rs), "s"(a.y), "s"(a.y_rs), "s"(a.M), "s"(a.N),
               "s"(a.ksplit), "s"(a.part), "s"(a.part_rs));
  constexpr bool SW = EPI == HTN_EPI_SWIGLU;
  const long n4 = (SW ? a.part_rs / 2 : a.part_rs) / 4;
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long m = i / n4;
  if (m >= a.M) return;
  const int n = static_cast<int>(i - m * n4) * 4;
  const long stride = static_cast<long>(a.M) * a.part_rs;
  const float* p = a.part + m * a.part_rs + n;
  f32x4_t g = *reinterpret_cast<const f32x4_t*>(p), u{};
  if (SW) u = *reinterpret_cast<const f32x4_t*>(p + a.part_rs / 2);
  for (int s = 1; s < a.ksplit; ++s) {
    g += *reinterpret_cast<const f32x4_t*>(p + s * stride);
    if (SW) u += *reinterpret_cast<const f32x4_t*>(p + s * stride + a.part_rs / 2);
  }
  float o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (SW)
      o[e] = silu_bf(round_bf(g[e])) * round_bf(u[e]);
    else if (EPI == HTN_EPI_RESIDUAL)
      o[e] = round_bf(g[e]) + (n + e < a.N ? bf2f(a.res[m * a.res_rs + n + e]) : 0.f);
    else
      o[e] = g[e];
  }
  bf16_t* dst = a.y + m * a.y_rs + n;
  if (n + 4 <= a.N) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
  } else {
    for (int e = 0; e < 4 && n + e < a.N; ++e) dst[e] = static_cast<bf16_t>(f2bf(o[e]));
  }
}

// Launch shape: the row tile (128, or 64 when the 128-row grid would leave
// CUs without a block: twice the blocks over the same weight tiles; 8B
// 256-token prefill 14.9 -> 13.9 ms, at a full first wave of 128-row blocks
// the 64-row tiles measured slower) and the k split.
struct TilePlan {
  int tm, ksplit, steps;
  long blocks, part_rs;
};

TilePlan plan_tiles(long rows, long n, long k, int epilogue) {
  const bool sw = epilogue == HTN_EPI_SWIGLU;
  const long cols = (((sw ? (n + 63) / 64 : (n + kTn - 1) / kTn) + 7) / 8) * 8;
  const long cus = device_cus();
  TilePlan p{};
  p.tm = cols * ((rows + 127) / 128) < cus ? 64 : 128;
  const long base = cols * ((rows + p.tm - 1) / p.tm);
  const long nk = k / kTk;
  // Blocks resident at once: 64-row tiles take 48 KB of the CU's 160 KB of
  // LDS (three blocks), 128-row tiles 64 KB (two). A split that overflows
  // one round of them measured slower (8B QKV at 1024 rows: 384 -> 768
  // blocks of 128 rows, 74 -> 87 us).
  const long slots = cus * (p.tm == 64 ? 3 : 2);
  long ks = 1;
  if (2 * base <= slots) {
    ks = slots / base;
    if (ks > nk / kMinSplitSteps) ks = nk / kMinSplitSteps;
    if (ks > kMaxSplit) ks = kMaxSplit;
    if (ks < 1) ks = 1;
  }
  p.steps = static_cast<int>((nk + ks - 1) / ks);
  p.ksplit = static_cast<int>((nk + p.steps - 1) / p.steps);
  p.blocks = base * p.ksplit;
  p.part_rs = (sw ? 2 : 1) * ((n + 3) / 4 * 4);
  return p;
}

long tiles_scratch_bytes(const TilePlan& p, long rows) {
  return p.ksplit > 1 ? static_cast<long>(p.ksplit) * rows * p.part_rs * 4 : 0;
}

template <int EPI, int TM>
int launch_tiles(TileArgs& a, long blocks, hipStream_t st) {
  const size_t lds = 2 * static_cast<size_t>(Stage<TM>::kBytes);
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&gemm_tiles_kernel<EPI, TM>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  (void)attr;  // a refused size surfaces as a launch error
  a.mtiles = static_cast<int>((a.M + TM - 1) / TM);
  hipLaunchKernelGGL((gemm_tiles_kernel<EPI, TM>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                     lds, st, a);
  return launch_status();
}

template <int EPI>
int launch_tiles_for(TileArgs& a, const TilePlan& p, hipStream_t st) {
  const int rc = p.tm == 64 ? launch_tiles<EPI, 64>(a, p.blocks, st)
                            : launch_tiles<EPI, 128>(a, p.blocks, st);
  if (rc != HTN_OK || a.ksplit == 1) return rc;
  const long groups = static_cast<long>(a.M) * ((a.N + 3) / 4);
  hipLaunchKernelGGL((gemm_tiles_finish<EPI>), dim3(static_cast<unsigned>((groups + 255) / 256)),
                     dim3(256), 0, st, a);
  return launch_status();
}

}  // namespace
}  // namespace htn

using namespace htn;

extern "C" int64_t htn_gemm_tiles_scratch_bytes(int64_t rows, int64_t n, int64_t k,
                                                int epilogue) {
  if (rows <= 0 || n <= 0 || k <= 0 || k % kTk) return 0;
  if (epilogue != HTN_EPI_STORE && epilogue != HTN_EPI_RESIDUAL && epilogue != HTN_EPI_SWIGLU)
    return 0;
  return tiles_scratch_bytes(plan_tiles(rows, n, k, epilogue), rows);
}

extern "C" int htn_gemm_tiles(const void* x, int64_t x_stride, const void* w, int64_t n,
                              int64_t k, int64_t rows, int epilogue, const void* residual,
                              int64_t res_stride, void* y, int64_t y_stride, void* scratch,
                              htn_stream_t stream) {
  if (!x || !w || !y || rows <= 0 || n <= 0 || k <= 0) return HTN_EINVAL;
  if (epilogue != HTN_EPI_STORE && epilogue != HTN_EPI_RESIDUAL && epilogue != HTN_EPI_SWIGLU)
    return HTN_EINVAL;
  if (epilogue == HTN_EPI_RESIDUAL && (!residual || res_stride < n)) return HTN_EINVAL;
  if (y_stride < n || x_stride < k) return HTN_EINVAL;  // rows must not overlap
  // 64-wide k steps of 16-byte chunks; 8-byte output stores; 32-bit offsets.
  if (k % kTk || k > (1L << 20) || x_stride % 8 || y_stride % 4 || !aligned16(x) || !aligned16(w) ||
      (reinterpret_cast<uintptr_t>(y) & 7u))
    return HTN_EUNSUPPORTED;
  const long wrows = epilogue == HTN_EPI_SWIGLU ? 2 * n : n;
  if (static_cast<long>(kTm) * x_stride * 2 >= (1L << 31) || k * 2 >= (1L << 31) ||
      wrows >= (1L << 31) || rows >= (1L << 31))
    return HTN_EUNSUPPORTED;
  TileArgs a{};
  a.x = static_cast<const bf16_t*>(x); a.x_rs = x_stride;
  a.w = static_cast<const bf16_t*>(w);
  a.res = static_cast<const bf16_t*>(residual); a.res_rs = res_stride;
  a.y = static_cast<bf16_t*>(y); a.y_rs = y_stride;
  a.M = static_cast<int>(rows); a.N = static_cast<int>(n); a.K = static_cast<int>(k);
  hipStream_t st = static_cast<hipStream_t>(stream);
  a.ntiles = static_cast<int>(epilogue == HTN_EPI_SWIGLU ? (n + 63) / 64 : (n + kTn - 1) / kTn);
  if (!aligned16(scratch)) return HTN_EUNSUPPORTED;
  TilePlan p = plan_tiles(rows, n, k, epilogue);
  if (!scratch) {  // no scratch: every tile sums its whole k range
    p.blocks /= p.ksplit;
    p.ksplit = 1;
    p.steps = static_cast<int>(k / kTk);
  }
  a.ksplit = p.ksplit;
  a.steps = p.steps;
  a.part = static_cast<float*>(scratch);
  a.part_rs = p.part_rs;
  switch (epilogue) {
    case HTN_EPI_STORE: return launch_tiles_for<HTN_EPI_STORE>(a, p, st);
    case HTN_EPI_RESIDUAL: return launch_tiles_for<HTN_EPI_RESIDUAL>(a, p, st);
    default: return launch_tiles_for<HTN_EPI_SWIGLU>(a, p, st);
  }
}
