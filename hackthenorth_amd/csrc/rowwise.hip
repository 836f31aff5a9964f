// Row-wise kernels: RMSNorm, residual-add + RMSNorm, SwiGLU, embedding gather.
//
// All four are pure HBM streams (no reuse), so the layout is one wave per row
// with 16-byte loads and stores, four rows per 256-thread block, and a
// wave64 DPP reduction for the sum of squares. Rows whose width or pointers
// do not allow 16-byte access take a scalar path with identical rounding.
#include <algorithm>

#include "common.h"

namespace htn {

// Shared RMSNorm body: v holds the fp32 row values this lane owns.
//   out = bf16(gain * bf16(v * inv)), inv = 1 / sqrt(sum(v^2) / cols + eps)
// The division and square root are correctly rounded, as in torch's CPU rsqrt.
__device__ __forceinline__ float rms_inv(float ss, int cols, float eps) {
  return 1.0f / sqrtf(wave_sum(ss) / static_cast<float>(cols) + eps);
}

template <bool ADD>
__global__ __launch_bounds__(kBlock) void norm_rows_vec(const bf16_t* __restrict__ x, long x_stride,
                                                        const bf16_t* __restrict__ r,
                                                        const bf16_t* __restrict__ gain,
                                                        bf16_t* __restrict__ summed,
                                                        bf16_t* __restrict__ out, long rows,
                                                        int cols, float eps) {
  // Arguments in scalar registers before their first use: one round of loads.
  asm volatile("" ::"s"(x), "s"(x_stride), "s"(r), "s"(gain), "s"(summed), "s"(out), "s"(rows),
               "s"(cols), "s"(eps));
  constexpr int kMaxVec = 16;  // up to 8192 columns per row
  const int lane = threadIdx.x & 63;
  const long row = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wave exits together
  const int nv = cols >> 3;
  uint4 vals[kMaxVec];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j) {
    const int v = j * 64 + lane;
    vals[j] = make_uint4(0, 0, 0, 0);
    if (v < nv) {
      uint4 xv = *reinterpret_cast<const uint4*>(x + row * x_stride + v * 8);
      if (ADD) {
        const uint4 rv = *reinterpret_cast<const uint4*>(r + row * static_cast<long>(cols) + v * 8);
        xv.x = pack_bf2(bf_lo(xv.x) + bf_lo(rv.x), bf_hi(xv.x) + bf_hi(rv.x));
        xv.y = pack_bf2(bf_lo(xv.y) + bf_lo(rv.y), bf_hi(xv.y) + bf_hi(rv.y));
        xv.z = pack_bf2(bf_lo(xv.z) + bf_lo(rv.z), bf_hi(xv.z) + bf_hi(rv.z));
        xv.w = pack_bf2(bf_lo(xv.w) + bf_lo(rv.w), bf_hi(xv.w) + bf_hi(rv.w));
        *reinterpret_cast<uint4*>(summed + row * static_cast<long>(cols) + v * 8) = xv;
      }
      vals[j] = xv;
      float f[8];
      unpack8(xv, f);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(f[i], f[i], ss);
    }
  }
  const float inv = rms_inv(ss, cols, eps);
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j) {
    const int v = j * 64 + lane;
    if (v < nv) {
      float f[8], g[8];
      unpack8(vals[j], f);
      unpack8(*reinterpret_cast<const uint4*>(gain + v * 8), g);
      uint4 o;
      o.x = pack_bf2(g[0] * round_bf(f[0] * inv), g[1] * round_bf(f[1] * inv));
      o.y = pack_bf2(g[2] * round_bf(f[2] * inv), g[3] * round_bf(f[3] * inv));
      o.z = pack_bf2(g[4] * round_bf(f[4] * inv), g[5] * round_bf(f[5] * inv));
      o.w = pack_bf2(g[6] * round_bf(f[6] * inv), g[7] * round_bf(f[7] * inv));
      *reinterpret_cast<uint4*>(out + row * static_cast<long>(cols) + v * 8) = o;
    }
  }
}

template <bool ADD>
__global__ __launch_bounds__(kBlock) void norm_rows_scalar(const bf16_t* __restrict__ x, long x_stride,
                                                           const bf16_t* __restrict__ r,
                                                           const bf16_t* __restrict__ gain,
                                                           bf16_t* __restrict__ summed,
                                                           bf16_t* __restrict__ out, long rows,
                                                           int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const long row = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float ss = 0.f;
  for (int c = lane; c < cols; c += kWave) {
    float f = bf2f(x[row * x_stride + c]);
    if (ADD) {
      const uint32_t s = f2bf(f + bf2f(r[row * cols + c]));
      summed[row * cols + c] = static_cast<bf16_t>(s);
      f = bf2f(s);
    }
    ss = fmaf(f, f, ss);
  }
  const float inv = rms_inv(ss, cols, eps);
  for (int c = lane; c < cols; c += kWave) {
    const float f = ADD ? bf2f(summed[row * cols + c]) : bf2f(x[row * x_stride + c]);
    out[row * cols + c] = static_cast<bf16_t>(f2bf(bf2f(gain[c]) * round_bf(f * inv)));
  }
}

// out = bf16(bf16(silu(g)) * u). Each thread takes two pieces of 8 columns,
// kBlock pieces apart, and has its four 16-byte loads (streaming: read once)
// in flight before the math; measured at [32768, 3072] two pieces beat one,
// four and eight, and streaming stores lost to plain ones. The launch keeps rows * cols / 8 below 2^31, so indices are 32-bit.
constexpr int kSwigluPieces = 2;
__global__ __launch_bounds__(kBlock) void swiglu_vec(const bf16_t* __restrict__ g, long gs,
                                                     const bf16_t* __restrict__ u, long us,
                                                     bf16_t* __restrict__ out, long rows, int cols) {
  asm volatile("" ::"s"(g), "s"(gs), "s"(u), "s"(us), "s"(out), "s"(rows), "s"(cols));
  const unsigned nv = static_cast<unsigned>(cols) >> 3;
  const unsigned total = static_cast<unsigned>(rows) * nv;
  const unsigned base = blockIdx.x * (kBlock * kSwigluPieces) + threadIdx.x;
  uint4 gv[kSwigluPieces], uv[kSwigluPieces];
  unsigned row[kSwigluPieces], v[kSwigluPieces];
#pragma unroll
  for (int k = 0; k < kSwigluPieces; ++k) {
    const unsigned i = base + k * kBlock;
    const unsigned ic = i < total ? i : total - 1;  // in bounds; stored only when i < total
    row[k] = ic / nv;
    v[k] = ic - row[k] * nv;
    gv[k] = load_stream16(g + static_cast<long>(row[k]) * gs + v[k] * 8);
    uv[k] = load_stream16(u + static_cast<long>(row[k]) * us + v[k] * 8);
  }
#pragma unroll
  for (int k = 0; k < kSwigluPieces; ++k) {
    if (base + k * kBlock >= total) break;
    float gf[8], uf[8], o[8];
    unpack8(gv[k], gf);
    unpack8(uv[k], uf);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = silu_bf(gf[j]) * uf[j];
    uint4 w;
    w.x = pack_bf2(o[0], o[1]);
    w.y = pack_bf2(o[2], o[3]);
    w.z = pack_bf2(o[4], o[5]);
    w.w = pack_bf2(o[6], o[7]);
    *reinterpret_cast<uint4*>(out + static_cast<long>(row[k]) * cols + v[k] * 8) = w;
  }
}

__global__ __launch_bounds__(kBlock) void swiglu_scalar(const bf16_t* __restrict__ g, long gs,
                                                        const bf16_t* __restrict__ u, long us,
                                                        bf16_t* __restrict__ out, long rows, int cols) {
  const long total = rows * cols;
  for (long i = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<long>(gridDim.x) * kBlock) {
    const long row = i / cols;
    const int c = static_cast<int>(i - row * cols);
    out[i] = static_cast<bf16_t>(f2bf(silu_bf(bf2f(g[row * gs + c])) * bf2f(u[row * us + c])));
  }
}

// One wave per four token ids: the ids first, then every 16-byte piece of
// the wave's rows, up to kEmbedPieces per lane in flight before the first
// store. Ids outside [0, vocab) give zero rows.
constexpr int kEmbedRows = 4, kEmbedPieces = 8;

struct EmbedJob {
  const int64_t* ids;
  long count;
  const bf16_t* table;
  long vocab;
  int hidden;
  bf16_t* out;
};

// Wave w of a job gathers ids 4w .. 4w + 3.
__device__ __forceinline__ void embed_wave(const EmbedJob& j, long w) {
  const int lane = threadIdx.x & 63;
  const long first = w * kEmbedRows;
  if (first >= j.count) return;
  const int nrows = j.count - first < kEmbedRows ? static_cast<int>(j.count - first) : kEmbedRows;
  int64_t id[kEmbedRows];
#pragma unroll
  for (int r = 0; r < kEmbedRows; ++r) {
    const int64_t v = r < nrows ? j.ids[first + r] : -1;
    id[r] = v >= 0 && v < j.vocab ? v : -1;
  }
  const unsigned nv = static_cast<unsigned>(j.hidden) >> 3;
  const unsigned items = nv * nrows;
  for (unsigned p0 = 0; p0 < items; p0 += 64 * kEmbedPieces) {
    uint4 val[kEmbedPieces];
    unsigned rr[kEmbedPieces], cc[kEmbedPieces];
#pragma unroll
    for (int k = 0; k < kEmbedPieces; ++k) {
      const unsigned i = p0 + k * 64 + lane;
      rr[k] = i / nv;
      cc[k] = i - rr[k] * nv;
      const int64_t idr = rr[k] == 0 ? id[0] : rr[k] == 1 ? id[1] : rr[k] == 2 ? id[2] : id[3];
      val[k] = make_uint4(0, 0, 0, 0);
      if (i < items && idr >= 0)
        val[k] = *reinterpret_cast<const uint4*>(j.table + idr * j.hidden + cc[k] * 8);
    }
#pragma unroll
    for (int k = 0; k < kEmbedPieces; ++k)
      if (p0 + k * 64 + lane < items)
        *reinterpret_cast<uint4*>(j.out + (first + rr[k]) * j.hidden + cc[k] * 8) = val[k];
  }
}

// A job's fields in scalar registers before their first use: one round of
// scalar loads instead of one per dependent use.
__device__ __forceinline__ void preload_job(const EmbedJob& j) {
  asm volatile("" ::"s"(j.ids), "s"(j.count), "s"(j.table), "s"(j.vocab), "s"(j.hidden), "s"(j.out));
}

__global__ __launch_bounds__(kBlock) void embed_vec(EmbedJob j) {
  preload_job(j);
  embed_wave(j, static_cast<long>(blockIdx.x) * (kBlock / kWave) +
                    __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
}

// Two gathers in one launch (the decode step's token row and RoPE row):
// blocks below split take job a, the rest job b.
__global__ __launch_bounds__(kBlock) void embed_pair(EmbedJob a, EmbedJob b, unsigned split) {
  preload_job(a);
  preload_job(b);
  asm volatile("" ::"s"(split));
  const long w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (blockIdx.x < split) embed_wave(a, static_cast<long>(blockIdx.x) * (kBlock / kWave) + w);
  else embed_wave(b, static_cast<long>(blockIdx.x - split) * (kBlock / kWave) + w);
}

__global__ __launch_bounds__(kBlock) void embed_scalar(const int64_t* __restrict__ ids,
                                                       const bf16_t* __restrict__ table, long vocab,
                                                       int hidden, bf16_t* __restrict__ out) {
  const long t = blockIdx.x;
  const int64_t id = ids[t];
  const bool ok = id >= 0 && id < vocab;
  for (int c = threadIdx.x; c < hidden; c += kBlock)
    out[t * hidden + c] = ok ? table[id * hidden + c] : static_cast<bf16_t>(0);
}

// Streaming read of `vecs` 16-byte vectors (the HBM read ceiling that the
// GEMVs are measured against): each wave reads consecutive 4 KB pieces (four
// 1 KB non-temporal loads in flight, lane-contiguous), two blocks per CU,
// folded with XOR into one word per block so the loads cannot be dropped.
// Of the grid-stride and per-wave-piece patterns with 4-16 loads in flight
// and 2-16 blocks per CU this one streamed fastest over 2 GB.
__global__ __launch_bounds__(kBlock) void stream_read(const uint4* __restrict__ src, long vecs,
                                                      uint32_t* __restrict__ out) {
  constexpr int U = 4;
  constexpr long kPiece = 64L * U;  // vectors per wave piece
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long pieces = vecs / kPiece;
  const long waves = static_cast<long>(gridDim.x) * (kBlock / kWave);
  uint32_t acc = 0;
  for (long c = static_cast<long>(blockIdx.x) * (kBlock / kWave) + wave; c < pieces; c += waves) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = load_stream16(src + c * kPiece + u * 64 + lane);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  // The last partial piece, vector by vector.
  for (long i = pieces * kPiece + static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; i < vecs;
       i += static_cast<long>(gridDim.x) * kBlock) {
    const uint4 v = load_stream16(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  __shared__ uint32_t red[kBlock / kWave];
  for (int m = 32; m >= 1; m >>= 1) acc ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), m, kWave));
  if (lane == 0) red[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

namespace {
int g_cus[64];
}

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (g_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_cus[dev] = n;
  }
  return g_cus[dev];
}

}  // namespace htn

using namespace htn;

extern "C" int htn_version(void) { return 1; }

extern "C" int64_t htn_stream_read_blocks(void) { return 2L * device_cus(); }

extern "C" int htn_stream_read(const void* src, int64_t bytes, uint32_t* out, htn_stream_t stream) {
  if (!src || !out || bytes <= 0 || bytes % 16 || !aligned16(src)) return HTN_EINVAL;
  hipLaunchKernelGGL(stream_read, dim3(2 * device_cus()), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4*>(src),
                     static_cast<long>(bytes / 16), out);
  return launch_status();
}

namespace {

int norm_launch(bool add, const void* x, int64_t x_stride, const void* r, const void* gain,
                void* summed, void* out, int64_t rows, int64_t cols, float eps,
                htn_stream_t stream) {
  if (!x || !gain || !out || rows <= 0 || cols <= 0 || cols > 16384 || x_stride < cols)
    return HTN_EINVAL;
  if (add && (!r || !summed)) return HTN_EINVAL;
  // Rows past 8192 columns (beyond one wave's registers) take the scalar path.
  const bool vec = cols <= 8192 && cols % 8 == 0 && x_stride % 8 == 0 && aligned16(x) && aligned16(gain) &&
                   aligned16(out) && (!add || (aligned16(r) && aligned16(summed)));
  const dim3 grid((rows + 3) / 4);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bf16_t* xp = static_cast<const bf16_t*>(x);
  const bf16_t* rp = static_cast<const bf16_t*>(r);
  const bf16_t* gp = static_cast<const bf16_t*>(gain);
  bf16_t* sp = static_cast<bf16_t*>(summed);
  bf16_t* op = static_cast<bf16_t*>(out);
  if (vec) {
    if (add)
      hipLaunchKernelGGL(norm_rows_vec<true>, grid, dim3(kBlock), 0, st, xp, x_stride, rp, gp, sp, op,
                         rows, static_cast<int>(cols), eps);
    else
      hipLaunchKernelGGL(norm_rows_vec<false>, grid, dim3(kBlock), 0, st, xp, x_stride, rp, gp, sp,
                         op, rows, static_cast<int>(cols), eps);
  } else {
    if (add)
      hipLaunchKernelGGL(norm_rows_scalar<true>, grid, dim3(kBlock), 0, st, xp, x_stride, rp, gp, sp,
                         op, rows, static_cast<int>(cols), eps);
    else
      hipLaunchKernelGGL(norm_rows_scalar<false>, grid, dim3(kBlock), 0, st, xp, x_stride, rp, gp,
                         sp, op, rows, static_cast<int>(cols), eps);
  }
  return launch_status();
}

}  // namespace

extern "C" int htn_rms_norm(const void* x, int64_t x_row_stride, const void* gain, void* out,
                            int64_t rows, int64_t cols, float eps, htn_stream_t stream) {
  return norm_launch(false, x, x_row_stride, nullptr, gain, nullptr, out, rows, cols, eps, stream);
}

extern "C" int htn_add_rms_norm(const void* x, const void* residual, const void* gain,
                                void* summed, void* normalized, int64_t rows, int64_t cols,
                                float eps, htn_stream_t stream) {
  return norm_launch(true, x, cols, residual, gain, summed, normalized, rows, cols, eps, stream);
}

extern "C" int htn_swiglu(const void* gate, int64_t gate_row_stride, const void* up,
                          int64_t up_row_stride, void* out, int64_t rows, int64_t cols,
                          htn_stream_t stream) {
  if (!gate || !up || !out || rows <= 0 || cols <= 0 || gate_row_stride < cols ||
      up_row_stride < cols)
    return HTN_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = cols % 8 == 0 && gate_row_stride % 8 == 0 && up_row_stride % 8 == 0 &&
                   aligned16(gate) && aligned16(up) && aligned16(out) &&
                   rows * (cols / 8) < (int64_t{1} << 31);
  const long per_block = static_cast<long>(kBlock) * kSwigluPieces;
  const long vec_blocks = (rows * (cols / 8) + per_block - 1) / per_block;
  const long scalar_blocks = std::min((rows * cols + kBlock - 1) / kBlock,
                                      static_cast<long>(device_cus()) * 16);
  if (vec)
    hipLaunchKernelGGL(swiglu_vec, dim3(vec_blocks), dim3(kBlock), 0, st, static_cast<const bf16_t*>(gate),
                       static_cast<long>(gate_row_stride), static_cast<const bf16_t*>(up),
                       static_cast<long>(up_row_stride), static_cast<bf16_t*>(out),
                       static_cast<long>(rows), static_cast<int>(cols));
  else
    hipLaunchKernelGGL(swiglu_scalar, dim3(scalar_blocks), dim3(kBlock), 0, st,
                       static_cast<const bf16_t*>(gate), static_cast<long>(gate_row_stride),
                       static_cast<const bf16_t*>(up), static_cast<long>(up_row_stride),
                       static_cast<bf16_t*>(out), static_cast<long>(rows), static_cast<int>(cols));
  return launch_status();
}

namespace {
long embed_blocks(int64_t count) {
  return (count + (kBlock / kWave) * kEmbedRows - 1) / ((kBlock / kWave) * kEmbedRows);
}
}  // namespace

extern "C" int htn_embed_gather_pair(const int64_t* ids_a, int64_t count_a, const void* table_a,
                                     int64_t vocab_a, int64_t hidden_a, void* out_a,
                                     const int64_t* ids_b, int64_t count_b, const void* table_b,
                                     int64_t vocab_b, int64_t hidden_b, void* out_b,
                                     htn_stream_t stream) {
  if (!ids_a || !table_a || !out_a || count_a <= 0 || vocab_a <= 0 || hidden_a <= 0 ||
      !ids_b || !table_b || !out_b || count_b <= 0 || vocab_b <= 0 || hidden_b <= 0 ||
      count_a > (1L << 31) || count_b > (1L << 31))
    return HTN_EINVAL;
  if (hidden_a % 8 || hidden_b % 8 || !aligned16(table_a) || !aligned16(out_a) ||
      !aligned16(table_b) || !aligned16(out_b))
    return HTN_EUNSUPPORTED;
  const long split = embed_blocks(count_a);
  hipLaunchKernelGGL(embed_pair, dim3(split + embed_blocks(count_b)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream),
                     EmbedJob{ids_a, static_cast<long>(count_a), static_cast<const bf16_t*>(table_a),
                              static_cast<long>(vocab_a), static_cast<int>(hidden_a),
                              static_cast<bf16_t*>(out_a)},
                     EmbedJob{ids_b, static_cast<long>(count_b), static_cast<const bf16_t*>(table_b),
                              static_cast<long>(vocab_b), static_cast<int>(hidden_b),
                              static_cast<bf16_t*>(out_b)},
                     static_cast<unsigned>(split));
  return launch_status();
}

extern "C" int htn_embed_gather(const int64_t* ids, int64_t count, const void* table,
                                int64_t vocab, int64_t hidden, void* out, htn_stream_t stream) {
  if (!ids || !table || !out || count <= 0 || vocab <= 0 || hidden <= 0 || count > (1L << 31))
    return HTN_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = hidden % 8 == 0 && aligned16(table) && aligned16(out);
  if (vec)
    hipLaunchKernelGGL(embed_vec, dim3(embed_blocks(count)), dim3(kBlock), 0, st,
                       EmbedJob{ids, static_cast<long>(count), static_cast<const bf16_t*>(table),
                                static_cast<long>(vocab), static_cast<int>(hidden),
                                static_cast<bf16_t*>(out)});
  else
    hipLaunchKernelGGL(embed_scalar, dim3(count), dim3(kBlock), 0, st, ids,
                       static_cast<const bf16_t*>(table), static_cast<long>(vocab),
                       static_cast<int>(hidden), static_cast<bf16_t*>(out));
  return launch_status();
}
