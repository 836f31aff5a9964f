// Decode attention for gfx950 (head_dim 128).
//
//  * qk-norm + RoPE: one wave per 128-wide head; lane l owns elements l and
//    l + 64, which are exactly the rotate_half partners, so RoPE needs no
//    cross-lane traffic and the sum of squares is one DPP reduction.
//  * grouped attention: grid (split, kv head, batch). A block loads the G*Q
//    query rows of its kv head once, streams its slice of K then V with
//    16-byte loads (16 lanes per 256-byte cache row, four rows per wave
//    instruction), keeps scores in LDS for an exact two-pass softmax, and
//    writes an unnormalised partial plus (max, sum); a second launch merges
//    the partials per output row (log-sum-exp weights). A block never waits
//    for other blocks: an agent-scope release per block (L2 write-back on
//    gfx950) costs far more than the extra launch.
//  * slots after a query's absolute position are masked; slots after the
//    largest position are never read.
//  * the fused prologue variant computes q and the newest k/v from the packed
//    projection row, appends k/v to the cache, and feeds the newest slot from
//    LDS so the appended row is never re-read from memory.
#include "common.h"

namespace htn {

constexpr int D = HTN_HEAD_DIM;
constexpr int kRowChunk = 8;        // query rows held in registers at once
constexpr int kMaxRows = 32;        // G * Q
constexpr int kSlotUnroll = 4;      // 16-slot groups per wave: 64 slots per block pass
constexpr int kMaxSplit = 16 * kSlotUnroll;
constexpr int kMergeUnroll = 8;     // partials loaded back to back in the merge

// Per-head RMSNorm then RoPE (rotate_half), reference rounding:
//   n = bf16(g * bf16(x * inv)); out_i = bf16(bf16(n_i cos_i) + bf16(rot(n)_i sin_i)).
__device__ __forceinline__ void norm_rope_wave(const bf16_t* x, const bf16_t* g, float eps,
                                               const bf16_t* cs, const bf16_t* sn, int lane,
                                               float& o0, float& o1) {
  const float a = bf2f(x[lane]), b = bf2f(x[lane + 64]);
  const float ss = wave_sum(a * a + b * b);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
  const float na = round_bf(bf2f(g[lane]) * round_bf(a * inv));
  const float nb = round_bf(bf2f(g[lane + 64]) * round_bf(b * inv));
  o0 = round_bf(round_bf(na * bf2f(cs[lane])) + round_bf(-nb * bf2f(sn[lane])));
  o1 = round_bf(round_bf(nb * bf2f(cs[lane + 64])) + round_bf(na * bf2f(sn[lane + 64])));
}

struct RopeArgs {
  const bf16_t* q; long q_sb, q_st;
  const bf16_t* k; long k_sb, k_st;
  const bf16_t* v; long v_sb, v_st;
  const bf16_t* qg; const bf16_t* kg; float q_eps, k_eps;
  const bf16_t* cos; const bf16_t* sin; long rope_st, rope_rows; int rope_by_pos;
  bf16_t* keys; bf16_t* values; long cap;
  const int64_t* pos;
  bf16_t* out_q; bf16_t* out_k;
  int B, T, Hq, Hkv;
};

__global__ __launch_bounds__(kBlock) void norm_rope_cache_kernel(RopeArgs a) {
  const int lane = threadIdx.x & 63;
  const long row = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const long q_rows = static_cast<long>(a.B) * a.T * a.Hq;
  const long total = q_rows + static_cast<long>(a.B) * a.T * a.Hkv;
  if (row >= total) return;
  const bool is_q = row < q_rows;
  const long r = is_q ? row : row - q_rows;
  const int heads = is_q ? a.Hq : a.Hkv;
  const long b = r / (static_cast<long>(a.T) * heads);
  const int t = static_cast<int>((r / heads) % a.T);
  const int h = static_cast<int>(r % heads);
  // Positions are only read when they select the rope row or the cache slot.
  const int64_t p = (a.rope_by_pos || a.keys) ? a.pos[t] : t;
  const long rr = a.rope_by_pos ? p : t;
  if (rr < 0 || rr >= a.rope_rows) return;
  const bf16_t* cs = a.cos + rr * a.rope_st;
  const bf16_t* sn = a.sin + rr * a.rope_st;
  float o0, o1;
  if (is_q) {
    norm_rope_wave(a.q + b * a.q_sb + t * a.q_st + h * D, a.qg, a.q_eps, cs, sn, lane, o0, o1);
    bf16_t* dst = a.out_q + ((b * a.T + t) * a.Hq + h) * D;
    dst[lane] = static_cast<bf16_t>(f2bf(o0));
    dst[lane + 64] = static_cast<bf16_t>(f2bf(o1));
    return;
  }
  norm_rope_wave(a.k + b * a.k_sb + t * a.k_st + h * D, a.kg, a.k_eps, cs, sn, lane, o0, o1);
  if (a.out_k) {
    bf16_t* dst = a.out_k + ((b * a.T + t) * a.Hkv + h) * D;
    dst[lane] = static_cast<bf16_t>(f2bf(o0));
    dst[lane + 64] = static_cast<bf16_t>(f2bf(o1));
  }
  if (a.keys && p >= 0 && p < a.cap) {
    const long slot = ((b * a.Hkv + h) * a.cap + p) * D;
    a.keys[slot + lane] = static_cast<bf16_t>(f2bf(o0));
    a.keys[slot + lane + 64] = static_cast<bf16_t>(f2bf(o1));
    const bf16_t* vs = a.v + b * a.v_sb + t * a.v_st + h * D;
    a.values[slot + lane] = vs[lane];
    a.values[slot + lane + 64] = vs[lane + 64];
  }
}

struct AttnArgs {
  // queries [b, h, t, :] (unfused)
  const bf16_t* q; long q_sb, q_sh, q_st;
  // packed projection row (fused prologue, Q == 1)
  const bf16_t* qkv; long qkv_sb, k_off, v_off;
  const bf16_t* qg; const bf16_t* kg; float q_eps, k_eps;
  const bf16_t* cos; const bf16_t* sin; long rope_st, rope_rows; int rope_by_pos;
  bf16_t* keys; bf16_t* values; long cap;
  const int64_t* pos;
  bf16_t* out;          // [B, Hq, Q, D]
  float* part;          // [B, Hq, Q, splits, D]
  float* ml;            // [B, Hq, Q, splits, 2]
  int B, Hq, Hkv, G, Q, splits, split;
  float scale;
};

template <bool FUSED>
__global__ __launch_bounds__(kBlock) void attention_kernel(AttnArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int rows = a.G * a.Q;
  float* qs = reinterpret_cast<float*>(smem);                     // [rows][D]
  float* sc = qs + rows * D;                                      // [rows][kMaxSplit]
  float* accr = sc + rows * kMaxSplit;                            // [4][kRowChunk][D]
  float* mrow = accr + 4 * kRowChunk * D;                         // [kMaxRows]
  float* lrow = mrow + kMaxRows;                                  // [kMaxRows]
  bf16_t* knew = reinterpret_cast<bf16_t*>(lrow + kMaxRows);      // [D]
  bf16_t* vnew = knew + D;                                        // [D]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane >> 4, e = lane & 15;
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const long kv_base = (static_cast<long>(b) * a.Hkv + kvh) * a.cap * D;

  int64_t maxpos = -1;
  for (int t = 0; t < a.Q; ++t) maxpos = a.pos[t] > maxpos ? a.pos[t] : maxpos;
  if (maxpos >= a.cap) maxpos = a.cap - 1;
  const long start = static_cast<long>(s) * a.split;
  long end = start + a.split;
  if (end > maxpos + 1) end = maxpos + 1;
  const bool active = start <= maxpos;
  const int64_t newest = FUSED ? a.pos[0] : -1;

  // ---- 1. issue this block's K and V loads first: they depend only on the
  // positions, so their HBM latency overlaps the query prologue. Lane (sub, e)
  // of wave w owns slot start + u*16 + w*4 + sub, dims e*8 .. e*8+7.
  uint4 kreg[kSlotUnroll], vreg[kSlotUnroll];
#pragma unroll
  for (int u = 0; u < kSlotUnroll; ++u) {
    const long j = start + u * 16 + wave * 4 + sub;
    kreg[u] = make_uint4(0, 0, 0, 0);
    vreg[u] = make_uint4(0, 0, 0, 0);
    if (active && j < end && !(FUSED && j == newest)) {
      kreg[u] = *reinterpret_cast<const uint4*>(a.keys + kv_base + j * D + e * 8);
      vreg[u] = *reinterpret_cast<const uint4*>(a.values + kv_base + j * D + e * 8);
    }
  }

  // ---- 2. query rows (and, fused, the newest k/v) into LDS
  if (FUSED) {
    const long rr = a.rope_by_pos ? newest : 0;
    const bool rope_ok = rr >= 0 && rr < a.rope_rows;
    const bf16_t* cs = a.cos + (rope_ok ? rr : 0) * a.rope_st;
    const bf16_t* sn = a.sin + (rope_ok ? rr : 0) * a.rope_st;
    const bf16_t* row = a.qkv + static_cast<long>(b) * a.qkv_sb;
    for (int g = wave; g < a.G; g += 4) {
      float o0, o1;
      norm_rope_wave(row + (static_cast<long>(kvh) * a.G + g) * D, a.qg, a.q_eps, cs, sn, lane, o0, o1);
      qs[g * D + lane] = o0;
      qs[g * D + lane + 64] = o1;
    }
    if (wave == (a.G & 3) && active && newest >= start && newest < end) {
      float o0, o1;
      norm_rope_wave(row + a.k_off + static_cast<long>(kvh) * D, a.kg, a.k_eps, cs, sn, lane, o0, o1);
      const bf16_t* vsrc = row + a.v_off + static_cast<long>(kvh) * D;
      const bf16_t k0 = static_cast<bf16_t>(f2bf(o0)), k1 = static_cast<bf16_t>(f2bf(o1));
      const bf16_t v0 = vsrc[lane], v1 = vsrc[lane + 64];
      knew[lane] = k0;
      knew[lane + 64] = k1;
      vnew[lane] = v0;
      vnew[lane + 64] = v1;
      const long slot = kv_base + newest * D;
      a.keys[slot + lane] = k0;
      a.keys[slot + lane + 64] = k1;
      a.values[slot + lane] = v0;
      a.values[slot + lane + 64] = v1;
    }
  } else {
    for (int i = tid; i < rows * D; i += kBlock) {
      const int r = i / D, d = i % D;
      const int h = kvh * a.G + r / a.Q, t = r % a.Q;
      qs[i] = bf2f(a.q[static_cast<long>(b) * a.q_sb + static_cast<long>(h) * a.q_sh +
                       static_cast<long>(t) * a.q_st + d]);
    }
  }
  __syncthreads();

  const int len = active ? static_cast<int>(end - start) : 0;
  if (active) {
    if (FUSED && newest >= start && newest < end) {
#pragma unroll
      for (int u = 0; u < kSlotUnroll; ++u) {
        if (start + u * 16 + wave * 4 + sub == newest) {
          kreg[u] = *reinterpret_cast<const uint4*>(knew + e * 8);
          vreg[u] = *reinterpret_cast<const uint4*>(vnew + e * 8);
        }
      }
    }
    // ---- 3. scores q.k * D^-1/2 into LDS (16 lanes per slot, DPP row sums)
    for (int r0 = 0; r0 < rows; r0 += kRowChunk) {
      const int nr = rows - r0 < kRowChunk ? rows - r0 : kRowChunk;
      float qr[kRowChunk][8];
#pragma unroll
      for (int r = 0; r < kRowChunk; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) qr[r][i] = r < nr ? qs[(r0 + r) * D + e * 8 + i] : 0.f;
#pragma unroll
      for (int u = 0; u < kSlotUnroll; ++u) {
        const long j = start + u * 16 + wave * 4 + sub;
#pragma unroll
        for (int r = 0; r < kRowChunk; ++r) {
          if (r < nr) {
            const float dsum = row16_sum(dot8(kreg[u], qr[r]));
            if (e == 0 && j < end) {
              const int rr = r0 + r;
              const int64_t qpos = a.pos[rr % a.Q];
              sc[rr * kMaxSplit + (j - start)] = j <= qpos ? dsum * a.scale : -INFINITY;
            }
          }
        }
      }
    }
    __syncthreads();

    // ---- 4. exact softmax numerators per row (the split's own max)
    for (int r = wave; r < rows; r += 4) {
      const float v = lane < len ? sc[r * kMaxSplit + lane] : -INFINITY;
      const float m = wave_max(v);
      const float p = (lane < len && m != -INFINITY) ? expf(v - m) : 0.f;
      if (lane < len) sc[r * kMaxSplit + lane] = p;
      const float l = wave_sum(p);
      if (lane == 0) {
        mrow[r] = m;
        lrow[r] = l;
      }
    }
    __syncthreads();

    // ---- 5. P.V from the V rows already in registers
    for (int r0 = 0; r0 < rows; r0 += kRowChunk) {
      const int nr = rows - r0 < kRowChunk ? rows - r0 : kRowChunk;
      float acc[kRowChunk][8];
#pragma unroll
      for (int r = 0; r < kRowChunk; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[r][i] = 0.f;
#pragma unroll
      for (int u = 0; u < kSlotUnroll; ++u) {
        const long j = start + u * 16 + wave * 4 + sub;
        if (j < end) {
          float vf[8];
          unpack8(vreg[u], vf);
#pragma unroll
          for (int r = 0; r < kRowChunk; ++r) {
            if (r < nr) {
              const float p = sc[(r0 + r) * kMaxSplit + (j - start)];
#pragma unroll
              for (int i = 0; i < 8; ++i) acc[r][i] = fmaf(p, vf[i], acc[r][i]);
            }
          }
        }
      }
      // fold the four slot rows of the wave, then the four waves through LDS
#pragma unroll
      for (int r = 0; r < kRowChunk; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          acc[r][i] += __shfl_xor(acc[r][i], 16, kWave);
          acc[r][i] += __shfl_xor(acc[r][i], 32, kWave);
        }
      if (sub == 0) {
#pragma unroll
        for (int r = 0; r < kRowChunk; ++r)
#pragma unroll
          for (int i = 0; i < 8; ++i) accr[(wave * kRowChunk + r) * D + e * 8 + i] = acc[r][i];
      }
      __syncthreads();
      for (int i = tid; i < nr * D; i += kBlock) {
        const int r = i / D, d = i % D;
        const float v = (accr[(0 * kRowChunk + r) * D + d] + accr[(1 * kRowChunk + r) * D + d]) +
                        (accr[(2 * kRowChunk + r) * D + d] + accr[(3 * kRowChunk + r) * D + d]);
        const int rr = r0 + r;
        const int h = kvh * a.G + rr / a.Q, t = rr % a.Q;
        const long orow = (static_cast<long>(b) * a.Hq + h) * a.Q + t;
        if (a.splits == 1) {
          a.out[orow * D + d] = static_cast<bf16_t>(f2bf(v / lrow[rr]));
        } else {
          a.part[(orow * a.splits + s) * D + d] = v;
          if (d == 0) {
            a.ml[(orow * a.splits + s) * 2] = mrow[rr];
            a.ml[(orow * a.splits + s) * 2 + 1] = lrow[rr];
          }
        }
      }
      __syncthreads();
    }
  }

}

// Merge of the split partials, one block per output row (b, h, t):
//   out = sum_s exp(m_s - M) acc_s / sum_s exp(m_s - M) l_s,  M = max_s m_s,
// over the splits that hold visible slots. Runs as its own launch after the
// partial kernel, so the partials are visible without any in-kernel fence.
__global__ __launch_bounds__(kBlock) void attention_merge(const float* __restrict__ part,
                                                          const float* __restrict__ ml,
                                                          const int64_t* __restrict__ pos, int Q,
                                                          long cap, int split, int splits,
                                                          bf16_t* __restrict__ out) {
  __shared__ float red[4];
  __shared__ float lsum[4];
  __shared__ float2 accs[4][D / 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long orow = blockIdx.x;
  int64_t maxpos = -1;
  for (int t = 0; t < Q; ++t) maxpos = pos[t] > maxpos ? pos[t] : maxpos;
  if (maxpos >= cap) maxpos = cap - 1;
  const int nact = maxpos < 0 ? 0 : (static_cast<int>(maxpos / split) + 1 < splits
                                         ? static_cast<int>(maxpos / split) + 1 : splits);
  const float* mlr = ml + orow * splits * 2;
  const float* pr = part + orow * splits * D;
  float m = -INFINITY;
  for (int i = tid; i < nact; i += kBlock) m = fmaxf(m, mlr[2 * i]);
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float2 acc = make_float2(0.f, 0.f);
  float l = 0.f;
  for (int s0 = wave; s0 < nact; s0 += 4 * kMergeUnroll) {
    float2 pv[kMergeUnroll];
    float mv[kMergeUnroll], lv[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const int sp = s0 + 4 * u;
      const int sc = sp < nact ? sp : s0;
      pv[u] = *reinterpret_cast<const float2*>(pr + static_cast<long>(sc) * D + 2 * lane);
      mv[u] = sp < nact ? mlr[2 * sc] : -INFINITY;
      lv[u] = mlr[2 * sc + 1];
    }
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const float w = mv[u] == -INFINITY ? 0.f : expf(mv[u] - m);
      acc.x = fmaf(w, pv[u].x, acc.x);
      acc.y = fmaf(w, pv[u].y, acc.y);
      l = fmaf(w, lv[u], l);
    }
  }
  accs[wave][lane] = acc;
  if (lane == 0) lsum[wave] = l;
  __syncthreads();
  if (wave == 0) {
    const float lt = (lsum[0] + lsum[1]) + (lsum[2] + lsum[3]);
    const float2 a0 = accs[0][lane], a1 = accs[1][lane], a2 = accs[2][lane], a3 = accs[3][lane];
    out[orow * D + 2 * lane] = static_cast<bf16_t>(f2bf(((a0.x + a1.x) + (a2.x + a3.x)) / lt));
    out[orow * D + 2 * lane + 1] = static_cast<bf16_t>(f2bf(((a0.y + a1.y) + (a2.y + a3.y)) / lt));
  }
}

// Split size: about two blocks per CU over (batch, kv head, split), slices of
// 32..64 cache slots (a 64-slot slice is one register-resident pass: four
// 16-slot groups per wave).
void choose_split(long B, long Hkv, long rows, long cap, int* split, int* splits) {
  const long target = 2L * device_cus();
  long per_head = target / (B * Hkv);
  if (per_head < 1) per_head = 1;
  const long want = (cap + per_head - 1) / per_head;
  long sz = 32;
  while (sz < want && sz < kMaxSplit) sz <<= 1;
  (void)rows;
  *split = static_cast<int>(sz);
  *splits = static_cast<int>((cap + sz - 1) / sz);
}

size_t attention_lds(int rows, int split) {
  (void)split;
  return static_cast<size_t>(rows) * D * 4 + static_cast<size_t>(rows) * kMaxSplit * 4 +
         4 * kRowChunk * D * 4 + 2 * kMaxRows * 4 + 2 * D * 2 + 16;
}

}  // namespace htn

using namespace htn;

namespace {

int run_attention(bool fused, AttnArgs& a, void* scratch, hipStream_t st) {
  const int rows = a.G * a.Q;
  if (rows <= 0 || rows > kMaxRows || a.B <= 0 || a.Hkv <= 0 || a.cap <= 0) return HTN_EUNSUPPORTED;
  choose_split(a.B, a.Hkv, rows, a.cap, &a.split, &a.splits);
  if (a.splits > 1 && !scratch) return HTN_EINVAL;
  const long nrow = static_cast<long>(a.B) * a.Hq * a.Q * a.splits;
  a.part = static_cast<float*>(scratch);
  a.ml = a.part ? a.part + nrow * D : nullptr;
  a.scale = 1.0f / sqrtf(static_cast<float>(D));
  const dim3 grid(a.splits, a.Hkv, a.B);
  const size_t lds = attention_lds(rows, a.split);
  if (fused)
    hipLaunchKernelGGL(attention_kernel<true>, grid, dim3(kBlock), lds, st, a);
  else
    hipLaunchKernelGGL(attention_kernel<false>, grid, dim3(kBlock), lds, st, a);
  if (a.splits == 1 || launch_status() != HTN_OK) return launch_status();
  hipLaunchKernelGGL(attention_merge, dim3(static_cast<long>(a.B) * a.Hq * a.Q), dim3(kBlock), 0, st,
                     a.part, a.ml, a.pos, a.Q, a.cap, a.split, a.splits, a.out);
  return launch_status();
}

}  // namespace

extern "C" int64_t htn_attention_scratch_bytes(int64_t B, int64_t Hq, int64_t Q, int64_t cap) {
  if (B <= 0 || Hq <= 0 || Q <= 0 || cap <= 0) return 0;
  // Worst case over kv-head counts dividing Hq: the split grows with Hkv * B.
  int split = 0, splits = 0;
  choose_split(B, 1, Hq * Q, cap, &split, &splits);
  int split_min = 32;
  const long most = (cap + split_min - 1) / split_min;
  const long n = static_cast<long>(B) * Hq * Q * (most > splits ? most : splits);
  return n * (D + 2) * 4;
}

extern "C" int htn_norm_rope_cache(const void* q, int64_t q_sb, int64_t q_st, const void* k,
                                   int64_t k_sb, int64_t k_st, const void* v, int64_t v_sb,
                                   int64_t v_st, const void* q_gain, const void* k_gain,
                                   float q_eps, float k_eps, const void* cos, const void* sin,
                                   int64_t rope_st, int64_t rope_rows, int rope_by_position,
                                   void* keys, void* values, int64_t cap,
                                   const int64_t* positions, void* out_q, void* out_k,
                                   int64_t B, int64_t T, int64_t Hq, int64_t Hkv,
                                   htn_stream_t stream) {
  if (!q || !k || !q_gain || !k_gain || !cos || !sin || !out_q) return HTN_EINVAL;
  if ((rope_by_position || keys) && !positions) return HTN_EINVAL;
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || rope_rows <= 0) return HTN_EINVAL;
  if ((keys || values) && (!keys || !values || !v || cap <= 0)) return HTN_EINVAL;
  RopeArgs a{};
  a.q = static_cast<const bf16_t*>(q); a.q_sb = q_sb; a.q_st = q_st;
  a.k = static_cast<const bf16_t*>(k); a.k_sb = k_sb; a.k_st = k_st;
  a.v = static_cast<const bf16_t*>(v); a.v_sb = v_sb; a.v_st = v_st;
  a.qg = static_cast<const bf16_t*>(q_gain); a.kg = static_cast<const bf16_t*>(k_gain);
  a.q_eps = q_eps; a.k_eps = k_eps;
  a.cos = static_cast<const bf16_t*>(cos); a.sin = static_cast<const bf16_t*>(sin);
  a.rope_st = rope_st; a.rope_rows = rope_rows; a.rope_by_pos = rope_by_position;
  a.keys = static_cast<bf16_t*>(keys); a.values = static_cast<bf16_t*>(values); a.cap = cap;
  a.pos = positions;
  a.out_q = static_cast<bf16_t*>(out_q); a.out_k = static_cast<bf16_t*>(out_k);
  a.B = static_cast<int>(B); a.T = static_cast<int>(T);
  a.Hq = static_cast<int>(Hq); a.Hkv = static_cast<int>(Hkv);
  const long total = B * T * (Hq + Hkv);
  hipLaunchKernelGGL(norm_rope_cache_kernel, dim3((total + 3) / 4), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status();
}

extern "C" int htn_grouped_attention(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                                     const void* keys, const void* values, int64_t cap,
                                     const int64_t* positions, void* out, int64_t B, int64_t Hq,
                                     int64_t Hkv, int64_t Q, void* scratch,
                                     htn_stream_t stream) {
  if (!q || !keys || !values || !positions || !out) return HTN_EINVAL;
  if (Hkv <= 0 || Hq % Hkv != 0 || Q <= 0) return HTN_EINVAL;
  AttnArgs a{};
  a.q = static_cast<const bf16_t*>(q); a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.keys = static_cast<bf16_t*>(const_cast<void*>(keys));
  a.values = static_cast<bf16_t*>(const_cast<void*>(values));
  a.cap = cap; a.pos = positions; a.out = static_cast<bf16_t*>(out);
  a.B = static_cast<int>(B); a.Hq = static_cast<int>(Hq); a.Hkv = static_cast<int>(Hkv);
  a.G = static_cast<int>(Hq / Hkv); a.Q = static_cast<int>(Q);
  return run_attention(false, a, scratch, static_cast<hipStream_t>(stream));
}

extern "C" int htn_prologue_attention(const void* qkv, int64_t qkv_sb, int64_t k_off,
                                      int64_t v_off, const void* q_gain, const void* k_gain,
                                      float q_eps, float k_eps, const void* cos, const void* sin,
                                      int64_t rope_st, int64_t rope_rows, int rope_by_position,
                                      void* keys, void* values, int64_t cap,
                                      const int64_t* positions, void* out, int64_t B,
                                      int64_t Hkv, int64_t groups, void* scratch,
                                      htn_stream_t stream) {
  if (!qkv || !q_gain || !k_gain || !cos || !sin || !keys || !values || !positions || !out)
    return HTN_EINVAL;
  if (Hkv <= 0 || groups <= 0 || rope_rows <= 0) return HTN_EINVAL;
  AttnArgs a{};
  a.qkv = static_cast<const bf16_t*>(qkv); a.qkv_sb = qkv_sb; a.k_off = k_off; a.v_off = v_off;
  a.qg = static_cast<const bf16_t*>(q_gain); a.kg = static_cast<const bf16_t*>(k_gain);
  a.q_eps = q_eps; a.k_eps = k_eps;
  a.cos = static_cast<const bf16_t*>(cos); a.sin = static_cast<const bf16_t*>(sin);
  a.rope_st = rope_st; a.rope_rows = rope_rows; a.rope_by_pos = rope_by_position;
  a.keys = static_cast<bf16_t*>(keys); a.values = static_cast<bf16_t*>(values);
  a.cap = cap; a.pos = positions; a.out = static_cast<bf16_t*>(out);
  a.B = static_cast<int>(B); a.Hkv = static_cast<int>(Hkv); a.G = static_cast<int>(groups);
  a.Hq = static_cast<int>(Hkv * groups); a.Q = 1;
  return run_attention(true, a, scratch, static_cast<hipStream_t>(stream));
}
