// Decode attention for gfx950 (head_dim 128).
//
//  * qk-norm + RoPE: one wave per 128-wide head; lane l owns elements l and
//    l + 64, which are exactly the rotate_half partners, so RoPE needs no
//    cross-lane traffic and the sum of squares is one DPP reduction.
//  * grouped attention: grid (split, kv head, batch). A block loads the G*Q
//    query rows of its kv head once, streams its slice of K then V with
//    16-byte loads (16 lanes per 256-byte cache row, four rows per wave
//    instruction), keeps scores in LDS for an exact two-pass softmax, and
//    writes an unnormalised partial plus (max, sum), merged per output row
//    with log-sum-exp weights. Workgroups are dispatched to the XCDs
//    round-robin, so the grid is laid out XCD-affine: every split of one
//    (batch, kv head) pair runs on the same XCD, and the last of them to
//    finish merges the pair's rows out of that XCD's L2 (the partials never
//    need to be visible to other XCDs, so no agent-scope release, which is an
//    L2 write-back on gfx950, is ever issued). Without that layout a second
//    launch merges the partials.
//  * slots after a query's absolute position are masked; slots after the
//    largest position are never read.
//  * the fused prologue variant computes q and the newest k/v from the packed
//    projection row, appends k/v to the cache, and feeds the newest slot from
//    LDS so the appended row is never re-read from memory.
#include "common.h"

#include <stdlib.h>

#include <atomic>
#include <vector>

namespace htn {

constexpr int D = HTN_HEAD_DIM;
constexpr int kMaxRows = 32;        // G * Q
constexpr int kSplit = 64;          // cache slots per tile
constexpr int kMinSplit = 16;       // fewest slots a block is given
constexpr int kMaxQ = 8;            // queries per launch (verify rows)
constexpr int kMergeUnroll = 16;    // partials loaded back to back in the merge
// Arrival counters of the in-kernel merge, at the head of the scratch buffer:
// one 128-byte line per (batch, kv head) pair, a 64-bit counter at its start.
constexpr int kCounterStride = 32;  // uint32 words
constexpr int kMaxCounterPairs = 256;
// After the counters, still in the region that starts zero and is left zero
// by every call, the fused output projection's 64-bit row accumulators (at
// most kOMaxRows output rows); the split partials follow the region.
constexpr long kOAccByte = static_cast<long>(kMaxCounterPairs) * kCounterStride * 4;
constexpr long kOMaxRows = 8192;
constexpr long kCounterBytes = kOAccByte + kOMaxRows * 8;
static_assert(kCounterBytes == HTN_ATTENTION_COUNTER_BYTES, "counter region size");
static_assert(kOAccByte == HTN_ATTENTION_OUTPUT_ACC_BYTE, "accumulator offset");
// Pair p's 64-bit counter sits at the start of its 128-byte line; the XCD
// mismatch count is the 32-bit word right after pair 0's counter.
constexpr long kXcdMismatchByte = HTN_ATTENTION_XCD_MISMATCH_BYTE;
// The fused output projection's words for pair p (at most 8 pairs) sit in
// counter line kReadyLine + p, apart from the pair's arrival counter (the
// output blocks poll them; polls on the counter's line slow its atomics):
// the ready word (nonzero once every split of the pair has stored its
// partial: 0x100 | the XCC_ID they ran on), and the count of the pair's
// output blocks that have read it (the last one clears both). The word at
// HTN_ATTENTION_OUTPUT_ERROR_BYTE of the region counts output blocks that
// could not use their pair's partials (another XCD, or no arrival in time).
constexpr int kReadyLine = 128, kReadyWord = 0, kReadersWord = 1;
constexpr long kOutputErrorByte = HTN_ATTENTION_OUTPUT_ERROR_BYTE;
static_assert(kXcdMismatchByte >= 8 && kXcdMismatchByte + 4 <= kCounterStride * 4,
              "mismatch word inside pair 0's line, past its counter");
static_assert(48 < 64, "six bits per XCD hold up to 48 splits");
static_assert(kMaxQ == 8, "load_pos8 reads eight positions");

// Per-head RMSNorm then RoPE (rotate_half), reference rounding:
//   n = bf16(g * bf16(x * inv)); out_i = bf16(bf16(n_i cos_i) + bf16(rot(n)_i sin_i)).
// 16 lanes per 128-wide head: lane e owns elements 4e..4e+3 and their
// rotate_half partners 64+4e..64+4e+3 (8-byte accesses), so RoPE needs no
// cross-lane traffic and the sum of squares is one 16-lane DPP row sum. Every
// kernel that normalises q or k uses these two functions, so the cache rows and
// queries they produce are bit-identical.
struct Head16 {
  uint2 xa, xb, ga, gb, ca, cb, sa, sb;
};

__device__ __forceinline__ void head16_load(const bf16_t* x, const bf16_t* g, const bf16_t* cs,
                                            const bf16_t* sn, int e, Head16& h) {
  h.xa = *reinterpret_cast<const uint2*>(x + 4 * e);
  h.xb = *reinterpret_cast<const uint2*>(x + 64 + 4 * e);
  h.ga = *reinterpret_cast<const uint2*>(g + 4 * e);
  h.gb = *reinterpret_cast<const uint2*>(g + 64 + 4 * e);
  h.ca = *reinterpret_cast<const uint2*>(cs + 4 * e);
  h.cb = *reinterpret_cast<const uint2*>(cs + 64 + 4 * e);
  h.sa = *reinterpret_cast<const uint2*>(sn + 4 * e);
  h.sb = *reinterpret_cast<const uint2*>(sn + 64 + 4 * e);
}

__device__ __forceinline__ void unpack4(uint2 v, float* o) {
  o[0] = bf_lo(v.x); o[1] = bf_hi(v.x); o[2] = bf_lo(v.y); o[3] = bf_hi(v.y);
}

// The head's sum of squares, the same in all 16 lanes of the row (every
// 16-lane row that calls it must be whole: DPP reduction).
__device__ __forceinline__ float head16_ss(uint2 x_a, uint2 x_b) {
  float xa[4], xb[4];
  unpack4(x_a, xa); unpack4(x_b, xb);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss = fmaf(xa[i], xa[i], ss);
#pragma unroll
  for (int i = 0; i < 4; ++i) ss = fmaf(xb[i], xb[i], ss);
  return row16_sum(ss);
}

__device__ __forceinline__ float head16_inv(float ss, float eps) {
  return 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
}

// Norm and RoPE of one head from unpacked operands and its 1 / rms: g, c, s
// hold this lane's gain, cos and sin elements 4e..4e+3 in [0..3] and their
// partners 64+4e.. in [4..7].
__device__ __forceinline__ void head16_finish(uint2 x_a, uint2 x_b, float inv, const float* g,
                                              const float* c, const float* s, uint2& oa,
                                              uint2& ob) {
  float xa[4], xb[4];
  unpack4(x_a, xa); unpack4(x_b, xb);
  const float *ga = g, *gb = g + 4, *ca = c, *cb = c + 4, *sa = s, *sb = s + 4;
  // Every rounding is done two values per v_cvt_pk_bf16_f32 (round_bf2):
  // the same bits as one at a time, fewer instructions.
  float na[4], nb[4], ra[4], rb[4], t0[4], t1[4];
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    round_bf2(xa[i] * inv, xa[i + 1] * inv, t0[i], t0[i + 1]);
    round_bf2(xb[i] * inv, xb[i + 1] * inv, t1[i], t1[i + 1]);
  }
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    round_bf2(ga[i] * t0[i], ga[i + 1] * t0[i + 1], na[i], na[i + 1]);
    round_bf2(gb[i] * t1[i], gb[i + 1] * t1[i + 1], nb[i], nb[i + 1]);
  }
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    round_bf2(na[i] * ca[i], na[i + 1] * ca[i + 1], t0[i], t0[i + 1]);
    round_bf2(-nb[i] * sa[i], -nb[i + 1] * sa[i + 1], t1[i], t1[i + 1]);
    ra[i] = t0[i] + t1[i];
    ra[i + 1] = t0[i + 1] + t1[i + 1];
    round_bf2(nb[i] * cb[i], nb[i + 1] * cb[i + 1], t0[i], t0[i + 1]);
    round_bf2(na[i] * sb[i], na[i + 1] * sb[i + 1], t1[i], t1[i + 1]);
    rb[i] = t0[i] + t1[i];
    rb[i + 1] = t0[i + 1] + t1[i + 1];
  }
  oa = make_uint2(pack_bf2(ra[0], ra[1]), pack_bf2(ra[2], ra[3]));
  ob = make_uint2(pack_bf2(rb[0], rb[1]), pack_bf2(rb[2], rb[3]));
}

// Norm and RoPE of one head from unpacked operands (16-lane rows whole).
__device__ __forceinline__ void head16_math_f(uint2 x_a, uint2 x_b, const float* g,
                                              const float* c, const float* s, float eps,
                                              uint2& oa, uint2& ob) {
  head16_finish(x_a, x_b, head16_inv(head16_ss(x_a, x_b), eps), g, c, s, oa, ob);
}

// All 64 lanes must call this (16-lane DPP reduction).
__device__ __forceinline__ void head16_math(const Head16& h, float eps, uint2& oa, uint2& ob) {
  float g[8], c[8], s[8];
  unpack4(h.ga, g); unpack4(h.gb, g + 4);
  unpack4(h.ca, c); unpack4(h.cb, c + 4);
  unpack4(h.sa, s); unpack4(h.sb, s + 4);
  head16_math_f(h.xa, h.xb, g, c, s, eps, oa, ob);
}

// Per-lane choice between two kernel arguments (q or k gain, q or k
// epsilon). A plain select of two arguments is folded into a per-lane load of
// the argument itself, a memory round trip ahead of the loads it addresses;
// an opaque SGPR value in between keeps the arguments scalar. The gain is
// reached as an offset from the q gain, so it stays a global address.
__device__ __forceinline__ const bf16_t* pick_gain(const bf16_t* qg, const bf16_t* kg, bool k) {
  long d = kg - qg;
  asm("" : "+s"(d));
  return qg + (k ? d : 0);
}
__device__ __forceinline__ float sgpr_f32(float f) {
  asm("" : "+s"(f));
  return f;
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

// One wave per (token, chunk of up to 16 heads): q chunks first, then k
// chunks, which also move the token's v rows into the cache. The wave loads
// and unpacks the gain and the token's cos/sin row once; its four 16-lane
// rows take heads h0 + row + 4j. Heads past the chunk's end recompute a valid
// head (a 16-lane row must run whole) and store nothing. The launch keeps
// tokens * chunks below 2^31.
__global__ __launch_bounds__(kBlock) void norm_rope_cache_kernel(RopeArgs a) {
  // Arguments in scalar registers at entry: one round of scalar loads.
  asm volatile("" ::"s"(a.q), "s"(a.q_sb), "s"(a.q_st), "s"(a.k), "s"(a.k_sb), "s"(a.k_st),
               "s"(a.v), "s"(a.v_sb), "s"(a.v_st), "s"(a.qg), "s"(a.kg), "s"(a.pos));
  asm volatile("" ::"s"(a.cos), "s"(a.sin), "s"(a.rope_st), "s"(a.rope_rows), "s"(a.keys),
               "s"(a.values), "s"(a.cap), "s"(a.B), "s"(a.T), "s"(a.Hq), "s"(a.Hkv));
  asm volatile("" ::"s"(a.q_eps), "s"(a.k_eps), "s"(a.rope_by_pos), "s"(a.out_q), "s"(a.out_k));
  const int lane = threadIdx.x & 63, e = lane & 15, row = lane >> 4;
  const unsigned qc = (a.Hq + 15) >> 4, chunks = qc + ((a.Hkv + 15) >> 4);
  const unsigned w = blockIdx.x * (kBlock / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned tok = w / chunks;
  if (tok >= static_cast<unsigned>(a.B) * static_cast<unsigned>(a.T)) return;
  const unsigned c = w - tok * chunks;
  const unsigned b = tok / static_cast<unsigned>(a.T);
  const int t = static_cast<int>(tok - b * static_cast<unsigned>(a.T));
  const bool is_q = c < qc;
  const int nh = is_q ? a.Hq : a.Hkv;
  const int h0 = static_cast<int>(is_q ? c : c - qc) * 16;
  const int nj = nh - h0 >= 16 ? 4 : (nh - h0 + 3) / 4;  // passes of the four rows
  // Positions are only read when they select the rope row or the cache slot.
  const int64_t p = (a.rope_by_pos || a.keys) ? a.pos[t] : t;
  const long rr = a.rope_by_pos ? p : t;
  if (rr < 0 || rr >= a.rope_rows) return;  // no rope row: the token stores nothing
  const bool append = !is_q && a.keys && p >= 0 && p < a.cap;

  const bf16_t* src = is_q ? a.q + b * a.q_sb + t * a.q_st : a.k + b * a.k_sb + t * a.k_st;
  const bf16_t* vsrc = a.v + b * a.v_sb + t * a.v_st;
  uint2 xa[4], xb[4], va[4], vb[4];
  int hh[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int h = h0 + row + 4 * j;
    hh[j] = h;
    if (j < nj) {  // wave-uniform
      const int hc = h < nh ? h : nh - 1;
      xa[j] = load_stream8(src + hc * D + 4 * e);  // read once: streaming loads
      xb[j] = load_stream8(src + hc * D + 64 + 4 * e);
      if (append) {
        va[j] = load_stream8(vsrc + hc * D + 4 * e);
        vb[j] = load_stream8(vsrc + hc * D + 64 + 4 * e);
      }
    }
  }
  const bf16_t* gain = is_q ? a.qg : a.kg;
  const bf16_t* cs = a.cos + rr * a.rope_st;
  const bf16_t* sn = a.sin + rr * a.rope_st;
  float g[8], co[8], si[8];
  unpack4(*reinterpret_cast<const uint2*>(gain + 4 * e), g);
  unpack4(*reinterpret_cast<const uint2*>(gain + 64 + 4 * e), g + 4);
  unpack4(*reinterpret_cast<const uint2*>(cs + 4 * e), co);
  unpack4(*reinterpret_cast<const uint2*>(cs + 64 + 4 * e), co + 4);
  unpack4(*reinterpret_cast<const uint2*>(sn + 4 * e), si);
  unpack4(*reinterpret_cast<const uint2*>(sn + 64 + 4 * e), si + 4);
  const float eps = is_q ? a.q_eps : a.k_eps;

  // The four passes' 1 / rms from one evaluation: lane e of a row holds pass
  // e & 3's sum of squares, and quad_perm [j,j,j,j] hands pass j's result
  // back to every lane of the row (same bits as one evaluation per pass).
  float ssj[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) ssj[j] = j < nj ? head16_ss(xa[j], xb[j]) : 1.0f;
  const int js = e & 3;
  const float sel = js == 0 ? ssj[0] : js == 1 ? ssj[1] : js == 2 ? ssj[2] : ssj[3];
  const float invs = head16_inv(sel, eps);
  float invj[4];
  invj[0] = dpp<0x00>(invs);
  invj[1] = dpp<0x55>(invs);
  invj[2] = dpp<0xAA>(invs);
  invj[3] = dpp<0xFF>(invs);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j >= nj) break;  // wave-uniform
    const int h = hh[j];
    uint2 oa, ob;
    head16_finish(xa[j], xb[j], invj[j], g, co, si, oa, ob);
    if (h >= nh) continue;
    if (is_q) {
      bf16_t* dst = a.out_q + (static_cast<long>(tok) * a.Hq + h) * D;
      *reinterpret_cast<uint2*>(dst + 4 * e) = oa;
      *reinterpret_cast<uint2*>(dst + 64 + 4 * e) = ob;
      continue;
    }
    if (a.out_k) {
      bf16_t* dst = a.out_k + (static_cast<long>(tok) * a.Hkv + h) * D;
      *reinterpret_cast<uint2*>(dst + 4 * e) = oa;
      *reinterpret_cast<uint2*>(dst + 64 + 4 * e) = ob;
    }
    if (append) {
      const long slot = ((static_cast<long>(b) * a.Hkv + h) * a.cap + p) * D;
      *reinterpret_cast<uint2*>(a.keys + slot + 4 * e) = oa;
      *reinterpret_cast<uint2*>(a.keys + slot + 64 + 4 * e) = ob;
      *reinterpret_cast<uint2*>(a.values + slot + 4 * e) = va[j];
      *reinterpret_cast<uint2*>(a.values + slot + 64 + 4 * e) = vb[j];
    }
  }
}

// Device positions read by wave-uniform index with scalar loads. They
// complete on the scalar counter, so waiting for them never waits for the
// K/V loads issued before: vector loads complete in issue order, and a
// position read as a plain load (the compiler cannot prove it unwritten by
// the kernel's LDS-direct loads, so it becomes a vector load) makes the first
// use wait for every load in flight. Positions are written by earlier
// launches (or the host) and only read here.
__device__ __forceinline__ int64_t load_pos(const int64_t* pos, int i) {
  const int64_t* p = pos + i;
  int64_t v;
  asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p));
  return v;
}

// pos[min(t, q - 1)] for t < kMaxQ: eight scalar loads in flight, one wait.
__device__ __forceinline__ void load_pos8(const int64_t* pos, int q, int64_t (&v)[8]) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int64_t* p = pos + (t < q ? t : q - 1);
    asm volatile("s_load_dwordx2 %0, %1, 0x0" : "=s"(v[t]) : "s"(p));
  }
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+s"(v[0]), "+s"(v[1]), "+s"(v[2]), "+s"(v[3]), "+s"(v[4]), "+s"(v[5]),
                 "+s"(v[6]), "+s"(v[7]));
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
  bf16_t* out;          // row (b, h, t) at b*o_sb + h*o_sh + t*o_st (dims contiguous)
  long o_sb, o_sh, o_st;
  float* part;          // [B, Hq, Q, splits, D]
  float* ml;            // [B, Hq, Q, splits, 2]
  int B, Hq, Hkv, G, Q, splits, split, stream;
  int ring;             // LDS-staged kernel: tiles staged ahead (0: other kernels)
  int mfma;             // LDS-staged kernel: tiles on the matrix cores
  float scale;
  unsigned* done;       // arrival counters: XCD-affine grid, in-kernel merge (else null)
  // Blocks from attn_blocks on read the next projection's weights (pf_units
  // spans of pf_unit_bytes; span u is multiplied by GEMV blocks on the XCD of
  // attention blocks with index u mod 8) so they wait in that XCD's L2.
  const unsigned char* pf;
  long pf_units;
  int pf_unit_bytes, pf_per_class, attn_blocks;
  // Output projection fused in (one sequence, in-kernel merge): o_blocks
  // blocks per pair past the attention grid, on the pair's XCD, multiply the
  // pair's columns of W_o (ow: [o_n, Hq D] bf16 or 8-bit, format o_fmt) by
  // the pair's attention rows and add them into the row accumulators.
  const unsigned char* ow;
  unsigned long long* oacc;  // [o_n] row accumulators, zero between launches
  int o_fmt, o_n, o_blocks, o_lpr;
  // The contribution that completes a row applies the 8-bit row scale,
  // rounds, adds the residual res_o and rounds into out_o:
  // bf16(bf16(sum) + residual) (projection.py:64-67).
  const float* o_scale;
  const bf16_t* res_o;
  bf16_t* out_o;
};

typedef __attribute__((address_space(3))) void lds_void_t;

// Prefetch role of the blocks past the attention grid: LDS-direct loads of
// the block's spans into its (otherwise unused) staging LDS, nothing
// multiplied or stored; the loads only have to pass through the XCD's L2.
// Every load has landed before the block ends (its LDS is then released).
__device__ __forceinline__ void prefetch_next(const AttnArgs& a, unsigned char* lds) {
  const int p = static_cast<int>(blockIdx.x) - a.attn_blocks;
  const int cls = p & 7, q = p >> 3;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  lds_void_t* dst = (lds_void_t*)(lds + wave * 1024);
  for (long u = cls + 8L * q; u < a.pf_units; u += 8L * a.pf_per_class) {
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.pf + u * a.pf_unit_bytes,
                                                  static_cast<uint32_t>(a.pf_unit_bytes));
    for (int o = wave * 1024; o < a.pf_unit_bytes; o += kBlock * 16)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, lane * 16, o, 0, 0);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// The kernel arguments the staged attention kernels read before their first
// vector load, named as scalar operands at entry: the compiler then issues
// their scalar loads as one round instead of one dependent round per use
// (four rounds, each a cold scalar-cache miss, before the first K/V load).
template <bool FUSED>
__device__ __forceinline__ void preload_args(const AttnArgs& a) {
  asm volatile("" ::"s"(a.pf), "s"(a.attn_blocks), "s"(a.done), "s"(a.splits), "s"(a.split),
               "s"(a.Hkv), "s"(a.B), "s"(a.G), "s"(a.cap), "s"(a.keys), "s"(a.values),
               "s"(a.pos));
  if constexpr (FUSED)
    asm volatile("" ::"s"(a.qkv), "s"(a.qkv_sb), "s"(a.k_off), "s"(a.v_off), "s"(a.qg),
                 "s"(a.kg), "s"(a.cos), "s"(a.sin));
  else
    asm volatile("" ::"s"(a.q), "s"(a.q_sb), "s"(a.q_sh), "s"(a.q_st), "s"(a.Q));
}

// Block coordinates (split s, kv head, batch). With the in-kernel merge the
// grid is one-dimensional: block L runs on XCD L % 8 (round-robin dispatch;
// on 1, 2 or 4 XCDs blocks with equal L % 8 still share one), and the splits
// of pair p = b * Hkv + kvh take blocks L = ((p / 8) * splits + s) * 8 + p % 8.
// Blocks past the last pair (pairs are padded to a multiple of 8) return false.
__device__ __forceinline__ bool split_coords(const AttnArgs& a, int& s, int& kvh, int& b) {
  if (!a.done) {
    s = blockIdx.x;
    kvh = blockIdx.y;
    b = blockIdx.z;
    return true;
  }
  // The divisions run on the vector unit: readfirstlane keeps the results
  // (block-uniform) in scalar registers for the descriptors built from them.
  const int L = blockIdx.x, j = L >> 3;
  const int g = __builtin_amdgcn_readfirstlane(j / a.splits);
  s = j - g * a.splits;
  const int p = g * 8 + (L & 7);
  b = __builtin_amdgcn_readfirstlane(p / a.Hkv);
  kvh = p - b * a.Hkv;
  return p < a.B * a.Hkv;
}

// Agent-scope (sc1) loads: they miss the CU's L1, so they observe what other
// CUs of this XCD stored to its L2.
__device__ __forceinline__ float2 load_f2_sc1(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                              uint32_t soff = 0) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 16);
  return make_float2(__uint_as_float(v.x), __uint_as_float(v.y));
}

// One output row of the in-kernel merge with every load in flight at once:
// lane j holds split j's (max, sum); N >= S partials per lane (past S the
// descriptor reads zeros, and those splits weigh 0).
template <int N>
__device__ __forceinline__ void merge_row_short(__amdgpu_buffer_rsrc_t prs, __amdgpu_buffer_rsrc_t mrs,
                                                int S, int lane, float& num_x, float& num_y,
                                                float& den) {
  // One lane offset for every load; split u's D floats u * D * 4 bytes on
  // (a constant offset, not one register per split).
  const uint32_t lo = static_cast<uint32_t>(lane) * 8;
  const float2 ml = load_f2_sc1(mrs, lo);
  float2 pv[N];
#pragma unroll
  for (int u = 0; u < N; ++u) pv[u] = load_f2_sc1(prs, lo, u * D * 4);
  __builtin_amdgcn_sched_barrier(0);  // all loads issued before the first wait
  const float M = wave_max(lane < S ? ml.x : -INFINITY);
  const float w = lane < S && ml.x != -INFINITY ? expf(ml.x - M) : 0.f;
  den = wave_sum(w * ml.y);
  num_x = num_y = 0.f;
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const float wu = readlane(w, u);
    num_x = fmaf(wu, pv[u].x, num_x);
    num_y = fmaf(wu, pv[u].y, num_y);
  }
}

// End of a split block on the XCD-affine grid. Every thread's partial stores
// have completed in the XCD's L2 before the block counts itself in; the block
// that brings its pair's count to `splits` merges the pair's G * Q rows (one
// wave per row) and rearms the counter for the next launch:
//   out = sum_s w_s acc_s / sum_s w_s l_s,  w_s = exp(m_s - M),  M = max_s m_s.
// Every load of a row is in flight at once (the host takes this path for at
// most four rows of at most 48 splits).
//
// The pair's 64-bit counter holds one 6-bit arrival count per XCD: a split
// adds 1 << (6 * its XCC_ID), so the block that completes the count also
// sees where every split ran. Were any split of the pair on another XCD
// than the merging block (dispatch not round-robin), its partial might not be
// visible in this L2: the merge still runs, and the mismatch count at byte
// kXcdMismatchByte of the counters is incremented for the host to read.
__device__ __forceinline__ void merge_tail(const AttnArgs& a, int b, int kvh, int* last) {
  // Everything the merge needs is computed before the arrival: the code after
  // it runs on one block per pair, cold in its CU's instruction cache, so it
  // is kept to the loads, the arithmetic and the store. The host takes this
  // path for at most four rows (one per wave).
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int p = b * a.Hkv + kvh;
  const int R = a.G * a.Q, S = a.splits;
  const int r = wave < R ? wave : 0;
  const long orow = static_cast<long>(p) * R + r;
  const float* prow = a.part + orow * S * D;
  const float* mrow = a.ml + orow * S * 2;
  const int h = kvh * a.G + r / a.Q, t = r % a.Q;
  bf16_t* dst = a.out + b * a.o_sb + h * a.o_sh + t * a.o_st + 2 * lane;
  asm volatile("" ::"s"(prow), "s"(mrow), "v"(dst), "s"(S));
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  unsigned long long* cnt =
      reinterpret_cast<unsigned long long*>(a.done + static_cast<long>(p) * kCounterStride);
  if (threadIdx.x == 0) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 7u;
    const unsigned long long mine = 1ull << (6 * xcc);
    const unsigned long long total =
        __hip_atomic_fetch_add(cnt, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + mine;
    unsigned arrived = 0;
#pragma unroll
    for (int x = 0; x < 8; ++x) arrived += static_cast<unsigned>(total >> (6 * x)) & 63u;
    const bool done = arrived == static_cast<unsigned>(a.splits);
    *last = done;
    if (done && total != static_cast<unsigned long long>(a.splits) << (6 * xcc))
      __hip_atomic_fetch_add(a.done + kXcdMismatchByte / 4, 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!*last) return;
  if (a.ow) {
    // Fused output projection: the pair's output blocks merge the rows
    // themselves. Every partial is in this XCD's L2; tell them so.
    if (threadIdx.x == 0) {
      unsigned xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
      __hip_atomic_store(a.done + static_cast<long>(kReadyLine + p) * kCounterStride + kReadyWord,
                         0x100u | (xcc & 0xffu), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(cnt, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  if (wave < R) {
    const __amdgpu_buffer_rsrc_t prs = buffer_rsrc(prow, static_cast<uint32_t>(S) * D * 4);
    const __amdgpu_buffer_rsrc_t mrs = buffer_rsrc(mrow, static_cast<uint32_t>(S) * 8);
    float nx, ny, den;
    // The fewest loads that cover the splits (each is a wave instruction
    // even where the descriptor returns zeros).
    if (S <= 8) merge_row_short<8>(prs, mrs, S, lane, nx, ny, den);
    else if (S <= 16) merge_row_short<16>(prs, mrs, S, lane, nx, ny, den);
    else if (S <= 24) merge_row_short<24>(prs, mrs, S, lane, nx, ny, den);
    else if (S <= 32) merge_row_short<32>(prs, mrs, S, lane, nx, ny, den);
    else merge_row_short<48>(prs, mrs, S, lane, nx, ny, den);
    *reinterpret_cast<uint32_t*>(dst) = pack_bf2(nx / den, ny / den);
  }
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte agent-scope loads (see load_f2_sc1).
__device__ __forceinline__ float4 load_f4_sc1(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                              uint32_t soff = 0) {
  typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
  const u32x4v v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 16);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                     __uint_as_float(v.w));
}

// v(lane) + v(lane ^ 32) in every lane (v_permlane32_swap of two copies).
__device__ __forceinline__ float swap_sum32(float v) {
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// merge_row_short with 16-byte loads, two splits per wave instruction:
// lanes 0-31 read split 2u, lanes 32-63 split 2u + 1, four dims per lane
// (NP pairs cover 2 NP >= S splits); the halves' sums are added at the end,
// so lane l < 32 holds dims 4 l .. 4 l + 3 of the row. Half the load
// instructions of merge_row_short (8B decode step 2.789 -> 2.772 ms with the
// fused output projection, whose blocks merge after the last split lands).
template <int NP>
__device__ __forceinline__ void merge_row_wide(__amdgpu_buffer_rsrc_t prs, __amdgpu_buffer_rsrc_t mrs,
                                               int S, int lane, float4& num, float& den) {
  const uint32_t half = static_cast<uint32_t>(lane) >> 5;
  const uint32_t lo = (static_cast<uint32_t>(lane) & 31u) * 16u + half * D * 4;
  const float2 ml = load_f2_sc1(mrs, static_cast<uint32_t>(lane) * 8);
  float4 pv[NP];
#pragma unroll
  for (int u = 0; u < NP; ++u) pv[u] = load_f4_sc1(prs, lo, u * 2 * D * 4);
  __builtin_amdgcn_sched_barrier(0);  // all loads issued before the first wait
  const float M = wave_max(lane < S ? ml.x : -INFINITY);
  const float w = lane < S && ml.x != -INFINITY ? expf(ml.x - M) : 0.f;
  den = wave_sum(w * ml.y);
  float4 n = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const float w0 = readlane(w, 2 * u), w1 = readlane(w, 2 * u + 1);
    const float wu = half ? w1 : w0;
    n.x = fmaf(wu, pv[u].x, n.x);
    n.y = fmaf(wu, pv[u].y, n.y);
    n.z = fmaf(wu, pv[u].z, n.z);
    n.w = fmaf(wu, pv[u].w, n.w);
  }
  num = make_float4(swap_sum32(n.x), swap_sum32(n.y), swap_sum32(n.z), swap_sum32(n.w));
}

// The merged row r of pair p (one wave), merge_tail's formula, into `arow`
// (64 words, word i holding the bf16 pair of dims 2 i, 2 i + 1).
__device__ __forceinline__ void merge_row_to(const AttnArgs& a, int p, int r, int lane,
                                             uint32_t* arow) {
  const int R = a.G * a.Q, S = a.splits;
  const long orow = static_cast<long>(p) * R + r;
  const __amdgpu_buffer_rsrc_t prs =
      uniform_rsrc(a.part + orow * S * D, static_cast<uint32_t>(S) * D * 4);
  const __amdgpu_buffer_rsrc_t mrs = uniform_rsrc(a.ml + orow * S * 2, static_cast<uint32_t>(S) * 8);
  // The host fuses the projection for at most kOMaxSplits splits, which
  // keeps the merge's loads and the block's weights within the registers.
  float4 nm;
  float den;
  if (S <= 8) merge_row_wide<4>(prs, mrs, S, lane, nm, den);
  else if (S <= 16) merge_row_wide<8>(prs, mrs, S, lane, nm, den);
  else merge_row_wide<12>(prs, mrs, S, lane, nm, den);
  if (lane < 32) {
    arow[2 * lane] = pack_bf2(nm.x / den, nm.y / den);
    arow[2 * lane + 1] = pack_bf2(nm.z / den, nm.w / den);
  }
}

// The fused output projection (one sequence): block o past the attention
// grid serves pair p = o % 8 (the XCD column of the pair's splits) and
// output rows [128 (o / 8), + 128). Each lane group of 16 lanes owns one row
// at a time: lane j holds bytes 16 j + 256 c (c < LPR) of the row's span of
// the pair's columns (G D weights), eight rows per group, all 8 LPR 16-byte
// loads issued at once, before the wait. When the pair's last split has
// stored its partial, the block merges the pair's G attention rows (the
// bf16 rows the unfused kernel writes, merge_tail's arithmetic) into LDS,
// takes its dot products, reduces each over the 16 lanes, and adds the row
// sums into the rows' accumulators, where the pairs' partials meet.
constexpr int kORowsPerGroup = 8;
// Smallest output projection fused: the 8B decode step's 33.6 MB and the 8-bit
// lines' 16.8 MB gain (2.841 -> 2.730 ms, int8 462 -> 486 tok/s at 8K). The
// 0.6B shape's 4 MiB gains 0.6% too, but its 64-step golden decode then flips
// a token (deficit 0.022) that the oracle's own evaluation orders do not
// explain, so it keeps the separate GEMV.
constexpr long kFuseMinBytes = 16L << 20;
constexpr int kOMaxSplits = 24;
constexpr int kORowsPerBlock = 4 * 4 * kORowsPerGroup;  // 128
constexpr int kOMaxPolls = 1 << 16;

// Adds one pair's contribution (fixed-point partial + 2^60) to output row
// `row`'s accumulator; the contribution that completes the pair count
// finishes the row and clears the word.
// `res` and `scale` are the row's residual and 8-bit row scale (1 for bf16
// weights), loaded before the block waited.
__device__ __forceinline__ void output_row_add(const AttnArgs& a, int row,
                                               unsigned long long add, double to_fix, float res,
                                               float scale) {
  const unsigned long long tot =
      __hip_atomic_fetch_add(a.oacc + row, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
  const unsigned k = static_cast<unsigned>((tot + (1ull << 59)) >> 60);
  if (k == static_cast<unsigned>(a.Hkv)) {
    const long long S = static_cast<long long>(tot - (static_cast<unsigned long long>(k) << 60));
    float sum = static_cast<float>(static_cast<double>(S) / to_fix);
    if (a.o_scale) sum *= scale;
    a.out_o[row] = static_cast<bf16_t>(f2bf(round_bf(sum) + res));
    __hip_atomic_store(a.oacc + row, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int WF, int LPR>
__device__ __forceinline__ void output_block(const AttnArgs& a, uint32_t* alds) {
  constexpr int kB = Fmt<WF>::kBytes;
  // Fixed point of the row partials: kFix fraction bits, |partial| < 2^(56 -
  // kFix), so eight pairs' partials and the count in bits 60-63 cannot carry
  // into each other.
  constexpr int kFix = WF == WF_BF16 ? 32 : 24;
  constexpr float kMaxPartial = static_cast<float>(1ull << (56 - kFix));
  const double to_fix = static_cast<double>(1ull << kFix);
  constexpr int kXW = WF == WF_BF16 ? 4 : 8;  // activation words per 16-byte weight load
  const int o = static_cast<int>(blockIdx.x) - a.attn_blocks;
  const int p = o & 7, q = o >> 3;
  if (p >= a.Hkv) return;  // no pair on this XCD column
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, j = lane & 15;
  unsigned* line = a.done + static_cast<long>(kReadyLine + p) * kCounterStride;
  // 1. The block's weights, all in flight at once (rows past o_n read zeros),
  // issued about a microsecond after the attention blocks' first K/V loads
  // (8B decode step at context 2048: 2.817 -> 2.798 ms; none or two
  // microseconds were slower, and so were three to seven at context 8192).
  __builtin_amdgcn_s_sleep(40);
  const uint32_t row_bytes = static_cast<uint32_t>(a.Hq) * D * kB;
  const __amdgpu_buffer_rsrc_t wrs =
      buffer_rsrc(a.ow, static_cast<uint32_t>(a.o_n) * row_bytes);
  const uint32_t col0 = static_cast<uint32_t>(p * a.G * D * kB) + 16u * j;
  const int row0 = q * kORowsPerBlock + wave * 4 * kORowsPerGroup + g;
  uint4 w[kORowsPerGroup][LPR];
#pragma unroll
  for (int it = 0; it < kORowsPerGroup; ++it) {
    const uint32_t voff = static_cast<uint32_t>(row0 + 4 * it) * row_bytes + col0;
#pragma unroll
    for (int c = 0; c < LPR; ++c) w[it][c] = buffer_load16_stream(wrs, voff + 256u * c, 0);
  }
  // The epilogue operands of the row this lane may finish (lane j < 8 of
  // each group: row it = j), behind the weights.
  const int frow = row0 + 4 * j;
  const int erow = frow < a.o_n ? frow : a.o_n - 1;
  const float res = bf2f(a.res_o[erow]);
  const float scale = a.o_scale ? a.o_scale[erow] : 1.f;
  // 2. Wait for the pair's splits (wave 0 polls, bounded).
  __shared__ unsigned ready;
  if (wave == 0) {
    unsigned v = 0;
    for (int i = 0; i < kOMaxPolls; ++i) {
      v = __hip_atomic_load(line + kReadyWord, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (v) break;
      __builtin_amdgcn_s_sleep(8);
    }
    if (lane == 0) ready = v;
  }
  __syncthreads();
  const unsigned rv = ready;
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  if (rv == 0 || (rv & 0xffu) != (xcc & 0xffu)) {
    // The partials are not visible here: count the failure for the host and
    // add only the count to the block's rows, so they complete (without this
    // pair's share) and their accumulators are cleared as usual.
    if (threadIdx.x == 0)
      __hip_atomic_fetch_add(a.done + kOutputErrorByte / 4, 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (j < kORowsPerGroup && frow < a.o_n) output_row_add(a, frow, 1ull << 60, to_fix, res, scale);
    return;
  }
  // 3. The pair's attention rows into LDS, then this block is done with the
  // ready word: the last of the pair's output blocks clears it.
  const int R = a.G;
  if (wave < R) merge_row_to(a, p, wave, lane, alds + wave * (D / 2));
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned n =
        __hip_atomic_fetch_add(line + kReadersWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
    if (n == static_cast<unsigned>(a.o_blocks)) {
      __hip_atomic_store(line + kReadersWord, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(line + kReadyWord, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // 4. Dot products: weight byte 16 j + 256 c of the span is column
  // (16 j + 256 c) / kB of the pair, whose bf16 activation sits at byte
  // 2 (16 j + 256 c) / kB of the staged rows.
  uint32_t x[LPR][kXW];
#pragma unroll
  for (int c = 0; c < LPR; ++c) {
    const uint32_t* src = alds + (2 * (16 * j + 256 * c) / kB) / 4;
#pragma unroll
    for (int u = 0; u < kXW; ++u) x[c][u] = src[u];
  }
  // 5. Each row's partial joins the other pairs' in one 64-bit word per
  // output row: the fp32 partial in fixed point (kFix fraction bits) plus
  // 2^60, added by one returning agent-scope atomic, which is performed at
  // the coherent level, so the XCDs' contributions meet without any L2
  // write-back. Integer addition is associative: whatever the arrival
  // order, the word ends as the exact sum of the pairs' partials, and the
  // contribution that brings the count in bits 60-63 to the pair count
  // sees that sum in its own return value. It finishes the row -- fp32 sum,
  // 8-bit row scale, bf16, + residual, bf16 (projection.py:64-67) -- and
  // clears the word for the next launch. The sum is rounded once to fp32
  // instead of after every pair: a summation order the reference's "any
  // order" contract allows (kernels/projection.py:25).
  // Lane j < 8 of each group adds row it = j's sum: the group's eight
  // returning atomics go out together.
  float mine = 0.f;
#pragma unroll
  for (int it = 0; it < kORowsPerGroup; ++it) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < LPR; ++c) s = dot_vec<WF>(w[it][c], x[c], s);
    s = row16_sum(s);  // in all 16 lanes of the group
    if (j == it) mine = s;
  }
  if (j < kORowsPerGroup && frow < a.o_n) {
    if (!(fabsf(mine) < kMaxPartial)) {  // out of the fixed-point range (or NaN)
      __hip_atomic_fetch_add(a.done + kOutputErrorByte / 4, 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      mine = 0.f;
    }
    output_row_add(a, frow,
                   static_cast<unsigned long long>(__double2ll_rn(static_cast<double>(mine) * to_fix)) +
                       (1ull << 60),
                   to_fix, res, scale);
  }
}

// Dispatch on the weight format and the span's 16-byte loads per lane.
__device__ __forceinline__ void output_role(const AttnArgs& a, uint32_t* alds) {
  if (a.o_fmt == WF_BF16) {
    if (a.o_lpr == 4) output_block<WF_BF16, 4>(a, alds);
    else if (a.o_lpr == 2) output_block<WF_BF16, 2>(a, alds);
    else output_block<WF_BF16, 1>(a, alds);
  } else if (a.o_fmt == WF_INT8) {
    if (a.o_lpr == 4) output_block<WF_INT8, 4>(a, alds);
    else if (a.o_lpr == 2) output_block<WF_INT8, 2>(a, alds);
    else output_block<WF_INT8, 1>(a, alds);
  } else {
    if (a.o_lpr == 4) output_block<WF_FP8, 4>(a, alds);
    else if (a.o_lpr == 2) output_block<WF_FP8, 2>(a, alds);
    else output_block<WF_FP8, 1>(a, alds);
  }
}

// The block's result per query row of the LDS-staged kernels, one wave per
// row (r = wave, wave + 4, ...: wave-uniform, so the per-row state is read
// by broadcast and its weights are computed once per wave): the four waves'
// states weighted by exp2(m_w - M), M = max_w m_w, lane l holding dims 2l
// and 2l + 1. With one split it is the output row; otherwise the split's
// partial and its (max, sum), the max back to base e for the merge. Row r is
// head r / Q, query r % Q of kv head kvh (one query unless MQ).
template <int ROWS, bool MQ>
__device__ __forceinline__ void write_rows(const AttnArgs& a, int b, int kvh, int s, int rows,
                                           int wave, int lane, const float (*wm)[ROWS],
                                           const float (*wl)[ROWS],
                                           const float (*wacc)[ROWS][D]) {
  constexpr int W = kBlock / kWave;
  for (int r = wave; r < rows; r += W) {
    float mw[W];
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      mw[w] = wm[w][r];
      M = fmaxf(M, mw[w]);
    }
    float nx = 0.f, ny = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = mw[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw[w] - M);
      const float2 v = *reinterpret_cast<const float2*>(&wacc[w][r][2 * lane]);
      nx = fmaf(f, v.x, nx);
      ny = fmaf(f, v.y, ny);
      den = fmaf(f, wl[w][r], den);
    }
    const int h = kvh * a.G + (MQ ? r / a.Q : r), t = MQ ? r % a.Q : 0;
    if (a.splits == 1) {
      bf16_t* dst = a.out + b * a.o_sb + h * a.o_sh + t * a.o_st + 2 * lane;
      dst[0] = static_cast<bf16_t>(f2bf(nx / den));
      dst[1] = static_cast<bf16_t>(f2bf(ny / den));
    } else {
      const long orow = (static_cast<long>(b) * a.Hq + h) * a.Q + t;
      *reinterpret_cast<float2*>(a.part + (orow * a.splits + s) * D + 2 * lane) =
          make_float2(nx, ny);
      if (lane == 0)
        *reinterpret_cast<float2*>(a.ml + (orow * a.splits + s) * 2) =
            make_float2(M * 0.6931471805599453f, den);
    }
  }
}

// Query source of the partial kernel: q rows from memory, or the fused
// prologue over the packed projection row with the RoPE row either already
// selected (row 0 of cos/sin) or looked up by the device position.
enum Prologue { PRO_NONE = 0, PRO_ROW = 1, PRO_BY_POSITION = 2 };

// Split-KV partial attention for one (split of 64 slots, kv head, batch).
// ROWS query rows (G heads x Q queries) are processed per chunk; K is read
// with 16 lanes per 256-byte row (q.k as bf16 dot2 steps finishing with DPP
// row sums), V with one wave per 16 slots and 4 bytes per lane (P.V needs no
// cross-lane reduction). K and V are read through buffer descriptors over the
// (batch, kv head) cache rows: slots past the capacity read as zeros, so the
// tile loads need no per-lane clamping. Splits past the last position write
// neutral partials (max -inf, sum 0) so the merge never needs the positions.
//
// Load order matters: vector loads complete in issue order, so a wait for one
// load waits for every load issued before it. The small loads that gate the
// query rows go first (unless their address needs the device position), then
// K, then V; positions are scalar loads on their own counter. Every load is
// unconditional: a branch that joins with fewer loads in flight, or a load
// under a per-lane condition, makes the compiler wait for all of them.
//
// TILES 64-slot tiles per block (2 when one tile per block would need more
// blocks than fit on the GPU at once): all tiles' loads are issued up front
// and the softmax spans the block's 64 * TILES slots.
template <int ROWS, int PRO, int TILES>
__global__ __launch_bounds__(kBlock) void attention_partial(AttnArgs a) {
  constexpr bool FUSED = PRO != PRO_NONE;
  preload_args<FUSED>(a);
  constexpr int SPLIT = kSplit * TILES;
  constexpr int kQLoads = kMaxRows * (D / 2) / kBlock;  // q pairs per thread, unfused
  __shared__ uint32_t qs[kMaxRows * D / 2];  // query rows as bf16 pairs
  __shared__ float sc[ROWS * SPLIT];
  __shared__ float accr[4 * ROWS * D];
  __shared__ float mrow[ROWS], lrow[ROWS];
  __shared__ int rowpos[kMaxRows];  // absolute position of each query row
  __shared__ __align__(16) bf16_t knew[D];
  __shared__ __align__(16) bf16_t vnew[D];
  __shared__ int last_split;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane >> 4, e = lane & 15;
  int s, kvh, b;
  if (!split_coords(a, s, kvh, b)) return;
  const int rows = a.G * a.Q;
  const long kv_base = (static_cast<long>(b) * a.Hkv + kvh) * a.cap * D;
  // The block owns slots [start, stop): a.split slots (at most SPLIT).
  const int start = s * a.split;
  const int stop = start + a.split < a.cap ? start + a.split : static_cast<int>(a.cap);

  // ---- 1. loads that gate the query rows.
  // Fused: 16 lanes per head slot, slots 0..G-1 the query heads, slot G the
  // new key (its value is copied at step 3).
  const int head_slot = wave * 4 + sub;
  const bool is_k = head_slot == a.G;
  const bf16_t* qrow = a.qkv + static_cast<long>(b) * a.qkv_sb;
  const bf16_t* hsrc = is_k ? qrow + a.k_off + static_cast<long>(kvh) * D
                            : qrow + (static_cast<long>(kvh) * a.G +
                                      (head_slot < a.G ? head_slot : 0)) * D;
  Head16 hq;
  if (PRO == PRO_ROW) head16_load(hsrc, pick_gain(a.qg, a.kg, is_k), a.cos, a.sin, e, hq);
  // Unfused: the q rows (bf16 pairs) and each row's position, clamped reads.
  uint32_t qv[kQLoads];
  int rpv = 0;
  if (!FUSED) {
#pragma unroll
    for (int i = 0; i < kQLoads; ++i) {
      const int idx = tid + i * kBlock;
      const int c = idx < rows * (D / 2) ? idx : 0;
      const int r = c / (D / 2), d = 2 * (c % (D / 2));
      const int h = kvh * a.G + r / a.Q, t = r % a.Q;
      qv[i] = *reinterpret_cast<const uint32_t*>(
          a.q + static_cast<long>(b) * a.q_sb + static_cast<long>(h) * a.q_sh +
          static_cast<long>(t) * a.q_st + d);
    }
    rpv = static_cast<int>(a.pos[(tid < rows ? tid : 0) % a.Q]);
  }

  // ---- 2. the split's K then V tiles (addresses from the block index only),
  // through descriptors over the block's range: slots past it read zeros
  // without touching memory. Slots past the last position are masked below
  // (scores -inf, V zeroed), so splits past it produce neutral partials with
  // no branch.
  const uint32_t range = stop > start ? static_cast<uint32_t>(stop - start) * D * 2 : 0u;
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(a.keys + kv_base + static_cast<long>(start) * D, range);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(a.values + kv_base + static_cast<long>(start) * D, range);
  uint4 kreg[4 * TILES];
  uint32_t vreg[16 * TILES];
  const uint32_t koff = static_cast<uint32_t>(((wave * 4 + sub) * D + e * 8) * 2);
#pragma unroll
  for (int u = 0; u < 4 * TILES; ++u) kreg[u] = buffer_load16(krs, koff, u * 16 * D * 2);
  const uint32_t voff = static_cast<uint32_t>((wave * 16 * D + 2 * lane) * 2);
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i)
      vreg[t * 16 + i] = buffer_load4(vrs, voff + i * D * 2, t * kSplit * D * 2);

  // Positions: scalar loads of pos[min(t, Q - 1)] (in bounds, branch-free).
  int qp[kMaxQ];
  int maxpos = -1;
  int64_t pq[kMaxQ];
  load_pos8(a.pos, a.Q, pq);
#pragma unroll
  for (int t = 0; t < kMaxQ; ++t) {
    const int64_t v = pq[t];
    // Positions outside [0, cap) never match a slot (clamped to -1 / cap).
    const int vc = v < 0 ? -1 : (v >= a.cap ? static_cast<int>(a.cap) : static_cast<int>(v));
    qp[t] = t < a.Q ? vc : -1;
    maxpos = qp[t] > maxpos ? qp[t] : maxpos;
  }
  if (maxpos >= a.cap) maxpos = static_cast<int>(a.cap) - 1;
  const int end = stop < maxpos + 1 ? stop : maxpos + 1;
  const bool active = start <= maxpos;
  const int newest = FUSED ? qp[0] : -1;
  const bool has_newest = FUSED && active && newest >= start && newest < end;
  if (PRO == PRO_BY_POSITION) {
    // The RoPE row needs the position: these loads queue behind K and V.
    const long ri = (newest >= 0 && newest < a.rope_rows) ? newest : 0;
    head16_load(hsrc, pick_gain(a.qg, a.kg, is_k), a.cos + ri * a.rope_st, a.sin + ri * a.rope_st, e, hq);
  }

  // ---- 3. query rows (and, fused, the newest k/v) into LDS
  if (FUSED) {
    const bool do_head = head_slot < a.G || (is_k && has_newest);
    uint2 oa, ob;
    head16_math(hq, is_k ? sgpr_f32(a.k_eps) : sgpr_f32(a.q_eps), oa, ob);
    if (tid < a.G) rowpos[tid] = newest;
    if (do_head && !is_k) {
      qs[head_slot * (D / 2) + 2 * e] = oa.x;
      qs[head_slot * (D / 2) + 2 * e + 1] = oa.y;
      qs[head_slot * (D / 2) + 32 + 2 * e] = ob.x;
      qs[head_slot * (D / 2) + 32 + 2 * e + 1] = ob.y;
    } else if (do_head) {
      const long slot = kv_base + static_cast<long>(newest) * D;
      const bf16_t* vsrc = qrow + a.v_off + static_cast<long>(kvh) * D;
      const uint2 va = *reinterpret_cast<const uint2*>(vsrc + 4 * e);
      const uint2 vb = *reinterpret_cast<const uint2*>(vsrc + 64 + 4 * e);
      *reinterpret_cast<uint2*>(knew + 4 * e) = oa;
      *reinterpret_cast<uint2*>(knew + 64 + 4 * e) = ob;
      *reinterpret_cast<uint2*>(vnew + 4 * e) = va;
      *reinterpret_cast<uint2*>(vnew + 64 + 4 * e) = vb;
      *reinterpret_cast<uint2*>(a.keys + slot + 4 * e) = oa;
      *reinterpret_cast<uint2*>(a.keys + slot + 64 + 4 * e) = ob;
      *reinterpret_cast<uint2*>(a.values + slot + 4 * e) = va;
      *reinterpret_cast<uint2*>(a.values + slot + 64 + 4 * e) = vb;
    }
  } else {
    if (tid < rows) rowpos[tid] = rpv;
#pragma unroll
    for (int i = 0; i < kQLoads; ++i)
      if (tid + i * kBlock < rows * (D / 2)) qs[tid + i * kBlock] = qv[i];
  }
  __syncthreads();
  if (has_newest) {  // block-uniform: the newest slot's k/v come from LDS, not memory
    const uint4 kn = *reinterpret_cast<const uint4*>(knew + e * 8);
    const uint32_t vn = *reinterpret_cast<const uint32_t*>(vnew + 2 * lane);
#pragma unroll
    for (int u = 0; u < 4 * TILES; ++u) {
      const int j = start + u * 16 + wave * 4 + sub;
      const bool hit = j == newest;
      kreg[u].x = hit ? kn.x : kreg[u].x;
      kreg[u].y = hit ? kn.y : kreg[u].y;
      kreg[u].z = hit ? kn.z : kreg[u].z;
      kreg[u].w = hit ? kn.w : kreg[u].w;
    }
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int j = start + t * kSplit + wave * 16 + i;
        vreg[t * 16 + i] = j == newest ? vn : vreg[t * 16 + i];
      }
  }

  const int len = active ? static_cast<int>(end - start) : 0;
  for (int r0 = 0; r0 < rows; r0 += ROWS) {
    float acc[ROWS][2];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r][0] = acc[r][1] = 0.f;
    // ---- 4. scores q.k * D^-1/2. Rows past `rows` (when ROWS does not
    // divide it) compute on whatever their LDS rows hold and are never stored.
    uint32_t qr[ROWS][4];
    int rp[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
#pragma unroll
      for (int i = 0; i < 4; ++i) qr[r][i] = qs[(r0 + r) * (D / 2) + e * 4 + i];
      rp[r] = rowpos[r0 + r];
    }
#pragma unroll
    for (int u = 0; u < 4 * TILES; ++u) {
      const int j = start + u * 16 + wave * 4 + sub;
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        float dot = dot2(kreg[u].x, qr[r][0], 0.f);
        dot = dot2(kreg[u].y, qr[r][1], dot);
        dot = dot2(kreg[u].z, qr[r][2], dot);
        dot = dot2(kreg[u].w, qr[r][3], dot);
        const float dsum = row16_sum(dot);
        if (e == 0 && j < end) sc[r * SPLIT + (j - start)] = j <= rp[r] ? dsum * a.scale : -INFINITY;
      }
    }
    __syncthreads();
    // ---- 5. exact softmax numerators per row over this split
#pragma unroll
    for (int r = wave; r < ROWS; r += 4) {
      float v[TILES];
      float m = -INFINITY;
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        const int js = t * kSplit + lane;
        v[t] = js < len ? sc[r * SPLIT + js] : -INFINITY;
        m = fmaxf(m, v[t]);
      }
      m = wave_max(m);
      float l = 0.f;
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        const int js = t * kSplit + lane;
        const float p = (js < len && m != -INFINITY) ? expf(v[t] - m) : 0.f;
        sc[r * SPLIT + js] = p;
        l += p;
      }
      l = wave_sum(l);
      if (lane == 0) {
        mrow[r] = m;
        lrow[r] = l;
      }
    }
    __syncthreads();
    // ---- 6. P.V: wave w owns slots w*16 .. w*16+15 of the split, each lane 2 dims;
    // slots past the end carry p = 0 and a zeroed V row (the cache may hold
    // anything there, NaN included).
#pragma unroll
    for (int i = 0; i < 16 * TILES; ++i) {
      const int js = (i / 16) * kSplit + wave * 16 + (i % 16);
      const uint32_t vv = js < len ? vreg[i] : 0u;
      const float v0 = bf_lo(vv), v1 = bf_hi(vv);
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        const float p = sc[r * SPLIT + js];
        acc[r][0] = fmaf(p, v0, acc[r][0]);
        acc[r][1] = fmaf(p, v1, acc[r][1]);
      }
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      accr[(wave * ROWS + r) * D + 2 * lane] = acc[r][0];
      accr[(wave * ROWS + r) * D + 2 * lane + 1] = acc[r][1];
    }
    __syncthreads();
    for (int i = tid; i < ROWS * D; i += kBlock) {
      const int r = i / D, d = i % D;
      const int rr = r0 + r;
      if (rr < rows) {
        const float v = (accr[(0 * ROWS + r) * D + d] + accr[(1 * ROWS + r) * D + d]) +
                        (accr[(2 * ROWS + r) * D + d] + accr[(3 * ROWS + r) * D + d]);
        const int h = kvh * a.G + rr / a.Q, t = rr % a.Q;
        const long orow = (static_cast<long>(b) * a.Hq + h) * a.Q + t;
        if (a.splits == 1) {
          a.out[b * a.o_sb + h * a.o_sh + t * a.o_st + d] = static_cast<bf16_t>(f2bf(v / lrow[r]));
        } else {
          a.part[(orow * a.splits + s) * D + d] = v;
          if (d == 0) {
            a.ml[(orow * a.splits + s) * 2] = mrow[r];
            a.ml[(orow * a.splits + s) * 2 + 1] = lrow[r];
          }
        }
      }
    }
    __syncthreads();
  }
  if (a.done) merge_tail(a, b, kvh, &last_split);
}

// Streaming split-KV attention for long contexts: a block owns T (even)
// consecutive 64-slot tiles and keeps the next tile's K/V loads in flight
// while it scores, normalises and accumulates the current one (online
// softmax: running max and sum per row, accumulators rescaled per tile).
// The buffer descriptors cover exactly the block's slot range, so tiles
// past it read zeros without touching memory; loads stay unconditional.
// Rows = G * Q must fit one chunk (<= ROWS). Query rows, positions and the
// fused prologue are as in attention_partial.
struct KVTile {
  uint4 k[4];
  uint32_t v[16];
};

__device__ __forceinline__ void issue_tile(__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                           uint32_t koff, uint32_t voff, int ti, KVTile& t) {
  const uint32_t tb = static_cast<uint32_t>(ti) * kSplit * D * 2;
#pragma unroll
  for (int u = 0; u < 4; ++u) t.k[u] = buffer_load16(krs, koff, tb + u * 16 * D * 2);
#pragma unroll
  for (int i = 0; i < 16; ++i) t.v[i] = buffer_load4(vrs, voff + i * D * 2, tb);
}

template <int ROWS>
__device__ __forceinline__ void stream_tile(const AttnArgs& a, KVTile& t, int tbase, int tend,
                                            bool has_newest, int newest, const uint4& kn,
                                            uint32_t vn, const uint32_t (&qr)[ROWS][4],
                                            const int (&rp)[ROWS], float* scb, float* mrun,
                                            float* lrun, float* alph, float (&acc)[ROWS][2]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane >> 4, e = lane & 15;
  if (has_newest && newest >= tbase && newest < tbase + kSplit) {  // block-uniform
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool hit = tbase + u * 16 + wave * 4 + sub == newest;
      t.k[u].x = hit ? kn.x : t.k[u].x;
      t.k[u].y = hit ? kn.y : t.k[u].y;
      t.k[u].z = hit ? kn.z : t.k[u].z;
      t.k[u].w = hit ? kn.w : t.k[u].w;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) t.v[i] = tbase + wave * 16 + i == newest ? vn : t.v[i];
  }
  // scores
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int j = tbase + u * 16 + wave * 4 + sub;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float dot = dot2(t.k[u].x, qr[r][0], 0.f);
      dot = dot2(t.k[u].y, qr[r][1], dot);
      dot = dot2(t.k[u].z, qr[r][2], dot);
      dot = dot2(t.k[u].w, qr[r][3], dot);
      const float dsum = row16_sum(dot);
      if (e == 0 && j < tend) scb[r * kSplit + (j - tbase)] = j <= rp[r] ? dsum * a.scale : -INFINITY;
    }
  }
  __syncthreads();
  // online softmax: wave w updates rows w, w + 4
  const int lt = tend - tbase;
  const int len = lt < 0 ? 0 : (lt > kSplit ? kSplit : lt);
#pragma unroll
  for (int r = wave; r < ROWS; r += 4) {
    const float v = lane < len ? scb[r * kSplit + lane] : -INFINITY;
    const float m_old = mrun[r];
    const float m_new = fmaxf(m_old, wave_max(v));
    const float alpha = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
    const float p = (lane < len && m_new != -INFINITY) ? expf(v - m_new) : 0.f;
    scb[r * kSplit + lane] = p;
    const float l = wave_sum(p);
    if (lane == 0) {
      mrun[r] = m_new;
      lrun[r] = fmaf(lrun[r], alpha, l);
      alph[r] = alpha;
    }
  }
  __syncthreads();
  // P.V (slots past the end carry p = 0 and a zeroed V row)
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const float al = alph[r];
    acc[r][0] *= al;
    acc[r][1] *= al;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int js = wave * 16 + i;
    const uint32_t vv = js < len ? t.v[i] : 0u;
    const float v0 = bf_lo(vv), v1 = bf_hi(vv);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const float p = scb[r * kSplit + js];
      acc[r][0] = fmaf(p, v0, acc[r][0]);
      acc[r][1] = fmaf(p, v1, acc[r][1]);
    }
  }
}

template <int ROWS, int PRO>
__global__ __launch_bounds__(kBlock) void attention_stream(AttnArgs a) {
  constexpr bool FUSED = PRO != PRO_NONE;
  preload_args<FUSED>(a);
  __shared__ uint32_t qs[kMaxRows * D / 2];
  __shared__ float sc[2][ROWS * kSplit];
  __shared__ float accr[4 * ROWS * D];
  __shared__ float mrun[ROWS], lrun[ROWS], alph[ROWS];
  __shared__ int rowpos[kMaxRows];
  __shared__ __align__(16) bf16_t knew[D];
  __shared__ __align__(16) bf16_t vnew[D];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane >> 4, e = lane & 15;
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int rows = a.G * a.Q;
  const long kv_base = (static_cast<long>(b) * a.Hkv + kvh) * a.cap * D;
  const int start = s * a.split;
  const int stop = start + a.split < a.cap ? start + a.split : static_cast<int>(a.cap);
  const int ntiles = ((a.split + kSplit - 1) / kSplit + 1) & ~1;  // even

  // ---- 1. loads that gate the query rows (as in attention_partial)
  const int head_slot = wave * 4 + sub;
  const bool is_k = head_slot == a.G;
  const bf16_t* qrow = a.qkv + static_cast<long>(b) * a.qkv_sb;
  const bf16_t* hsrc = is_k ? qrow + a.k_off + static_cast<long>(kvh) * D
                            : qrow + (static_cast<long>(kvh) * a.G +
                                      (head_slot < a.G ? head_slot : 0)) * D;
  Head16 hq;
  if (PRO == PRO_ROW) head16_load(hsrc, pick_gain(a.qg, a.kg, is_k), a.cos, a.sin, e, hq);
  uint32_t qv = 0;
  int rpv = 0;
  if (!FUSED) {
    const int c = tid < rows * (D / 2) ? tid : 0;  // rows <= 4 here: one pair per thread
    const int r = c / (D / 2), d = 2 * (c % (D / 2));
    const int h = kvh * a.G + r / a.Q, tq = r % a.Q;
    qv = *reinterpret_cast<const uint32_t*>(a.q + static_cast<long>(b) * a.q_sb +
                                            static_cast<long>(h) * a.q_sh +
                                            static_cast<long>(tq) * a.q_st + d);
    rpv = static_cast<int>(a.pos[(tid < rows ? tid : 0) % a.Q]);
  }

  // ---- 2. the first two tiles of the block's range
  const uint32_t range = stop > start ? static_cast<uint32_t>(stop - start) * D * 2 : 0u;
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(a.keys + kv_base + static_cast<long>(start) * D, range);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(a.values + kv_base + static_cast<long>(start) * D, range);
  const uint32_t koff = static_cast<uint32_t>(((wave * 4 + sub) * D + e * 8) * 2);
  const uint32_t voff = static_cast<uint32_t>((wave * 16 * D + 2 * lane) * 2);
  KVTile ta, tb;
  issue_tile(krs, vrs, koff, voff, 0, ta);
  issue_tile(krs, vrs, koff, voff, 1, tb);

  int qp[kMaxQ];
  int maxpos = -1;
  int64_t pq[kMaxQ];
  load_pos8(a.pos, a.Q, pq);
#pragma unroll
  for (int t = 0; t < kMaxQ; ++t) {
    const int64_t v = pq[t];
    // Positions outside [0, cap) never match a slot (clamped to -1 / cap).
    const int vc = v < 0 ? -1 : (v >= a.cap ? static_cast<int>(a.cap) : static_cast<int>(v));
    qp[t] = t < a.Q ? vc : -1;
    maxpos = qp[t] > maxpos ? qp[t] : maxpos;
  }
  if (maxpos >= a.cap) maxpos = static_cast<int>(a.cap) - 1;
  const int end = stop < maxpos + 1 ? stop : maxpos + 1;
  const bool active = start <= maxpos;
  const int newest = FUSED ? qp[0] : -1;
  const bool has_newest = FUSED && active && newest >= start && newest < end;
  if (PRO == PRO_BY_POSITION) {
    const long ri = (newest >= 0 && newest < a.rope_rows) ? newest : 0;
    head16_load(hsrc, pick_gain(a.qg, a.kg, is_k), a.cos + ri * a.rope_st, a.sin + ri * a.rope_st, e, hq);
  }

  // ---- 3. query rows (and, fused, the newest k/v) into LDS
  if (FUSED) {
    const bool do_head = head_slot < a.G || (is_k && has_newest);
    uint2 oa, ob;
    head16_math(hq, is_k ? sgpr_f32(a.k_eps) : sgpr_f32(a.q_eps), oa, ob);
    if (tid < a.G) rowpos[tid] = newest;
    if (do_head && !is_k) {
      qs[head_slot * (D / 2) + 2 * e] = oa.x;
      qs[head_slot * (D / 2) + 2 * e + 1] = oa.y;
      qs[head_slot * (D / 2) + 32 + 2 * e] = ob.x;
      qs[head_slot * (D / 2) + 32 + 2 * e + 1] = ob.y;
    } else if (do_head) {
      const long slot = kv_base + static_cast<long>(newest) * D;
      const bf16_t* vsrc = qrow + a.v_off + static_cast<long>(kvh) * D;
      const uint2 va = *reinterpret_cast<const uint2*>(vsrc + 4 * e);
      const uint2 vb = *reinterpret_cast<const uint2*>(vsrc + 64 + 4 * e);
      *reinterpret_cast<uint2*>(knew + 4 * e) = oa;
      *reinterpret_cast<uint2*>(knew + 64 + 4 * e) = ob;
      *reinterpret_cast<uint2*>(vnew + 4 * e) = va;
      *reinterpret_cast<uint2*>(vnew + 64 + 4 * e) = vb;
      *reinterpret_cast<uint2*>(a.keys + slot + 4 * e) = oa;
      *reinterpret_cast<uint2*>(a.keys + slot + 64 + 4 * e) = ob;
      *reinterpret_cast<uint2*>(a.values + slot + 4 * e) = va;
      *reinterpret_cast<uint2*>(a.values + slot + 64 + 4 * e) = vb;
    }
  } else {
    if (tid < rows) rowpos[tid] = rpv;
    if (tid < rows * (D / 2)) qs[tid] = qv;
  }
  if (tid < ROWS) {
    mrun[tid] = -INFINITY;
    lrun[tid] = 0.f;
  }
  __syncthreads();
  uint4 kn = make_uint4(0, 0, 0, 0);
  uint32_t vn = 0;
  if (has_newest) {
    kn = *reinterpret_cast<const uint4*>(knew + e * 8);
    vn = *reinterpret_cast<const uint32_t*>(vnew + 2 * lane);
  }
  uint32_t qr[ROWS][4];
  int rp[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) qr[r][i] = qs[r * (D / 2) + e * 4 + i];
    rp[r] = rowpos[r];
  }
  float acc[ROWS][2];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) acc[r][0] = acc[r][1] = 0.f;

  // ---- 4. tiles, two per iteration, the next one always in flight (tiles
  // past the block's range load nothing)
#pragma unroll 1
  for (int ti = 0; ti < ntiles; ti += 2) {
    stream_tile<ROWS>(a, ta, start + ti * kSplit, end, has_newest, newest, kn, vn, qr, rp, sc[0],
                      mrun, lrun, alph, acc);
    issue_tile(krs, vrs, koff, voff, ti + 2, ta);
    stream_tile<ROWS>(a, tb, start + (ti + 1) * kSplit, end, has_newest, newest, kn, vn, qr, rp,
                      sc[1], mrun, lrun, alph, acc);
    issue_tile(krs, vrs, koff, voff, ti + 3, tb);
  }

  // ---- 5. reduce the four waves' accumulators, write the partial (or the row)
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    accr[(wave * ROWS + r) * D + 2 * lane] = acc[r][0];
    accr[(wave * ROWS + r) * D + 2 * lane + 1] = acc[r][1];
  }
  __syncthreads();
  for (int i = tid; i < ROWS * D; i += kBlock) {
    const int r = i / D, d = i % D;
    if (r < rows) {
      const float v = (accr[(0 * ROWS + r) * D + d] + accr[(1 * ROWS + r) * D + d]) +
                      (accr[(2 * ROWS + r) * D + d] + accr[(3 * ROWS + r) * D + d]);
      const int h = kvh * a.G + r / a.Q, tq = r % a.Q;
      const long orow = (static_cast<long>(b) * a.Hq + h) * a.Q + tq;
      if (a.splits == 1) {
        a.out[b * a.o_sb + h * a.o_sh + tq * a.o_st + d] = static_cast<bf16_t>(f2bf(v / lrun[r]));
      } else {
        a.part[(orow * a.splits + s) * D + d] = v;
        if (d == 0) {
          a.ml[(orow * a.splits + s) * 2] = mrun[r];
          a.ml[(orow * a.splits + s) * 2 + 1] = lrun[r];
        }
      }
    }
  }
}

// Decode attention with K/V staged through LDS (one query per sequence, up
// to 8 query rows per kv head). A block owns `nt` consecutive 64-slot tiles;
// each of its four waves owns 16 slots of every tile and loads exactly those
// K and V rows straight into its own LDS region with 16-byte LDS-direct
// buffer loads (no registers held while in flight), RING tiles ahead. A wave
// then reads back only what it loaded itself and runs its own online
// softmax, so the tile loop has no block barrier: lane (sub, e) holds dims
// 8e..8e+7 of slots 4u + sub, a score is a 16-lane DPP row sum, the tile
// maximum combines the four row groups with readlane, and P.V accumulates
// per lane. The four wave states merge in LDS at the end into the block's
// partial (or the output row when the block owns the whole cache).
//
// LDS-direct loads count on vmcnt like any vector load and complete in issue
// order. The staging ring is read only through inline-asm ds_read with an
// explicit vmcnt wait (the compiler would otherwise wait for every
// outstanding LDS-direct load before each LDS read of that buffer), and the
// block barriers are inline-asm s_barrier for the same reason; all other LDS
// traffic uses separate static arrays.
constexpr int kLdsWaveTile = 2 * 16 * D * 2;               // K + V bytes of one wave's 16 slots
constexpr int kLdsTile = kLdsWaveTile * (kBlock / kWave);  // 32 KB per 64-slot tile


__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// K then V of this wave's 16 slots of one tile: eight 1 KB LDS-direct loads.
__device__ __forceinline__ void stage_tile(__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                           unsigned char* wave_lds, int lane, uint32_t tile_off) {
#pragma unroll
  for (int u = 0; u < 4; ++u)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_t*)(wave_lds + u * 1024), 16, lane * 16,
                                             tile_off + u * 1024, 0, 0);
#pragma unroll
  for (int u = 0; u < 4; ++u)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_t*)(wave_lds + 4096 + u * 1024), 16,
                                             lane * 16, tile_off + u * 1024, 0, 0);
}

// Wait until at most WAIT vector-memory operations are outstanding, then
// read this lane's 16 bytes of K and V for the four slot quads.
template <int WAIT>
__device__ __forceinline__ void read_tile(uint32_t addr, uint4 (&ko)[4], uint4 (&vo)[4]) {
  u32x4 k[4], v[4];
  asm volatile(
      "s_waitcnt vmcnt(%8)\n\t"
      "ds_read_b128 %0, %9\n\t"
      "ds_read_b128 %1, %9 offset:1024\n\t"
      "ds_read_b128 %2, %9 offset:2048\n\t"
      "ds_read_b128 %3, %9 offset:3072\n\t"
      "ds_read_b128 %4, %9 offset:4096\n\t"
      "ds_read_b128 %5, %9 offset:5120\n\t"
      "ds_read_b128 %6, %9 offset:6144\n\t"
      "ds_read_b128 %7, %9 offset:7168\n\t"
      "s_waitcnt lgkmcnt(0)"
      // early-clobber outputs: a destination must never share the address
      // register, which the later reads of the sequence still use
      : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(v[0]), "=&v"(v[1]),
        "=&v"(v[2]), "=&v"(v[3])
      : "n"(WAIT), "v"(addr)
      : "memory");
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ko[i] = make_uint4(k[i].x, k[i].y, k[i].z, k[i].w);
    vo[i] = make_uint4(v[i].x, v[i].y, v[i].z, v[i].w);
  }
}

template <int ROWS, int PRO, int RING, bool OUT>
__global__ __launch_bounds__(kBlock) void attention_lds(AttnArgs a) {
  // OUT: the launch carries the fused output projection's blocks (their
  // weights stay in registers, so only those launches pay for them).
  constexpr bool FUSED = PRO != PRO_NONE;
  extern __shared__ __align__(16) unsigned char ring[];  // RING tiles of K/V staging
  preload_args<FUSED>(a);
  if ((a.pf || a.ow) && static_cast<int>(blockIdx.x) >= a.attn_blocks) {
    if constexpr (OUT) output_role(a, reinterpret_cast<uint32_t*>(ring));
    else prefetch_next(a, ring);
    return;
  }
  __shared__ uint32_t qs[ROWS * D / 2];
  __shared__ float wm[kBlock / kWave][ROWS], wl[kBlock / kWave][ROWS];
  __shared__ float wacc[kBlock / kWave][ROWS][D];
  __shared__ __align__(16) bf16_t knew[D];
  __shared__ __align__(16) bf16_t vnew[D];
  __shared__ int last_split;

  // The wave index is uniform: readfirstlane keeps LDS and tile offsets scalar.
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sub = lane >> 4, e = lane & 15;
  int s, kvh, b;
  if (!split_coords(a, s, kvh, b)) return;
  const int rows = a.G;
  const long kv_base = (static_cast<long>(b) * a.Hkv + kvh) * a.cap * D;
  const int start = s * a.split;
  const int stop = start + a.split < a.cap ? start + a.split : static_cast<int>(a.cap);
  const int nt = (a.split + kSplit - 1) / kSplit;

  // ---- 1. loads that gate the query rows (as in attention_partial), the
  // newest v row, then the position.
  const int head_slot = wave * 4 + sub;
  const bool is_k = head_slot == a.G;
  const bf16_t* qrow = a.qkv + static_cast<long>(b) * a.qkv_sb;
  const bf16_t* hsrc = is_k ? qrow + a.k_off + static_cast<long>(kvh) * D
                            : qrow + (static_cast<long>(kvh) * a.G +
                                      (head_slot < a.G ? head_slot : 0)) * D;
  Head16 hq;
  uint2 va = make_uint2(0, 0), vb = make_uint2(0, 0);
  if (PRO == PRO_ROW) head16_load(hsrc, pick_gain(a.qg, a.kg, is_k), a.cos, a.sin, e, hq);
  if (FUSED) {
    const bf16_t* vsrc = qrow + a.v_off + static_cast<long>(kvh) * D;
    va = *reinterpret_cast<const uint2*>(vsrc + 4 * e);
    vb = *reinterpret_cast<const uint2*>(vsrc + 64 + 4 * e);
  }
  constexpr int kQL = (ROWS * (D / 2) + kBlock - 1) / kBlock;  // q pairs per thread
  uint32_t qv[kQL];
  if (!FUSED) {
#pragma unroll
    for (int j = 0; j < kQL; ++j) {
      const int idx = tid + j * kBlock;
      const int c = idx < rows * (D / 2) ? idx : 0;
      const int h = kvh * a.G + c / (D / 2), d = 2 * (c % (D / 2));
      qv[j] = *reinterpret_cast<const uint32_t*>(a.q + static_cast<long>(b) * a.q_sb +
                                                 static_cast<long>(h) * a.q_sh + d);
    }
  }
  // ---- 2. stage the first RING tiles at once, through descriptors over the
  // block's slots up to the capacity (slots past the newest position are
  // masked below); later tiles use descriptors over the visible slots only,
  // which read as zeros past them without touching memory.
  const uint32_t cap_range = static_cast<uint32_t>(stop - start) * D * 2;
  const bf16_t* kb = a.keys + kv_base + static_cast<long>(start) * D;
  const bf16_t* vb0 = a.values + kv_base + static_cast<long>(start) * D;
  unsigned char* wave_ring = ring + wave * kLdsWaveTile;
  const uint32_t wave_off = static_cast<uint32_t>(wave) * 16 * D * 2;  // this wave's 16 slots
  {
    const __amdgpu_buffer_rsrc_t krs0 = buffer_rsrc(kb, cap_range);
    const __amdgpu_buffer_rsrc_t vrs0 = buffer_rsrc(vb0, cap_range);
#pragma unroll
    for (int t = 0; t < RING; ++t)
      stage_tile(krs0, vrs0, wave_ring + t * kLdsTile, lane, t * kSplit * D * 2 + wave_off);
  }
  const int64_t pv = load_pos(a.pos, 0);
  const int pos = pv < 0 ? -1 : (pv >= a.cap ? static_cast<int>(a.cap) : static_cast<int>(pv));
  const int last = pos < a.cap ? pos : static_cast<int>(a.cap) - 1;
  const int end = stop < last + 1 ? stop : last + 1;  // slots [start, end) are visible
  const int newest = FUSED && pos >= 0 && pos < a.cap ? pos : -1;
  const bool has_newest = newest >= start && newest < end;
  if (PRO == PRO_BY_POSITION) {
    const long ri = (newest >= 0 && newest < a.rope_rows) ? newest : 0;
    head16_load(hsrc, pick_gain(a.qg, a.kg, is_k), a.cos + ri * a.rope_st,
                a.sin + ri * a.rope_st, e, hq);
  }

  const uint32_t range = end > start ? static_cast<uint32_t>(end - start) * D * 2 : 0u;
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(kb, range);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(vb0, range);

  // ---- 3. query rows (and, fused, the newest k/v) into LDS
  if (FUSED) {
    const bool do_head = head_slot < a.G || (is_k && has_newest);
    uint2 oa, ob;
    head16_math(hq, is_k ? sgpr_f32(a.k_eps) : sgpr_f32(a.q_eps), oa, ob);
    if (do_head && !is_k) {
      qs[head_slot * (D / 2) + 2 * e] = oa.x;
      qs[head_slot * (D / 2) + 2 * e + 1] = oa.y;
      qs[head_slot * (D / 2) + 32 + 2 * e] = ob.x;
      qs[head_slot * (D / 2) + 32 + 2 * e + 1] = ob.y;
    } else if (do_head) {
      const long slot = kv_base + static_cast<long>(newest) * D;
      *reinterpret_cast<uint2*>(knew + 4 * e) = oa;
      *reinterpret_cast<uint2*>(knew + 64 + 4 * e) = ob;
      *reinterpret_cast<uint2*>(vnew + 4 * e) = va;
      *reinterpret_cast<uint2*>(vnew + 64 + 4 * e) = vb;
      *reinterpret_cast<uint2*>(a.keys + slot + 4 * e) = oa;
      *reinterpret_cast<uint2*>(a.keys + slot + 64 + 4 * e) = ob;
      *reinterpret_cast<uint2*>(a.values + slot + 4 * e) = va;
      *reinterpret_cast<uint2*>(a.values + slot + 64 + 4 * e) = vb;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kQL; ++j)
      if (tid + j * kBlock < rows * (D / 2)) qs[tid + j * kBlock] = qv[j];
  }
  lds_barrier();
  uint4 kn = make_uint4(0, 0, 0, 0), vn = make_uint4(0, 0, 0, 0);
  if (has_newest) {
    kn = *reinterpret_cast<const uint4*>(knew + e * 8);
    vn = *reinterpret_cast<const uint4*>(vnew + e * 8);
  }
  // Rows past G (ROWS rounds G up) score row 0 and are never stored.
  uint32_t qr[ROWS][4];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const int rr = r < rows ? r : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) qr[r][i] = qs[rr * (D / 2) + e * 4 + i];
  }
  const float scale2 = a.scale * 1.4426950408889634f;  // log2(e) / sqrt(D)
  float m[ROWS], l[ROWS], acc[ROWS][8];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[r][i] = 0.f;
  }

  // ---- 4. tiles: wait for this wave's staged rows of tile t (the tiles
  // staged after it may stay in flight), score, online softmax, P.V, then
  // stage tile t + RING into the slot just read.
  const uint32_t lane_addr =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)(wave_ring))) + lane * 16;
#pragma unroll 1
  for (int t = 0; t < nt; ++t) {
    const int q = t % RING;
    uint4 kt[4], vt[4];
    const int later = nt - 1 - t < RING - 1 ? nt - 1 - t : RING - 1;  // tiles staged after t
    const uint32_t at = lane_addr + q * kLdsTile;
    if (RING == 1 || later == 0) read_tile<0>(at, kt, vt);
    else if (RING == 2 || later == 1) read_tile<8>(at, kt, vt);
    else if (later == 2) read_tile<16>(at, kt, vt);
    else read_tile<24>(at, kt, vt);
    const int tbase = start + t * kSplit + wave * 16;  // this wave's first slot
    if (has_newest && newest >= tbase && newest < tbase + 16) {  // wave-uniform
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool hit = tbase + 4 * u + sub == newest;
        kt[u].x = hit ? kn.x : kt[u].x; kt[u].y = hit ? kn.y : kt[u].y;
        kt[u].z = hit ? kn.z : kt[u].z; kt[u].w = hit ? kn.w : kt[u].w;
        vt[u].x = hit ? vn.x : vt[u].x; vt[u].y = hit ? vn.y : vt[u].y;
        vt[u].z = hit ? vn.z : vt[u].z; vt[u].w = hit ? vn.w : vt[u].w;
      }
    }
    // Scores live in the base-2 domain (q.k * log2(e) / sqrt(D)) so each
    // weight is one v_exp_f32; masks are only applied on the tile that
    // crosses the end of the visible slots.
    const bool full = tbase + 16 <= end;  // wave-uniform
    float vf[4][8];
    bool ok[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      ok[u] = full || tbase + 4 * u + sub < end;
      unpack8(vt[u], vf[u]);
    }
    if (!full) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) vf[u][i] = ok[u] ? vf[u][i] : 0.f;  // never NaN * 0
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float sc[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float dot = dot2(kt[u].x, qr[r][0], 0.f);
        dot = dot2(kt[u].y, qr[r][1], dot);
        dot = dot2(kt[u].z, qr[r][2], dot);
        dot = dot2(kt[u].w, qr[r][3], dot);
        const float dsum = row16_sum(dot);
        sc[u] = ok[u] ? dsum * scale2 : -INFINITY;
        tmax = fmaxf(tmax, sc[u]);
      }
      tmax = fmaxf(fmaxf(readlane(tmax, 0), readlane(tmax, 16)),
                   fmaxf(readlane(tmax, 32), readlane(tmax, 48)));
      const float m_new = fmaxf(m[r], tmax);
      if (m_new != -INFINITY) {  // wave-uniform
        // exp2(-inf) is 0: a first tile (m = -inf) or a masked slot weighs 0
        const float alpha = __builtin_amdgcn_exp2f(m[r] - m_new);
        m[r] = m_new;
        float ls = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[r][i] *= alpha;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float pu = __builtin_amdgcn_exp2f(sc[u] - m_new);
          ls += pu;
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[r][i] = fmaf(pu, vf[u][i], acc[r][i]);
        }
        l[r] = fmaf(l[r], alpha, ls);
      }
    }
    const int tn = t + RING;
    if (tn < nt)  // wave-uniform
      stage_tile(krs, vrs, wave_ring + q * kLdsTile, lane, tn * kSplit * D * 2 + wave_off);
  }
  // Every staging load has landed before the block's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- 5. sum the four row groups (same dims, different slots), merge the
  // waves' states in LDS, write the block's partial (or the rows).
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      acc[r][i] += __shfl_xor(acc[r][i], 16, kWave);
      acc[r][i] += __shfl_xor(acc[r][i], 32, kWave);
    }
    // every lane of a row group holds that group's sum
    const float lw =
        (readlane(l[r], 0) + readlane(l[r], 16)) + (readlane(l[r], 32) + readlane(l[r], 48));
    if (lane < 16) {
#pragma unroll
      for (int i = 0; i < 8; ++i) wacc[wave][r][8 * e + i] = acc[r][i];
    }
    if (lane == 0) {
      wm[wave][r] = m[r];
      wl[wave][r] = lw;
    }
  }
  lds_barrier();
  write_rows<ROWS, false>(a, b, kvh, s, rows, wave, lane, wm, wl, wacc);
  if (a.done) merge_tail(a, b, kvh, &last_split);
}

// ------------------------------------------------------------------ matrix-core tiles
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the four quads'
// copies of one query row): gfx950's row-swap permutes, no LDS round trip.
// permlane16_swap pairs row r with row r ^ 1 and permlane32_swap the wave's
// halves; both results of each swap hold the two partners.
__device__ __forceinline__ float quad_max(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float quad_sum(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// V^T operands by transpose reads (gfx950 ds_read_b64_tr_b16). Within each
// 16-lane group the read returns to lane j element j % 4 of the 8 bytes at
// the address of lane 4 k + j / 4, for k = 0..3 (the layout a probe of the
// instruction showed). Lane (col, quad) of the P.V operand needs
// V[slot 4 quad + k][dim 16 j + col], k = 0..3; so lane i of group quad
// addresses slot 4 quad + i / 4, dims 16 j + 4 (i % 4) .. + 3, and one read
// per j returns the four elements in order.
template <int OFF>
__device__ __forceinline__ void read_vt_tr(const uint32_t (&va)[8], uint2 (&vt)[8]) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  u32x2 w[8];
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8 offset:%16\n\t"
      "ds_read_b64_tr_b16 %1, %9 offset:%16\n\t"
      "ds_read_b64_tr_b16 %2, %10 offset:%16\n\t"
      "ds_read_b64_tr_b16 %3, %11 offset:%16\n\t"
      "ds_read_b64_tr_b16 %4, %12 offset:%16\n\t"
      "ds_read_b64_tr_b16 %5, %13 offset:%16\n\t"
      "ds_read_b64_tr_b16 %6, %14 offset:%16\n\t"
      "ds_read_b64_tr_b16 %7, %15 offset:%16\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]),
        "=&v"(w[6]), "=&v"(w[7])
      : "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]), "v"(va[4]), "v"(va[5]), "v"(va[6]),
        "v"(va[7]), "n"(OFF)
      : "memory");
#pragma unroll
  for (int j = 0; j < 8; ++j) vt[j] = make_uint2(w[j].x, w[j].y);
}

// K then V of this wave's 16 slots of one tile, both rows rotated through
// per-lane source offsets (K: kvoff, chunk c of slot s at column (c + s) % 16;
// V: vvoff, at column (c + 2 (s % 8)) % 16): eight 1 KB LDS-direct loads, as
// stage_tile.
__device__ __forceinline__ void stage_tile_mf(__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                              unsigned char* wave_lds, const uint32_t (&kvoff)[4],
                                              const uint32_t (&vvoff)[4], uint32_t tile_off) {
#pragma unroll
  for (int u = 0; u < 4; ++u)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_t*)(wave_lds + u * 1024), 16, kvoff[u],
                                             tile_off, 0, 0);
#pragma unroll
  for (int u = 0; u < 4; ++u)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_t*)(wave_lds + 4096 + u * 1024), 16,
                                             vvoff[u], tile_off, 0, 0);
}

// Wait until at most WAIT vector-memory operations are outstanding, then read
// this lane's score operand (four 16-byte K chunks) and its V^T operands by
// transpose reads (read_vt_tr): element k of vt[j] is
// V[slot 4 * quad + k][dim 16 * j + col].
template <int WAIT>
__device__ __forceinline__ void read_tile_mf(const uint32_t (&kaddr)[4], const uint32_t (&vaddr)[8],
                                             uint32_t ro, uint4 (&k)[4], uint2 (&vt)[8]) {
  u32x4 k0, k1, k2, k3;
  asm volatile(
      "s_waitcnt vmcnt(%4)\n\t"
      "ds_read_b128 %0, %5\n\t"
      "ds_read_b128 %1, %6\n\t"
      "ds_read_b128 %2, %7\n\t"
      "ds_read_b128 %3, %8"
      : "=&v"(k0), "=&v"(k1), "=&v"(k2), "=&v"(k3)
      : "n"(WAIT), "v"(kaddr[0] + ro), "v"(kaddr[1] + ro), "v"(kaddr[2] + ro), "v"(kaddr[3] + ro)
      : "memory");
  uint32_t va[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) va[j] = vaddr[j] + ro;
  read_vt_tr<0>(va, vt);
  k[0] = make_uint4(k0.x, k0.y, k0.z, k0.w);
  k[1] = make_uint4(k1.x, k1.y, k1.z, k1.w);
  k[2] = make_uint4(k2.x, k2.y, k2.z, k2.w);
  k[3] = make_uint4(k3.x, k3.y, k3.z, k3.w);
}

template <int ROWS, int PRO, int RING, bool OUT>
__global__ __launch_bounds__(kBlock) void attention_mfma(AttnArgs a) {
  constexpr bool FUSED = PRO != PRO_NONE;
  extern __shared__ __align__(16) unsigned char ring[];  // RING tiles of K/V staging
  preload_args<FUSED>(a);
  if ((a.pf || a.ow) && static_cast<int>(blockIdx.x) >= a.attn_blocks) {
    if constexpr (OUT) output_role(a, reinterpret_cast<uint32_t*>(ring));
    else prefetch_next(a, ring);
    return;
  }
  // MQ: several queries per sequence (16 or 32 rows = heads x queries, each
  // with its own position); otherwise one query, up to 8 heads per kv head.
  constexpr bool MQ = ROWS > 8;
  constexpr int NT = (ROWS + 15) / 16;  // 16-row tiles of query rows
  __shared__ uint32_t qs[ROWS * D / 2];
  __shared__ float wm[kBlock / kWave][ROWS], wl[kBlock / kWave][ROWS];
  __shared__ __align__(16) bf16_t knew[D];
  __shared__ __align__(16) bf16_t vnew[D];
  __shared__ int rowpos[MQ ? ROWS : 1];  // absolute position of each query row
  __shared__ int last_split;
  // The waves' partial states: with several queries they reuse the staging
  // ring once every tile is read (the launch sizes it for both).
  __shared__ float wacc_s[MQ ? 1 : kBlock / kWave][MQ ? 1 : ROWS][D];
  float (*wacc)[ROWS][D] = MQ ? reinterpret_cast<float (*)[ROWS][D]>(ring)
                              : reinterpret_cast<float (*)[ROWS][D]>(&wacc_s[0][0][0]);

  // The wave index is uniform: readfirstlane keeps LDS and tile offsets scalar.
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sub = lane >> 4, e = lane & 15;
  int s, kvh, b;
  if (!split_coords(a, s, kvh, b)) return;
  const int rows = a.G * a.Q;
  const long kv_base = (static_cast<long>(b) * a.Hkv + kvh) * a.cap * D;
  const int start = s * a.split;
  const int stop = start + a.split < a.cap ? start + a.split : static_cast<int>(a.cap);
  const int nt = (a.split + kSplit - 1) / kSplit;

  // ---- 1. loads that gate the query rows (as in attention_partial), the
  // newest v row, then the position.
  const int head_slot = wave * 4 + sub;
  const bool is_k = head_slot == a.G;
  const bf16_t* qrow = a.qkv + static_cast<long>(b) * a.qkv_sb;
  const bf16_t* hsrc = is_k ? qrow + a.k_off + static_cast<long>(kvh) * D
                            : qrow + (static_cast<long>(kvh) * a.G +
                                      (head_slot < a.G ? head_slot : 0)) * D;
  Head16 hq;
  uint2 va = make_uint2(0, 0), vb = make_uint2(0, 0);
  if (PRO == PRO_ROW) head16_load(hsrc, pick_gain(a.qg, a.kg, is_k), a.cos, a.sin, e, hq);
  if (FUSED) {
    const bf16_t* vsrc = qrow + a.v_off + static_cast<long>(kvh) * D;
    va = *reinterpret_cast<const uint2*>(vsrc + 4 * e);
    vb = *reinterpret_cast<const uint2*>(vsrc + 64 + 4 * e);
  }
  constexpr int kQL = (ROWS * (D / 2) + kBlock - 1) / kBlock;  // q pairs per thread
  uint32_t qv[kQL];
  int rpv = 0;
  if (!FUSED) {
#pragma unroll
    for (int j = 0; j < kQL; ++j) {
      const int idx = tid + j * kBlock;
      const int c = idx < rows * (D / 2) ? idx : 0;
      const int r = c / (D / 2), d = 2 * (c % (D / 2));
      const int h = kvh * a.G + r / a.Q, t = r % a.Q;
      qv[j] = *reinterpret_cast<const uint32_t*>(a.q + static_cast<long>(b) * a.q_sb +
                                                 static_cast<long>(h) * a.q_sh +
                                                 static_cast<long>(t) * a.q_st + d);
    }
    const int64_t v = a.pos[(tid < rows ? tid : 0) % a.Q];
    rpv = v < 0 ? -1 : (v >= a.cap ? static_cast<int>(a.cap) : static_cast<int>(v));
    // Keep these loads ahead of the K/V staging: loads complete in issue
    // order, so q issued behind the tiles would wait for all of them.
    __builtin_amdgcn_sched_barrier(0);
  }
  // ---- 2. stage the first RING tiles at once, through descriptors over the
  // block's slots up to the capacity (slots past the newest position are
  // masked below); later tiles use descriptors over the visible slots only,
  // which read as zeros past them without touching memory.
  const uint32_t cap_range = static_cast<uint32_t>(stop - start) * D * 2;
  const bf16_t* kb = a.keys + kv_base + static_cast<long>(start) * D;
  const bf16_t* vb0 = a.values + kv_base + static_cast<long>(start) * D;
  unsigned char* wave_ring = ring + wave * kLdsWaveTile;
  const uint32_t wave_off = static_cast<uint32_t>(wave) * 16 * D * 2;  // this wave's 16 slots
  // K rows are staged rotated: chunk c of slot s sits at column (c + s) % 16
  // of the slot's 256-byte row, so the score operand's 16 slots (one column
  // each) fall in 16 different bank groups.
  uint32_t kvoff[4], vvoff[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int sl = 4 * u + (lane >> 4);
    kvoff[u] = static_cast<uint32_t>(sl * 256 + (((lane & 15) - sl) & 15) * 16);
    vvoff[u] = static_cast<uint32_t>(sl * 256 + (((lane & 15) - 2 * (sl & 7)) & 15) * 16);
  }
  {
    const __amdgpu_buffer_rsrc_t krs0 = buffer_rsrc(kb, cap_range);
    const __amdgpu_buffer_rsrc_t vrs0 = buffer_rsrc(vb0, cap_range);
#pragma unroll
    for (int t = 0; t < RING; ++t)
      stage_tile_mf(krs0, vrs0, wave_ring + t * kLdsTile, kvoff, vvoff,
                    t * kSplit * D * 2 + wave_off);
  }
  // Positions outside [0, cap) never match a slot (clamped to -1 / cap).
  int maxpos = -1, minpos = 1 << 30;
  if (MQ) {
    // Scalar loads of pos[min(t, Q - 1)] (in bounds, branch-free).
    int64_t pq[kMaxQ];
    load_pos8(a.pos, a.Q, pq);
#pragma unroll
    for (int t = 0; t < kMaxQ; ++t) {
      const int64_t v = pq[t];
      const int vc = v < 0 ? -1 : (v >= a.cap ? static_cast<int>(a.cap) : static_cast<int>(v));
      maxpos = vc > maxpos ? vc : maxpos;
      minpos = vc < minpos ? vc : minpos;
    }
  } else {
    const int64_t v = load_pos(a.pos, 0);
    minpos = maxpos = v < 0 ? -1 : (v >= a.cap ? static_cast<int>(a.cap) : static_cast<int>(v));
  }
  const int pos = minpos;  // one query: its position
  const int last = maxpos < a.cap ? maxpos : static_cast<int>(a.cap) - 1;
  const int end = stop < last + 1 ? stop : last + 1;  // slots [start, end) are visible to some row
  const int newest = FUSED && pos >= 0 && pos < a.cap ? pos : -1;
  const bool has_newest = newest >= start && newest < end;
  if (PRO == PRO_BY_POSITION) {
    const long ri = (newest >= 0 && newest < a.rope_rows) ? newest : 0;
    head16_load(hsrc, pick_gain(a.qg, a.kg, is_k), a.cos + ri * a.rope_st,
                a.sin + ri * a.rope_st, e, hq);
  }

  const uint32_t range = end > start ? static_cast<uint32_t>(end - start) * D * 2 : 0u;
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(kb, range);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(vb0, range);

  // ---- 3. query rows (and, fused, the newest k/v) into LDS
  if (FUSED) {
    const bool do_head = head_slot < a.G || (is_k && has_newest);
    uint2 oa, ob;
    head16_math(hq, is_k ? sgpr_f32(a.k_eps) : sgpr_f32(a.q_eps), oa, ob);
    if (do_head && !is_k) {
      qs[head_slot * (D / 2) + 2 * e] = oa.x;
      qs[head_slot * (D / 2) + 2 * e + 1] = oa.y;
      qs[head_slot * (D / 2) + 32 + 2 * e] = ob.x;
      qs[head_slot * (D / 2) + 32 + 2 * e + 1] = ob.y;
    } else if (do_head) {
      const long slot = kv_base + static_cast<long>(newest) * D;
      *reinterpret_cast<uint2*>(knew + 4 * e) = oa;
      *reinterpret_cast<uint2*>(knew + 64 + 4 * e) = ob;
      *reinterpret_cast<uint2*>(vnew + 4 * e) = va;
      *reinterpret_cast<uint2*>(vnew + 64 + 4 * e) = vb;
      *reinterpret_cast<uint2*>(a.keys + slot + 4 * e) = oa;
      *reinterpret_cast<uint2*>(a.keys + slot + 64 + 4 * e) = ob;
      *reinterpret_cast<uint2*>(a.values + slot + 4 * e) = va;
      *reinterpret_cast<uint2*>(a.values + slot + 64 + 4 * e) = vb;
    }
  } else {
    if (MQ && tid < rows) rowpos[tid] = rpv;
#pragma unroll
    for (int j = 0; j < kQL; ++j)
      if (tid + j * kBlock < rows * (D / 2)) qs[tid + j * kBlock] = qv[j];
  }
  lds_barrier();
  // ---- 4. tiles on the matrix cores. Per wave and tile (its 16 slots):
  //   S^T = K Q^T   v_mfma_f32_16x16x32_bf16 x 4: slots are the M index,
  //                 query rows (padded to 16) the N index, 32 dims per step;
  //   O^T += V^T P^T  v_mfma_f32_16x16x32_bf16 x 8: 16 dims per step, K = the
  //                 16 slots, each once with the hi and once with the lo half
  //                 of its weight. The scores' D layout (lane: row = slot
  //                 4 * quad + i, column = query row) is exactly the P^T
  //                 operand layout, so P never leaves the registers.
  // P enters the product as two bf16 operands, hi = bf16(P) and
  // lo = bf16(P - hi), so the weights keep about 16 bits (the VALU kernels
  // multiply fp32 weights; a bf16-only P drifts from them by up to 2^-9
  // relative per weight, enough to flip greedy near-ties between the
  // one-query and the verify paths). The denominator sums the fp32 weights.
  // Online softmax in base 2.
  const int col = lane & 15, quad = lane >> 4;
  // Per 16-row tile n: B operand of the scores (query row col + 16 n, 16-byte
  // chunk 4 * quad + j), the row's position, and its softmax state (the same
  // in all four quads).
  uint4 qb[NT][4];
  int rp[NT];
  f32x4_t acc_o[NT][8];
  float m_r[NT], l_r[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int row = col + 16 * n;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      qb[n][j] = row < rows ? *reinterpret_cast<const uint4*>(qs + row * (D / 2) + (4 * quad + j) * 4)
                            : make_uint4(0, 0, 0, 0);
    rp[n] = MQ ? (row < rows ? rowpos[row] : -1) : pos;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc_o[n][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    m_r[n] = -INFINITY;
    l_r[n] = 0.f;
  }
  const float scale2 = a.scale * 1.4426950408889634f;  // log2(e) / sqrt(D)
  const uint32_t wave_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)(wave_ring)));
  uint32_t kaddr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    kaddr[j] = wave_base + static_cast<uint32_t>(col * 256 + ((4 * quad + j + col) & 15) * 16);
  // V^T transpose reads: slot r = 4 quad + col / 4, dims 16 j + 4 (col % 4)
  // .. + 3, 8 bytes of chunk 2 j + (col % 4) / 2 at its rotated column.
  uint32_t vaddr[8];
  const int vr = 4 * quad + (col >> 2);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    vaddr[j] = wave_base + 4096 +
               static_cast<uint32_t>(vr * 256 + (((2 * j + ((col & 3) >> 1) + 2 * (vr & 7)) & 15) * 16) +
                                     (col & 1) * 8);

#pragma unroll 1
  for (int t = 0; t < nt; ++t) {
    const int q = t % RING;
    const uint32_t ro = static_cast<uint32_t>(q * kLdsTile);
    const int later = nt - 1 - t < RING - 1 ? nt - 1 - t : RING - 1;  // tiles staged after t
    uint4 kreg[4];
    uint2 vt[8];
    if (RING == 1 || later == 0) read_tile_mf<0>(kaddr, vaddr, ro, kreg, vt);
    else if (RING == 2 || later == 1) read_tile_mf<8>(kaddr, vaddr, ro, kreg, vt);
    else if (later == 2) read_tile_mf<16>(kaddr, vaddr, ro, kreg, vt);
    else read_tile_mf<24>(kaddr, vaddr, ro, kreg, vt);
    const int tbase = start + t * kSplit + wave * 16;  // this wave's first slot
    if (has_newest && newest >= tbase && newest < tbase + 16) {  // wave-uniform
      // The staged copy of the newest slot predates this step's append.
      const int sn = newest - tbase;
      if (col == sn) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          kreg[j] = *reinterpret_cast<const uint4*>(knew + (4 * quad + j) * 8);
      }
      const int kn = sn - 4 * quad;  // element of this lane's V^T operand, if in 0..3
      if (kn >= 0 && kn < 4) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t v = vnew[16 * j + col];
          if (kn == 0) vt[j].x = (vt[j].x & 0xffff0000u) | v;
          else if (kn == 1) vt[j].x = (vt[j].x & 0xffffu) | (v << 16);
          else if (kn == 2) vt[j].y = (vt[j].y & 0xffff0000u) | v;
          else vt[j].y = (vt[j].y & 0xffffu) | (v << 16);
        }
      }
    }
    const bool full = tbase + 16 <= end;  // wave-uniform: every slot visible to some row
    if (!full) {
      // Slots past the visible ones: V rows to zero (the cache may hold
      // anything there, NaN included; never NaN * 0), scores to -inf below.
      const int sb = tbase + 4 * quad;
      const uint32_t mx = (sb < end ? 0xffffu : 0u) | (sb + 1 < end ? 0xffff0000u : 0u);
      const uint32_t my = (sb + 2 < end ? 0xffffu : 0u) | (sb + 3 < end ? 0xffff0000u : 0u);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        vt[j].x &= mx;
        vt[j].y &= my;
      }
    }
    // Rows see slots up to their own position: masks are per lane, needed
    // unless every row sees the wave's 16 slots.
    const bool all_visible = tbase + 15 <= pos;  // wave-uniform (pos: the smallest position)
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      // Two accumulation chains of two steps each (shorter dependency chain).
      f32x4_t st0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, st1 = st0;
#pragma unroll
      for (int j = 0; j < 4; j += 2) {
        st0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kreg[j]),
                                                      __builtin_bit_cast(bf16x8_t, qb[n][j]), st0, 0, 0, 0);
        st1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kreg[j + 1]),
                                                      __builtin_bit_cast(bf16x8_t, qb[n][j + 1]), st1, 0, 0, 0);
      }
      const f32x4_t st = st0 + st1;
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[i] = st[i] * scale2;
        if (!all_visible) sc[i] = tbase + 4 * quad + i <= rp[n] ? sc[i] : -INFINITY;
      }
      const float tmax = quad_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
      // One query: visibility depends on the slot only, so a wave whose 16
      // slots are all hidden skips the tile (wave-uniform).
      if (!MQ && tmax == -INFINITY) continue;
      const float m_new = fmaxf(m_r[n], tmax);
      // A row with nothing visible yet keeps weight 0 (no inf - inf).
      const float ms = MQ && m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_r[n] - ms);  // 0 while m is -inf
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(sc[i] - ms);
      l_r[n] = fmaf(l_r[n], alpha, (p[0] + p[1]) + (p[2] + p[3]));
      m_r[n] = m_new;
      const uint2 pb = make_uint2(pack_bf2(p[0], p[1]), pack_bf2(p[2], p[3]));
      const uint2 pl = make_uint2(pack_bf2(p[0] - bf_lo(pb.x), p[1] - bf_hi(pb.x)),
                                  pack_bf2(p[2] - bf_lo(pb.y), p[3] - bf_hi(pb.y)));
      // One K = 32 step per 16 dims: this lane's k values 0-3 pair its four
      // V elements with hi, 4-7 the same V elements with lo.
      const uint4 phl = make_uint4(pb.x, pb.y, pl.x, pl.y);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc_o[n][j] *= alpha;
        acc_o[n][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, make_uint4(vt[j].x, vt[j].y, vt[j].x, vt[j].y)),
            __builtin_bit_cast(bf16x8_t, phl), acc_o[n][j], 0, 0, 0);
      }
    }
    const int tn = t + RING;
    if (tn < nt)  // wave-uniform
      stage_tile_mf(krs, vrs, wave_ring + q * kLdsTile, kvoff, vvoff,
                    tn * kSplit * D * 2 + wave_off);
  }
  // Every staging load has landed before the block's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- 5. the wave's state per query row: the denominator summed over the
  // four quads' slots; O^T is spread one (dim, row) pair per lane register.
  // With several queries the states reuse the ring: every wave has finished
  // reading it first.
  if (MQ) lds_barrier();
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int row = col + 16 * n;
    const float ln = quad_sum(l_r[n]);
    if (row < rows) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) wacc[wave][row][16 * j + 4 * quad + i] = acc_o[n][j][i];
      if (quad == 0) {
        wm[wave][row] = m_r[n];
        wl[wave][row] = ln;
      }
    }
  }
  lds_barrier();
  write_rows<ROWS, MQ>(a, b, kvh, s, rows, wave, lane, wm, wl, wacc);
  if (a.done) merge_tail(a, b, kvh, &last_split);
}

// ------------------------------------------------------------------ causal prefill

// Operand reads of the prefill kernel's staged tiles (LDS-direct data, read
// by inline asm: the compiler would wait for every load in flight before an
// ordinary LDS read of such a buffer), issued without their waits: issue, run
// other work, then a wait that names the registers as operands so no use of
// them moves above it. K: one 32-dim step for the four 16-slot M-tiles of a
// 64-slot tile; V^T: transpose reads as read_vt_tr.
template <int OFF>
__device__ __forceinline__ void issue_k_pf(uint32_t addr, u32x4 (&k)[4]) {
  asm volatile(
      "ds_read_b128 %0, %4 offset:%5\n\t"
      "ds_read_b128 %1, %4 offset:%6\n\t"
      "ds_read_b128 %2, %4 offset:%7\n\t"
      "ds_read_b128 %3, %4 offset:%8"
      : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3])
      : "v"(addr), "n"(OFF), "n"(OFF + 4096), "n"(OFF + 8192), "n"(OFF + 12288)
      : "memory");
}

typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

template <int OFF>
__device__ __forceinline__ void issue_vt_tr(const uint32_t (&va)[8], u32x2_t (&w)[8]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8 offset:%16\n\t"
      "ds_read_b64_tr_b16 %1, %9 offset:%16\n\t"
      "ds_read_b64_tr_b16 %2, %10 offset:%16\n\t"
      "ds_read_b64_tr_b16 %3, %11 offset:%16\n\t"
      "ds_read_b64_tr_b16 %4, %12 offset:%16\n\t"
      "ds_read_b64_tr_b16 %5, %13 offset:%16\n\t"
      "ds_read_b64_tr_b16 %6, %14 offset:%16\n\t"
      "ds_read_b64_tr_b16 %7, %15 offset:%16"
      : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]),
        "=&v"(w[6]), "=&v"(w[7])
      : "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]), "v"(va[4]), "v"(va[5]), "v"(va[6]),
        "v"(va[7]), "n"(OFF)
      : "memory");
}

__device__ __forceinline__ void wait_k16(u32x4 (&k)[4][4]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(k[0][0]), "+v"(k[0][1]), "+v"(k[0][2]), "+v"(k[0][3]), "+v"(k[1][0]),
                 "+v"(k[1][1]), "+v"(k[1][2]), "+v"(k[1][3]), "+v"(k[2][0]), "+v"(k[2][1]),
                 "+v"(k[2][2]), "+v"(k[2][3]), "+v"(k[3][0]), "+v"(k[3][1]), "+v"(k[3][2]),
                 "+v"(k[3][3])
               :
               : "memory");
}

__device__ __forceinline__ void wait_v32(u32x2_t (&w)[4][8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(w[0][0]), "+v"(w[0][1]), "+v"(w[0][2]), "+v"(w[0][3]), "+v"(w[0][4]),
                 "+v"(w[0][5]), "+v"(w[0][6]), "+v"(w[0][7]), "+v"(w[1][0]), "+v"(w[1][1]),
                 "+v"(w[1][2]), "+v"(w[1][3]), "+v"(w[1][4]), "+v"(w[1][5]), "+v"(w[1][6]),
                 "+v"(w[1][7]), "+v"(w[2][0]), "+v"(w[2][1]), "+v"(w[2][2]), "+v"(w[2][3]),
                 "+v"(w[2][4]), "+v"(w[2][5]), "+v"(w[2][6]), "+v"(w[2][7]), "+v"(w[3][0]),
                 "+v"(w[3][1]), "+v"(w[3][2]), "+v"(w[3][3]), "+v"(w[3][4]), "+v"(w[3][5]),
                 "+v"(w[3][6]), "+v"(w[3][7])
               :
               : "memory");
}

constexpr int kPfQ = 64;                          // queries per prefill block
constexpr int kPfTileBytes = 2 * kSplit * D * 2;  // K then V of one staged 64-slot tile

// Causal attention over many queries per sequence (a prompt's prefill): one
// launch per layer, no split, no merge. Block = (64-query tile, query head h,
// batch b), four waves of 16 queries, or HPB = 2 query heads of one kv head
// (eight waves: the second head's waves 4-7) sharing each staged tile. The
// block stages each 64-slot K/V tile of kv head h / G once for its waves
// (four waves a quarter each, LDS-direct, K and V, or with eight waves K by
// waves 0-3 and V by 4-7; the next tile in flight), then every wave
// multiplies all 64 slots against
// its queries on the matrix cores as the decode kernel does per 16-slot
// group: S^T = K Q^T (slots as M, queries as N: four 16-slot M-tiles x four
// 32-dim steps), an online softmax per query in base 2, O^T += V^T P^T with P
// as hi/lo bf16 halves (weights keep ~16 bits; the denominator sums the fp32
// weights). A query sees slots <= its own position (masked per lane); the
// block reads tiles up to its largest position, the latest query tiles
// first. K rows are staged rotated (chunk c of slot s at column (c + s) % 16)
// and V rows by two chunks per slot (c + 2 (s % 8)); V^T operands come from
// transpose reads, one per 16 dims and 16 slots.
template <int HPB>
__global__ __launch_bounds__(HPB * kBlock) void attention_prefill(AttnArgs a) {
  preload_args<false>(a);
  constexpr int NW = HPB * kBlock / kWave;  // waves: HPB heads x four 16-query groups
  extern __shared__ __align__(16) unsigned char ring[];  // two staged tiles
  __shared__ int wave_pos[NW];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qw = wave & 3;  // this wave's 16 queries of the block's 64
  const int col = lane & 15, quad = lane >> 4;
  const int ntq = (a.Q + kPfQ - 1) / kPfQ;
  const int qt = ntq - 1 - static_cast<int>(blockIdx.x);  // latest queries first
  const int h = blockIdx.y * HPB + (wave >> 2), b = blockIdx.z, kvh = h / a.G;
  const int t = qt * kPfQ + qw * 16 + col;  // this lane's query
  const int tq = t < a.Q ? t : a.Q - 1;
  // Visible slots [0, pos]; a position past the cache sees every slot, a
  // negative one (and a padding query) none.
  const int64_t pv = a.pos[tq];
  const int pos = t >= a.Q || pv < 0 ? -1 : (pv >= a.cap ? static_cast<int>(a.cap) - 1 : static_cast<int>(pv));
  // B operand of S^T = K Q^T: dims 32 ks + 8 quad .. + 7 of this lane's query.
  const bf16_t* qrow = a.q + b * a.q_sb + h * a.q_sh + tq * a.q_st + 8 * quad;
  u32x4 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qf[ks] = *reinterpret_cast<const u32x4*>(qrow + 32 * ks);
  const float wmax = wave_max(static_cast<float>(pos));     // exact: |pos| < 2^24
  const float wmin = -wave_max(-static_cast<float>(pos));
  if (lane == 0) wave_pos[wave] = static_cast<int>(wmax);
  lds_barrier();
  int bmax = wave_pos[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) bmax = wave_pos[w] > bmax ? wave_pos[w] : bmax;
  const int nkt = bmax < 0 ? 0 : bmax / kSplit + 1;  // tiles [0, nkt) hold every visible slot
  const int wave_last = static_cast<int>(wmax), wave_first = static_cast<int>(wmin);

  // Staging: wave w loads slots 16 w .. 16 w + 15 of each tile (K, then V),
  // through descriptors over the slots up to the block's largest position:
  // later slots (the cache may hold anything there, NaN included) read as
  // zeros, so masked weights never multiply NaN.
  const long kv_base = (static_cast<long>(b) * a.Hkv + kvh) * a.cap * D;
  const uint32_t range = static_cast<uint32_t>(bmax + 1) * D * 2;  // block-uniform (from LDS)
  const __amdgpu_buffer_rsrc_t krs = uniform_rsrc(a.keys + kv_base, range);
  const __amdgpu_buffer_rsrc_t vrs = uniform_rsrc(a.values + kv_base, range);
  uint32_t kvoff[4], vvoff[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int sl = 4 * u + (lane >> 4);
    kvoff[u] = static_cast<uint32_t>(sl * 256 + (((lane & 15) - sl) & 15) * 16);
    vvoff[u] = static_cast<uint32_t>(sl * 256 + (((lane & 15) - 2 * (sl & 7)) & 15) * 16);
  }
  // With two heads per block (eight waves), waves 0-3 stage the K rows and
  // waves 4-7 the V rows of their 16 slots.
  auto stage = [&](int kt) {
    unsigned char* tb = ring + (kt & 1) * kPfTileBytes + qw * 4096;
    const uint32_t off = static_cast<uint32_t>(kt * kSplit + qw * 16) * D * 2;
    if (HPB == 1 || wave < 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_t*)(tb + u * 1024), 16, kvoff[u], off, 0, 0);
    }
    if (HPB == 1 || wave >= 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_t*)(tb + kSplit * D * 2 + u * 1024), 16,
                                                 vvoff[u], off, 0, 0);
    }
  };
  if (nkt > 0) stage(0);

  // Operand addresses in tile buffer 0 (buffer 1 is kPfTileBytes further):
  // K slot 16 mt + col, chunk 4 ks + quad, rotated by the slot; for the V^T
  // transpose reads, slot 16 mt + r (r = 4 quad + col / 4), dims
  // 16 j + 4 (col % 4) .. + 3: 8 bytes of chunk 2 j + (col % 4) / 2, whose
  // position the slot rotates by 2 (r % 8).
  const uint32_t ring_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)ring));
  uint32_t kaddr[4], vaddr[8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    kaddr[ks] = ring_base + static_cast<uint32_t>(col * 256 + (((4 * ks + quad + col) & 15) * 16));
  const int vr = 4 * quad + (col >> 2);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    vaddr[j] = ring_base + kSplit * D * 2 +
               static_cast<uint32_t>(vr * 256 + (((2 * j + ((col & 3) >> 1) + 2 * (vr & 7)) & 15) * 16) +
                                     (col & 1) * 8);

  const float scale2 = a.scale * 1.4426950408889634f;  // log2(e) / sqrt(D)
  f32x4_t acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  for (int kt = 0; kt < nkt; ++kt) {
    // This wave's part of tile kt has landed; after the barrier everyone's
    // has, and every wave has finished tile kt - 1, whose buffer tile kt + 1
    // now takes (in flight during this tile's work).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    if (kt + 1 < nkt) stage(kt + 1);
    const int s0 = kt * kSplit;
    if (s0 <= wave_last) {  // wave-uniform: some slot of the tile is visible to the wave
      const uint32_t tb = static_cast<uint32_t>((kt & 1) * kPfTileBytes);
      // All sixteen K fragments at once, then the scores.
      u32x4 kf[4][4];
      issue_k_pf<0>(kaddr[0] + tb, kf[0]);
      issue_k_pf<0>(kaddr[1] + tb, kf[1]);
      issue_k_pf<0>(kaddr[2] + tb, kf[2]);
      issue_k_pf<0>(kaddr[3] + tb, kf[3]);
      wait_k16(kf);
      f32x4_t st[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) st[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          st[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf[ks][mt]),
                                                           __builtin_bit_cast(bf16x8_t, qf[ks]),
                                                           st[mt], 0, 0, 0);
      // The V^T operands of the whole tile in flight during the softmax.
      uint32_t va[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) va[j] = vaddr[j] + tb;
      u32x2_t vw[4][8];
      issue_vt_tr<0>(va, vw[0]);
      issue_vt_tr<4096>(va, vw[1]);
      issue_vt_tr<8192>(va, vw[2]);
      issue_vt_tr<12288>(va, vw[3]);
      // Scores in base 2; slots past the query's position masked unless the
      // whole tile is visible to every query of the wave (a wave-uniform
      // branch: the mask is computed only on the tiles that need it).
      float sc[4][4];
      float tmax = -INFINITY;
      if (__builtin_expect(s0 + kSplit - 1 <= wave_first, 1)) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            sc[mt][i] = st[mt][i] * scale2;
            tmax = fmaxf(tmax, sc[mt][i]);
          }
      } else {
        // Slot s0 + 16 mt + 4 quad + i is visible iff 16 mt + i <= lim.
        const int lim = pos - s0 - 4 * quad;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float v = st[mt][i] * scale2;
            sc[mt][i] = 16 * mt + i <= lim ? v : -INFINITY;
            tmax = fmaxf(tmax, sc[mt][i]);
          }
      }
      tmax = quad_max(tmax);
      const float m_new = fmaxf(m, tmax);
      // A query with nothing visible yet keeps weight 0 (no inf - inf).
      const float ms = m_new == -INFINITY ? 0.f : m_new;
      // Where no lane's max moved, alpha is exactly 1 (or 0 on an all-zero
      // state) and the products are identities: the wave skips them.
      if (!__all(m_new == m)) {
        const float alpha = __builtin_amdgcn_exp2f(m - ms);  // 0 while m is -inf
        l *= alpha;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] *= alpha;
      }
      m = m_new;
      uint4 phl[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(sc[mt][i] - ms);
        l += (p[0] + p[1]) + (p[2] + p[3]);
        const uint2 pb = make_uint2(pack_bf2(p[0], p[1]), pack_bf2(p[2], p[3]));
        const uint2 pl = make_uint2(pack_bf2(p[0] - bf_lo(pb.x), p[1] - bf_hi(pb.x)),
                                    pack_bf2(p[2] - bf_lo(pb.y), p[3] - bf_hi(pb.y)));
        phl[mt] = make_uint4(pb.x, pb.y, pl.x, pl.y);
      }
      wait_v32(vw);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, make_uint4(vw[mt][j].x, vw[mt][j].y, vw[mt][j].x, vw[mt][j].y)),
              __builtin_bit_cast(bf16x8_t, phl[mt]), acc[j], 0, 0, 0);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // O[query][dim 16 j + 4 quad + i] = acc[j][i] / (the four quads' sums).
  const float ln = quad_sum(l);
  if (t < a.Q) {
    bf16_t* dst = a.out + b * a.o_sb + h * a.o_sh + static_cast<long>(t) * a.o_st + 4 * quad;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<uint2*>(dst + 16 * j) =
          make_uint2(pack_bf2(acc[j][0] / ln, acc[j][1] / ln), pack_bf2(acc[j][2] / ln, acc[j][3] / ln));
  }
}

// Merge of the split partials, one block per output row (b, h, t):
//   out = sum_s exp(m_s - M) acc_s / sum_s exp(m_s - M) l_s,  M = max_s m_s.
// Each wave folds every fourth split with an online max (one pass over the
// partials, loads unrolled), then the four wave states combine in LDS. It runs
// as its own launch, so the partials are visible without any in-kernel fence.
struct MergeArgs {
  const float* part;
  const float* ml;
  bf16_t* out;
  long o_sb, o_sh, o_st;
  int splits, Hq, Q;
};

__global__ __launch_bounds__(kBlock) void attention_merge(MergeArgs a) {
  asm volatile("" ::"s"(a.part), "s"(a.ml), "s"(a.out), "s"(a.o_sb), "s"(a.o_sh), "s"(a.o_st),
               "s"(a.splits), "s"(a.Hq), "s"(a.Q));
  const float* __restrict__ part = a.part;
  const float* __restrict__ ml = a.ml;
  const int splits = a.splits;
  __shared__ float wm[4], wl[4];
  __shared__ float2 wacc[4][D / 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long orow = blockIdx.x;
  const float* mlr = ml + orow * splits * 2;
  const float* pr = part + orow * splits * D;
  float m = -INFINITY, l = 0.f;
  float2 acc = make_float2(0.f, 0.f);
  for (int s0 = wave; s0 < splits; s0 += 4 * kMergeUnroll) {
    float2 pv[kMergeUnroll];
    float mv[kMergeUnroll], lv[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const int sp = s0 + 4 * u;
      const int sc = sp < splits ? sp : s0;
      pv[u] = *reinterpret_cast<const float2*>(pr + static_cast<long>(sc) * D + 2 * lane);
      mv[u] = sp < splits ? mlr[2 * sc] : -INFINITY;
      lv[u] = mlr[2 * sc + 1];
    }
    float mb = m;
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) mb = fmaxf(mb, mv[u]);
    if (mb != -INFINITY) {
      const float scale = m == -INFINITY ? 0.f : expf(m - mb);
      acc.x *= scale;
      acc.y *= scale;
      l *= scale;
#pragma unroll
      for (int u = 0; u < kMergeUnroll; ++u) {
        const float w = mv[u] == -INFINITY ? 0.f : expf(mv[u] - mb);
        acc.x = fmaf(w, pv[u].x, acc.x);
        acc.y = fmaf(w, pv[u].y, acc.y);
        l = fmaf(w, lv[u], l);
      }
      m = mb;
    }
  }
  wacc[wave][lane] = acc;
  if (lane == 0) {
    wm[wave] = m;
    wl[wave] = l;
  }
  __syncthreads();
  if (wave == 0) {
    const float M = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    float sx = 0.f, sy = 0.f, lt = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = wm[w] == -INFINITY ? 0.f : expf(wm[w] - M);
      sx = fmaf(f, wacc[w][lane].x, sx);
      sy = fmaf(f, wacc[w][lane].y, sy);
      lt = fmaf(f, wl[w], lt);
    }
    const long t = orow % a.Q, bh = orow / a.Q, h = bh % a.Hq, b = bh / a.Hq;
    bf16_t* dst = a.out + b * a.o_sb + h * a.o_sh + t * a.o_st;
    dst[2 * lane] = static_cast<bf16_t>(f2bf(sx / lt));
    dst[2 * lane + 1] = static_cast<bf16_t>(f2bf(sy / lt));
  }
}

// The XCD (hardware register XCC_ID) each block of a one-dimensional grid
// runs on: the check of the round-robin dispatch that the XCD-affine
// attention grid relies on.
__global__ __launch_bounds__(kWave) void xcc_ids_kernel(int32_t* out, long n) {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  if (threadIdx.x == 0 && blockIdx.x < n) out[blockIdx.x] = static_cast<int32_t>(v & 0xfu);
}

}  // namespace htn

using namespace htn;

namespace {

// (split, kv head, batch), or the one-dimensional XCD-affine grid: eight
// block columns, each holding the splits of every eighth pair.
dim3 split_grid(const AttnArgs& a) {
  if (!a.done) return dim3(a.splits, a.Hkv, a.B);
  const long pairs = static_cast<long>(a.B) * a.Hkv;
  return dim3(static_cast<unsigned>(8 * ((pairs + 7) / 8) * a.splits +
                                    (a.pf ? 8 * a.pf_per_class : 0) + (a.ow ? 8 * a.o_blocks : 0)));
}

template <int ROWS, int TILES>
void launch_partial_t(bool fused, const AttnArgs& a, hipStream_t st) {
  const dim3 grid = split_grid(a);
  if (!fused)
    hipLaunchKernelGGL((attention_partial<ROWS, PRO_NONE, TILES>), grid, dim3(kBlock), 0, st, a);
  else if (a.rope_by_pos)
    hipLaunchKernelGGL((attention_partial<ROWS, PRO_BY_POSITION, TILES>), grid, dim3(kBlock), 0, st, a);
  else
    hipLaunchKernelGGL((attention_partial<ROWS, PRO_ROW, TILES>), grid, dim3(kBlock), 0, st, a);
}

template <int ROWS>
void launch_stream(bool fused, const AttnArgs& a, hipStream_t st) {
  const dim3 grid(a.splits, a.Hkv, a.B);
  if (!fused)
    hipLaunchKernelGGL((attention_stream<ROWS, PRO_NONE>), grid, dim3(kBlock), 0, st, a);
  else if (a.rope_by_pos)
    hipLaunchKernelGGL((attention_stream<ROWS, PRO_BY_POSITION>), grid, dim3(kBlock), 0, st, a);
  else
    hipLaunchKernelGGL((attention_stream<ROWS, PRO_ROW>), grid, dim3(kBlock), 0, st, a);
}

template <int ROWS, int PRO, int RING, bool OUT>
void launch_lds_o(const AttnArgs& a, hipStream_t st) {
  const size_t lds = static_cast<size_t>(RING) * kLdsTile;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&attention_lds<ROWS, PRO, RING, OUT>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  (void)attr;  // a refused size surfaces as a launch error
  hipLaunchKernelGGL((attention_lds<ROWS, PRO, RING, OUT>), split_grid(a), dim3(kBlock), lds, st, a);
}

// The fused output projection only runs with the fused prologue.
template <int ROWS, int PRO, int RING>
void launch_lds_t(const AttnArgs& a, hipStream_t st) {
  if constexpr (PRO != PRO_NONE) {
    if (a.ow) return launch_lds_o<ROWS, PRO, RING, true>(a, st);
  }
  launch_lds_o<ROWS, PRO, RING, false>(a, st);
}

template <int ROWS, int PRO, int RING, bool OUT>
void launch_mfma_o(const AttnArgs& a, hipStream_t st) {
  // The ring, which with several queries (ROWS > 8) the waves' partial states
  // reuse after the last tile.
  constexpr size_t kStates = ROWS > 8 ? static_cast<size_t>(kBlock / kWave) * ROWS * D * 4 : 0;
  const size_t lds = static_cast<size_t>(RING) * kLdsTile > kStates ? static_cast<size_t>(RING) * kLdsTile
                                                                     : kStates;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&attention_mfma<ROWS, PRO, RING, OUT>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  (void)attr;  // a refused size surfaces as a launch error
  hipLaunchKernelGGL((attention_mfma<ROWS, PRO, RING, OUT>), split_grid(a), dim3(kBlock), lds, st, a);
}

template <int ROWS, int PRO, int RING>
void launch_mfma_t(const AttnArgs& a, hipStream_t st) {
  if constexpr (PRO != PRO_NONE) {
    if (a.ow) return launch_mfma_o<ROWS, PRO, RING, true>(a, st);
  }
  launch_mfma_o<ROWS, PRO, RING, false>(a, st);
}

// Several queries per sequence (verify rows): 16 or 32 query rows per kv head.
void launch_mfma_rows(const AttnArgs& a, hipStream_t st) {
  const int rows = a.G * a.Q;
  if (rows <= 16) {
    if (a.ring == 1) launch_mfma_t<16, PRO_NONE, 1>(a, st);
    else launch_mfma_t<16, PRO_NONE, 2>(a, st);
  } else {
    if (a.ring == 1) launch_mfma_t<32, PRO_NONE, 1>(a, st);
    else launch_mfma_t<32, PRO_NONE, 2>(a, st);
  }
}

template <int ROWS, int PRO>
void launch_lds_p(const AttnArgs& a, hipStream_t st) {
  if (a.mfma) {
    if (a.ring == 1) launch_mfma_t<ROWS, PRO, 1>(a, st);
    else if (a.ring == 2) launch_mfma_t<ROWS, PRO, 2>(a, st);
    else launch_mfma_t<ROWS, PRO, 4>(a, st);
    return;
  }
  if (a.ring == 1) launch_lds_t<ROWS, PRO, 1>(a, st);
  else if (a.ring == 2) launch_lds_t<ROWS, PRO, 2>(a, st);
  else launch_lds_t<ROWS, PRO, 4>(a, st);
}

template <int ROWS>
void launch_partial(bool fused, const AttnArgs& a, hipStream_t st) {
  if constexpr (ROWS <= 8) {  // the LDS-staged kernel when the plan chose it
    if (a.ring) {
      if (!fused) return launch_lds_p<ROWS, PRO_NONE>(a, st);
      if (a.rope_by_pos) return launch_lds_p<ROWS, PRO_BY_POSITION>(a, st);
      return launch_lds_p<ROWS, PRO_ROW>(a, st);
    }
  }
  if constexpr (ROWS <= 4) {  // the streaming kernel when the plan chose it
    if (a.stream) return launch_stream<ROWS>(fused, a, st);
  }
  if (a.split > kSplit) launch_partial_t<ROWS, 2>(fused, a, st);
  else launch_partial_t<ROWS, 1>(fused, a, st);
}

// Per device: 0 unknown, 1 in-kernel merge on, 2 off.
std::atomic<int> merge_state[64];

// Launches a grid of kProbeBlocks blocks that each record their XCD and
// checks that block i ran on the XCD of block i mod 8, the dispatch the
// in-kernel merge relies on. Allocates and synchronises, so it runs only
// outside stream capture, once per device.
bool round_robin_dispatch(int dev) {
  constexpr long kProbeBlocks = 2048;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess ||
      !(n == 1 || n == 2 || n == 4 || n == 8))
    return false;
  int32_t* ids = nullptr;
  hipStream_t s = nullptr;
  std::vector<int32_t> host(kProbeBlocks, -1);
  bool ok = hipMalloc(&ids, kProbeBlocks * sizeof(int32_t)) == hipSuccess &&
            hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess;
  if (ok) {
    hipLaunchKernelGGL(xcc_ids_kernel, dim3(kProbeBlocks), dim3(kWave), 0, s, ids, kProbeBlocks);
    ok = hipGetLastError() == hipSuccess &&
         hipMemcpyAsync(host.data(), ids, kProbeBlocks * sizeof(int32_t), hipMemcpyDeviceToHost,
                        s) == hipSuccess &&
         hipStreamSynchronize(s) == hipSuccess;
  }
  if (s) (void)hipStreamDestroy(s);
  if (ids) (void)hipFree(ids);
  if (!ok) return false;
  for (long i = 0; i < kProbeBlocks; ++i)
    if (host[i] < 0 || host[i] != host[i % 8]) return false;
  return true;
}

// The in-kernel merge needs every block with equal index mod 8 on one XCD.
// The first call on a device outside stream capture launches the dispatch
// probe and keeps its answer; until then (a first call under capture) the
// separate merge launch runs, which is correct under any dispatch. Setting
// HTN_ATTENTION_MERGE_LAUNCH=1, or htn_attention_disable_in_kernel_merge(),
// keeps the merge launch.
bool xcd_affine_merge(hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  int state = merge_state[dev].load();
  if (state == 0) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &capture) != hipSuccess ||
        capture != hipStreamCaptureStatusNone)
      return false;
    const char* env = getenv("HTN_ATTENTION_MERGE_LAUNCH");
    const bool ok = !(env && env[0] == '1') && round_robin_dispatch(dev);
    int expected = 0;
    merge_state[dev].compare_exchange_strong(expected, ok ? 1 : 2);
    state = merge_state[dev].load();
  }
  return state == 1;
}

// The projection that reads this attention's output, for the prefetch blocks.
struct NextWeights {
  const void* w;
  long n, k;
  int format;
};

// The output projection fused into the attention launch (one sequence): its
// weights (n rows of k = Hq D weights, format 0 bf16 or 8-bit) and the fp32
// partial rows [Hkv, n] the output blocks write.
struct FusedOutput {
  const void* w;
  long n, k;
  int format;
  unsigned long long* acc;
  const float* scale;
  const bf16_t* res;
  bf16_t* out;
};

// Prefetch blocks per XCD, and the bytes they read into each XCD's 4 MB L2
// (measured on 0.6B and 8B decode steps: 8 blocks beat 2, 4, 16 and 32 -- few
// blocks outlast the attention, many crowd its loads -- and 3 MB per XCD beat
// all of the 8B's 4 MB, 2 MB and 1 MB). With the staging ring every block
// holds at least 32 KB of LDS, so they run on CUs the attention leaves free.
constexpr int kPrefetchPerXcd = 8;
constexpr long kPrefetchXcdBytes = 3L << 20;
// Long contexts (six tiles per split): the attention outlasts the prefetch by
// far and its 176 blocks crowd the CUs, so half as many prefetch blocks (8B
// int8 / fp8 at context 8192: 2.223 -> 2.186 and 2.133 -> 2.096 ms per step;
// two per XCD outlast the attention, 2.44 ms).
constexpr int kPrefetchPerXcdLong = 4;

// Many queries per sequence (a prefill): the causal kernel, one launch, no
// scratch. Needs 16-byte query fragments and 8-byte output stores.
int run_prefill_attention(AttnArgs& a, hipStream_t st) {
  if (a.B <= 0 || a.cap <= 0 || a.Q > (1 << 30) || a.Hq > 65535 || a.B > 65535)
    return HTN_EUNSUPPORTED;
  if (a.cap > (1L << 31) / (D * 2) - 2 * kSplit) return HTN_EUNSUPPORTED;  // 32-bit byte offsets
  if ((reinterpret_cast<uintptr_t>(a.q) & 15u) || ((a.q_sb | a.q_sh | a.q_st) & 7) ||
      (reinterpret_cast<uintptr_t>(a.out) & 7u) || ((a.o_sb | a.o_sh | a.o_st) & 3))
    return HTN_EUNSUPPORTED;
  a.scale = 1.0f / sqrtf(static_cast<float>(D));
  const size_t lds = 2 * static_cast<size_t>(kPfTileBytes);
  static const hipError_t attr1 = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&attention_prefill<1>), hipFuncAttributeMaxDynamicSharedMemorySize,
      static_cast<int>(lds));
  static const hipError_t attr2 = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&attention_prefill<2>), hipFuncAttributeMaxDynamicSharedMemorySize,
      static_cast<int>(lds));
  (void)attr1;  // a refused size surfaces as a launch error
  (void)attr2;
  // Two query heads of one kv head per block share each staged tile while
  // the grid keeps two blocks per CU (8B, 2048 queries: 151 -> 146 us; at
  // 512 queries the halved grid measured slower, 18.6 -> 23.0 us).
  const long ntq = (a.Q + kPfQ - 1) / kPfQ;
  const int hpb =
      a.G % 2 == 0 && ntq * (a.Hq / 2) * a.B >= 2L * device_cus() ? 2 : 1;
  const dim3 grid(static_cast<unsigned>(ntq), static_cast<unsigned>(a.Hq / hpb),
                  static_cast<unsigned>(a.B));
  if (hpb == 2)
    hipLaunchKernelGGL(attention_prefill<2>, grid, dim3(2 * kBlock), lds, st, a);
  else
    hipLaunchKernelGGL(attention_prefill<1>, grid, dim3(kBlock), lds, st, a);
  return launch_status();
}

int run_attention(bool fused, AttnArgs& a, void* scratch, hipStream_t st,
                  const NextWeights* next = nullptr, const FusedOutput* fo = nullptr) {
  const int rows = a.G * a.Q;
  if (rows <= 0 || rows > kMaxRows || a.Q > kMaxQ || a.B <= 0 || a.Hkv <= 0 || a.cap <= 0)
    return HTN_EUNSUPPORTED;
  // One (batch, kv head) cache row is addressed with 32-bit byte offsets.
  if (a.cap > (1L << 31) / (D * 2) - 2 * kSplit) return HTN_EUNSUPPORTED;
  if (fused && a.G + 1 > 16) return HTN_EUNSUPPORTED;  // 16 head slots in the fused prologue
  // One query per sequence (decode): the LDS-staged kernel. One 64-slot
  // tile per block while the blocks fit two per CU; past that, just enough
  // tiles per block to keep the grid within one block per CU (all blocks
  // resident at once; a second residency round doubles the time), with two
  // or four tiles staged ahead.
  // Several queries (verify rows): one 64-slot tile per block (more, smaller
  // splits were measured slower: the merge grows); two tiles once one per
  // block would need more blocks than fit on the GPU at once (about four per
  // CU). Long contexts (rows <= 4 per kv head, at least four tiles per block
  // at about one block per CU): the streaming kernel over an even number of
  // tiles, ranges balanced.
  const long tiles = (a.cap + kSplit - 1) / kSplit;
  const long heads = static_cast<long>(a.Hkv) * a.B;
  const long cus = device_cus();
  const long per_head = (cus + heads - 1) / heads;
  long split = kSplit;
  a.stream = 0;
  a.ring = 0;
  a.mfma = 0;
  if (a.Q == 1 && rows <= 8 && heads <= 8 && tiles <= 144) {
    // Up to 8 (batch, kv head) pairs and 9K slots (measured, 2 and 4 query
    // rows per kv head, 512 to 8192 slots): one tile per block up to 24
    // tiles, then two, then three up to 80 tiles (fewer splits leave the
    // in-kernel merge less to read), then six: past ~80 tiles three-tile
    // splits outnumber the CUs and the blocks sharing a CU finish last,
    // while six keep one block per CU (8B at 6144 and 8192 slots: about
    // 1.3 us less per layer; a ring of four tiles, one 128 KB block per CU,
    // was slower). Four or more query rows per kv head score and weigh on
    // the matrix cores; two rows are faster on the vector unit.
    const long nt = tiles <= 24 ? 1 : (tiles <= 40 ? 2 : (tiles <= 80 ? 3 : 6));
    a.ring = nt == 1 ? 1 : 2;
    a.mfma = rows >= 3;
    split = nt * kSplit;
  } else if (!fused && a.Q > 1 && rows <= 32 && heads <= 8 && tiles <= 144) {
    // Several queries (verify rows): the matrix-core kernel with per-row
    // positions, 16 or 32 rows per block, the same split plan.
    const long nt = tiles <= 24 ? 1 : (tiles <= 40 ? 2 : 3);
    a.ring = nt == 1 ? 1 : 2;
    a.mfma = 1;
    split = nt * kSplit;
  } else if (a.Q == 1 && rows <= 8 &&
             (heads * tiles <= cus || heads * tiles > 2 * cus || rows >= 3)) {
    // LDS per block: 32 KB per staged tile plus up to 19 KB (8 rows) of
    // state; two-tile rings fit two blocks per CU for rows <= 4. Between one
    // and two single-tile blocks per CU the register kernel below was
    // measured faster for two rows per kv head (8B shape, 2K context). Three
    // or more query rows per kv head score and weigh on the matrix cores here
    // (8B, 16 sequences at context 512: 4.39 -> 4.28 ms per step, one tile
    // more or fewer per block measured slower, 4.31 / 4.33 ms; 4 sequences,
    // between one and two blocks per CU: 3.55 -> 3.52 ms).
    const long per_cu = rows <= 4 ? 2 : 1;
    long nt = 1;
    if (heads * tiles > 2 * cus) nt = (heads * tiles + per_cu * cus - 1) / (per_cu * cus);
    a.ring = nt == 1 ? 1 : (per_cu == 2 || nt < 4 ? 2 : 4);
    a.mfma = rows >= 3;
    split = nt * kSplit;
  } else if (rows <= 4 && tiles >= 4 * per_head) {
    const long t = 2 * (tiles / (2 * per_head));  // even tile count
    const long nsplit = (a.cap + t * kSplit - 1) / (t * kSplit);
    split = (a.cap + nsplit - 1) / nsplit;  // <= t tiles, balanced
    a.stream = 1;
  } else if (rows <= 8 && tiles * heads > 4L * cus) {
    split = 2 * kSplit;
  }
  a.split = static_cast<int>(split);
  a.splits = static_cast<int>((a.cap + a.split - 1) / a.split);
  if (a.splits > 1 && !scratch) return HTN_EINVAL;
  // Scratch: the arrival counters, then the partials and their (max, sum).
  const long nrow = static_cast<long>(a.B) * a.Hq * a.Q * a.splits;
  unsigned char* sbase = static_cast<unsigned char*>(scratch);
  a.part = sbase ? reinterpret_cast<float*>(sbase + kCounterBytes) : nullptr;
  a.ml = a.part ? a.part + nrow * D : nullptr;
  a.done = nullptr;
  // The in-kernel merge stores each lane's two output dims as one 32-bit word.
  const bool out_pairs = !(reinterpret_cast<uintptr_t>(a.out) & 3u) && !((a.o_sb | a.o_sh | a.o_st) & 1);
  // One block merges a pair's rows, each row's loads all in flight: worth it
  // up to four rows (one per wave) of at most 48 splits. More rows or splits
  // go to the merge launch, which spreads the rows over the GPU.
  if (a.splits > 1 && a.splits <= 48 && rows <= 4 && !a.stream && heads <= kMaxCounterPairs &&
      out_pairs && xcd_affine_merge(st))
    a.done = reinterpret_cast<unsigned*>(sbase);
  a.scale = 1.0f / sqrtf(static_cast<float>(D));
  // The output projection in the same launch: one sequence on the
  // XCD-affine grid of the staged kernels (each kv head's splits on one XCD),
  // merged by the output blocks from at most kOMaxSplits partials, with the
  // pair's span of each weight row a whole number (1, 2 or 4) of 256-byte
  // pieces and 32-bit byte offsets over the weights.
  a.ow = nullptr;
  a.oacc = nullptr;
  if (fo && fo->w && fo->acc && a.done && a.ring > 0 && !a.stream && a.B == 1 && a.Q == 1 &&
      a.Hkv <= 8 && a.splits <= kOMaxSplits && fo->k == static_cast<long>(a.Hq) * D) {
    const long kb = fo->format == 0 ? 2 : 1;
    const long span = static_cast<long>(a.G) * D * kb;
    const long lpr = span / 256;
    if (span % 256 == 0 && (lpr == 1 || lpr == 2 || lpr == 4) && fo->n > 0 &&
        fo->n <= kOMaxRows && fo->n * fo->k * kb < (1L << 31) &&
        fo->n * fo->k * kb >= kFuseMinBytes) {
      a.ow = static_cast<const unsigned char*>(fo->w);
      a.oacc = fo->acc;
      a.o_fmt = fo->format;
      a.o_n = static_cast<int>(fo->n);
      a.o_lpr = static_cast<int>(lpr);
      a.o_blocks = static_cast<int>((fo->n + kORowsPerBlock - 1) / kORowsPerBlock);
      a.attn_blocks = static_cast<int>(8 * a.splits);  // one pair per XCD column
      a.o_scale = fo->format != 0 ? fo->scale : nullptr;
      a.res_o = fo->res;
      a.out_o = fo->out;
    }
  }
  // Prefetch of the next projection's weights: only with the XCD-affine grid
  // of the LDS-staged kernels (one dimension, eight block columns) and a
  // GEMV grid of whole columns, so span u and its GEMV block share an XCD.
  a.pf = nullptr;
  long gemv_blocks = 0;
  int gemv_rows = 0;
  if (next && next->w && !a.ow && a.done && a.ring > 0 && !a.stream &&
      gemv_plain_layout(next->n, next->k, next->format, &gemv_blocks, &gemv_rows) &&
      gemv_blocks % 8 == 0) {
    const long row_bytes = next->k * (next->format == 0 ? 2 : 1);
    a.pf = static_cast<const unsigned char*>(next->w);
    a.pf_unit_bytes = static_cast<int>(gemv_rows * row_bytes);
    const long units = next->n / gemv_rows;  // whole spans only
    const long cap_units = 8 * kPrefetchXcdBytes / a.pf_unit_bytes;
    a.pf_units = units < cap_units ? units : cap_units;
    a.pf_per_class = a.split >= 6 * kSplit ? kPrefetchPerXcdLong : kPrefetchPerXcd;
    const long pairs = static_cast<long>(a.B) * a.Hkv;
    a.attn_blocks = static_cast<int>(8 * ((pairs + 7) / 8) * a.splits);
  }
  if (a.mfma && a.Q > 1) launch_mfma_rows(a, st);
  else if (rows <= 1) launch_partial<1>(fused, a, st);
  else if (rows <= 2) launch_partial<2>(fused, a, st);
  else if (rows <= 4) launch_partial<4>(fused, a, st);
  else launch_partial<8>(fused, a, st);
  if (a.splits == 1 || a.done || launch_status() != HTN_OK) return launch_status();
  MergeArgs m{a.part, a.ml, a.out, a.o_sb, a.o_sh, a.o_st, a.splits, a.Hq, a.Q};
  hipLaunchKernelGGL(attention_merge, dim3(static_cast<long>(a.B) * a.Hq * a.Q), dim3(kBlock), 0,
                     st, m);
  return launch_status();
}

}  // namespace

extern "C" int64_t htn_attention_scratch_bytes(int64_t B, int64_t Hq, int64_t Q, int64_t cap) {
  if (B <= 0 || Hq <= 0 || Q <= 0 || cap <= 0) return 0;
  if (Q > kMaxQ) return kCounterBytes;  // the prefill kernel keeps no partials
  // The smallest split the plan picks is kMinSplit slots.
  const long splits = (cap + kMinSplit - 1) / kMinSplit;
  return kCounterBytes + static_cast<long>(B) * Hq * Q * splits * (D + 2) * 4;
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
  // Heads are moved in 8-byte pieces: 4-element aligned rows only.
  const void* ptrs[] = {q, k, v, q_gain, k_gain, cos, sin, keys, values, out_q, out_k};
  for (const void* p : ptrs)
    if (!aligned8(p)) return HTN_EUNSUPPORTED;
  if ((q_sb | q_st | k_sb | k_st | rope_st | (v ? (v_sb | v_st) : 0)) & 3) return HTN_EUNSUPPORTED;
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
  // One wave per (token, 16-head chunk), four waves per block.
  const int64_t waves = B * T * ((Hq + 15) / 16 + (Hkv + 15) / 16);
  if (waves >= (int64_t{1} << 31)) return HTN_EUNSUPPORTED;
  hipLaunchKernelGGL(norm_rope_cache_kernel, dim3((waves + 3) / 4), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status();
}

extern "C" int htn_grouped_attention(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                                     const void* keys, const void* values, int64_t cap,
                                     const int64_t* positions, void* out, int64_t o_sb,
                                     int64_t o_sh, int64_t o_st, int64_t B, int64_t Hq,
                                     int64_t Hkv, int64_t Q, void* scratch,
                                     htn_stream_t stream) {
  if (!q || !keys || !values || !positions || !out) return HTN_EINVAL;
  if (o_sb < 0 || o_sh < 0 || o_st < 0) return HTN_EINVAL;
  if (Hkv <= 0 || Hq % Hkv != 0 || Q <= 0) return HTN_EINVAL;
  if (!aligned16(keys) || !aligned16(values)) return HTN_EUNSUPPORTED;
  // Query rows are read as bf16 pairs.
  if ((reinterpret_cast<uintptr_t>(q) & 3u) || ((q_sb | q_sh | q_st) & 1)) return HTN_EUNSUPPORTED;
  AttnArgs a{};
  a.q = static_cast<const bf16_t*>(q); a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.keys = static_cast<bf16_t*>(const_cast<void*>(keys));
  a.values = static_cast<bf16_t*>(const_cast<void*>(values));
  a.cap = cap; a.pos = positions; a.out = static_cast<bf16_t*>(out);
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.B = static_cast<int>(B); a.Hq = static_cast<int>(Hq); a.Hkv = static_cast<int>(Hkv);
  a.G = static_cast<int>(Hq / Hkv); a.Q = static_cast<int>(Q);
  if (Q > kMaxQ) return run_prefill_attention(a, static_cast<hipStream_t>(stream));
  return run_attention(false, a, scratch, static_cast<hipStream_t>(stream));
}

namespace {
int prologue_attention(const void* qkv, int64_t qkv_sb, int64_t k_off, int64_t v_off,
                       const void* q_gain, const void* k_gain, float q_eps, float k_eps,
                       const void* cos, const void* sin, int64_t rope_st, int64_t rope_rows,
                       int rope_by_position, void* keys, void* values, int64_t cap,
                       const int64_t* positions, void* out, int64_t B, int64_t Hkv,
                       int64_t groups, void* scratch, const NextWeights* next,
                       htn_stream_t stream, const FusedOutput* fo = nullptr,
                       bool* fused_output = nullptr) {
  if (!qkv || !q_gain || !k_gain || !cos || !sin || !keys || !values || !positions || !out)
    return HTN_EINVAL;
  if (Hkv <= 0 || groups <= 0 || rope_rows <= 0) return HTN_EINVAL;
  const void* ptrs[] = {qkv, q_gain, k_gain, cos, sin};
  for (const void* p : ptrs)
    if (!aligned8(p)) return HTN_EUNSUPPORTED;
  if ((qkv_sb | k_off | v_off | rope_st) & 3) return HTN_EUNSUPPORTED;
  if (!aligned16(keys) || !aligned16(values)) return HTN_EUNSUPPORTED;
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
  a.o_sh = D; a.o_st = D; a.o_sb = static_cast<long>(a.Hq) * D;  // out [B, Hq, 128]
  const int rc = run_attention(true, a, scratch, static_cast<hipStream_t>(stream), next, fo);
  if (fused_output) *fused_output = a.ow != nullptr;
  return rc;
}
}  // namespace

extern "C" int htn_prologue_attention(const void* qkv, int64_t qkv_sb, int64_t k_off,
                                      int64_t v_off, const void* q_gain, const void* k_gain,
                                      float q_eps, float k_eps, const void* cos, const void* sin,
                                      int64_t rope_st, int64_t rope_rows, int rope_by_position,
                                      void* keys, void* values, int64_t cap,
                                      const int64_t* positions, void* out, int64_t B,
                                      int64_t Hkv, int64_t groups, void* scratch,
                                      htn_stream_t stream) {
  return prologue_attention(qkv, qkv_sb, k_off, v_off, q_gain, k_gain, q_eps, k_eps, cos, sin,
                            rope_st, rope_rows, rope_by_position, keys, values, cap, positions,
                            out, B, Hkv, groups, scratch, nullptr, stream);
}

extern "C" int htn_prologue_attention_prefetch(
    const void* qkv, int64_t qkv_sb, int64_t k_off, int64_t v_off, const void* q_gain,
    const void* k_gain, float q_eps, float k_eps, const void* cos, const void* sin,
    int64_t rope_st, int64_t rope_rows, int rope_by_position, void* keys, void* values,
    int64_t cap, const int64_t* positions, void* out, int64_t B, int64_t Hkv, int64_t groups,
    void* scratch, const void* next_w, int64_t next_n, int64_t next_k, int next_format,
    htn_stream_t stream) {
  if (!next_w || next_n <= 0 || next_k <= 0 ||
      (next_format != 0 && next_format != HTN_WEIGHT_INT8 && next_format != HTN_WEIGHT_FP8_E4M3))
    return HTN_EINVAL;
  const NextWeights next{next_w, next_n, next_k, next_format};
  return prologue_attention(qkv, qkv_sb, k_off, v_off, q_gain, k_gain, q_eps, k_eps, cos, sin,
                            rope_st, rope_rows, rope_by_position, keys, values, cap, positions,
                            out, B, Hkv, groups, scratch, &next, stream);
}

namespace {
// Scratch of htn_prologue_attention_output: the attention's (counters and
// the fused projection's row accumulators, then split partials), then the
// attention rows of the unfused fallback.
long output_scratch_layout(long B, long Hq, long cap, long* rows_off) {
  *rows_off = (htn_attention_scratch_bytes(B, Hq, 1, cap) + 255) / 256 * 256;
  return *rows_off + B * Hq * D * 2;
}

// Calls of htn_prologue_attention_output that ran the fused projection.
std::atomic<long> fused_output_calls{0};
}  // namespace

extern "C" int64_t htn_attention_output_scratch_bytes(int64_t B, int64_t Hq, int64_t Hkv,
                                                      int64_t cap, int64_t n) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || cap <= 0 || n <= 0) return 0;
  long ro = 0;
  return output_scratch_layout(B, Hq, cap, &ro);
}

extern "C" int htn_prologue_attention_output(
    const void* qkv, int64_t qkv_sb, int64_t k_off, int64_t v_off, const void* q_gain,
    const void* k_gain, float q_eps, float k_eps, const void* cos, const void* sin,
    int64_t rope_st, int64_t rope_rows, int rope_by_position, void* keys, void* values,
    int64_t cap, const int64_t* positions, int64_t B, int64_t Hkv, int64_t groups,
    const void* o_weight, const float* o_scale, int o_format, int64_t n,
    const void* residual, void* out, void* scratch, htn_stream_t stream) {
  if (!o_weight || !residual || !out || !scratch || n <= 0 || B <= 0 || Hkv <= 0 || groups <= 0)
    return HTN_EINVAL;
  if (o_format != 0 && o_format != HTN_WEIGHT_INT8 && o_format != HTN_WEIGHT_FP8_E4M3)
    return HTN_EINVAL;
  if (o_format != 0 && !o_scale) return HTN_EINVAL;
  const long Hq = Hkv * groups, k = Hq * D;
  long ro = 0;
  output_scratch_layout(B, Hq, cap, &ro);
  unsigned char* sb = static_cast<unsigned char*>(scratch);
  unsigned long long* acc = reinterpret_cast<unsigned long long*>(sb + kOAccByte);
  bf16_t* rows = reinterpret_cast<bf16_t*>(sb + ro);
  const FusedOutput fo{o_weight, n, k, o_format, acc, o_scale,
                       static_cast<const bf16_t*>(residual), static_cast<bf16_t*>(out)};
  // Unfused, the attention's idle CUs still prefetch W_o into L2.
  const NextWeights next{o_weight, n, k, o_format};
  bool fused = false;
  int rc = prologue_attention(qkv, qkv_sb, k_off, v_off, q_gain, k_gain, q_eps, k_eps, cos, sin,
                              rope_st, rope_rows, rope_by_position, keys, values, cap, positions,
                              rows, B, Hkv, groups, scratch, &next, stream, &fo, &fused);
  if (rc != HTN_OK) return rc;
  if (fused) {
    fused_output_calls.fetch_add(1);
    return HTN_OK;  // the launch wrote `out`
  }
  // Unfused: the attention rows went to scratch; the residual GEMV follows.
  for (long b = 0; b < B; ++b) {
    const bf16_t* x = rows + b * k;
    const bf16_t* r = static_cast<const bf16_t*>(residual) + b * n;
    bf16_t* y = static_cast<bf16_t*>(out) + b * n;
    rc = o_format == 0 ? htn_gemv_residual(x, o_weight, r, y, n, k, stream)
                       : htn_gemv_residual_w8(x, o_weight, o_scale, o_format, r, y, n, k, stream);
    if (rc != HTN_OK) return rc;
  }
  return HTN_OK;
}

extern "C" int64_t htn_attention_output_fused_calls() { return fused_output_calls.load(); }

extern "C" int htn_xcc_ids(int32_t* out, int64_t blocks, htn_stream_t stream) {
  if (!out || blocks <= 0 || blocks > (1L << 20)) return HTN_EINVAL;
  hipLaunchKernelGGL(xcc_ids_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kWave), 0,
                     static_cast<hipStream_t>(stream), out, static_cast<long>(blocks));
  return launch_status();
}

extern "C" int htn_attention_merge_in_kernel() { return xcd_affine_merge(nullptr) ? 1 : 0; }

extern "C" int htn_attention_disable_in_kernel_merge() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return HTN_EINVAL;
  merge_state[dev].store(2);
  return HTN_OK;
}
