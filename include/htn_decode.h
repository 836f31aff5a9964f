/* htn_decode.h -- C ABI of the MI355X (gfx950) batch-one Qwen3 decode kernels.
 *
 * Every entry point takes raw device pointers, explicit sizes/strides and a
 * HIP stream (passed as void*), launches asynchronously on that stream and
 * returns HTN_OK or a negative error code. No entry point allocates device
 * memory, synchronises the host or reads device data on the host, so all of
 * them may be captured into a HIP graph.
 *
 * bf16 tensors are raw 16-bit patterns. Unless a stride is given, tensors are
 * contiguous row-major. Positions and token ids are int64 device arrays that
 * the kernels read on the device (graph replays see updated values).
 *
 * "scratch" buffers are caller-owned device memory for per-block partial
 * results, sized as each entry point states; no initial contents are
 * required, except the attention scratch's leading arrival counters (see
 * htn_attention_scratch_bytes). Calls that run concurrently on one scratch
 * buffer race.
 * Cross-block reductions are finished by a second, stream-ordered launch,
 * except the split-KV attention merge, which the last split of each (batch,
 * kv head) pair performs in the same launch (see htn_grouped_attention).
 *
 * Reference interfaces cited as file:line are in rickytang666/hackthenorth,
 * under dryft/engine/.
 */
#ifndef HTN_DECODE_H
#define HTN_DECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HTN_OK 0
#define HTN_EINVAL (-1)       /* bad pointer, size, stride or alignment */
#define HTN_EUNSUPPORTED (-2) /* shape the kernels do not implement */
#define HTN_ELAUNCH (-3)      /* the HIP launch failed */

#define HTN_HEAD_SCRATCH_BYTES 65536
#define HTN_HEAD_DIM 128

/* 8-bit weight formats of the *_w8 GEMVs (one byte per weight, row-major,
 * one fp32 scale per weight row). */
#define HTN_WEIGHT_INT8 1     /* two's complement int8 */
#define HTN_WEIGHT_FP8_E4M3 2 /* OCP fp8 e4m3fn (bias 7, no infinities, 0x7f/0xff NaN) */

/* Epilogues of htn_gemm_rows. */
#define HTN_EPI_STORE 0    /* y = bf16(dot) */
#define HTN_EPI_RESIDUAL 1 /* y = bf16(bf16(dot) + residual) */
#define HTN_EPI_SWIGLU 2   /* y = bf16(bf16(silu(bf16 gate)) * bf16 up), w holds 2n rows */
#define HTN_EPI_ARGMAX 3   /* tokens[m] = argmax_n bf16(dot), lowest id on ties */
#define HTN_EPI_RESIDUAL_NORM 4 /* scratch query of htn_gemm_rows_residual_norm */

typedef void* htn_stream_t;

/* Library version, for the loader's sanity check. */
int htn_version(void);

/* ---------------------------------------------------------------- weights */

/* out[i] = bf16(f32(IrwinHall4(hash(seed, stream, start + i)) - 131070) * scale),
 * i < count. Bit-identical to the numpy generator used by the tests.
 * Replaces the reference's torch RNG initialisation of random weights. */
int htn_fill_normal_bf16(void* out, int64_t count, uint64_t seed, uint64_t stream,
                         int64_t start, float scale, htn_stream_t stream_);

/* out[i] = floor((hash >> 32) * high / 2^32) as int64. */
int htn_fill_randint_i64(int64_t* out, int64_t count, uint64_t seed, uint64_t stream,
                         int64_t high, htn_stream_t stream_);

/* out[i] = lo + span * (f32(hash >> 40) * 2^-24), each operation rounded
 * once in fp32 (synthetic per-channel weight scales, lo = 0.001 and span =
 * 0.009 for U(0.001, 0.01)). No reference counterpart: the 8-bit weight
 * variants are an addition to the reference's bf16-only decode path. */
int htn_fill_uniform_f32(float* out, int64_t count, uint64_t seed, uint64_t stream, float lo,
                         float span, htn_stream_t stream_);

/* Synthetic 8-bit weights: v = floor((hash >> 32) * 255 / 2^32) - 127, a
 * uniform integer in [-127, 127], stored as int8 (format HTN_WEIGHT_INT8) or
 * as its round-to-nearest-even fp8 e4m3fn encoding (HTN_WEIGHT_FP8_E4M3).
 * No reference counterpart (see htn_fill_uniform_f32). */
int htn_fill_weights_w8(void* out, int64_t count, uint64_t seed, uint64_t stream, int format,
                        htn_stream_t stream_);

/* ---------------------------------------------------------------- gather */

/* out[t, :] = table[ids[t], :] for t < count (bf16 rows of `hidden`).
 * Ids outside [0, vocab) produce a zero row instead of an out-of-bounds read.
 * Replaces base.embed_tokens(token_ids), decode.py:81. */
int htn_embed_gather(const int64_t* ids, int64_t count, const void* table, int64_t vocab,
                     int64_t hidden, void* out, htn_stream_t stream);

/* Two htn_embed_gather calls in one launch (hidden sizes multiples of 8,
 * tables and outputs 16-byte aligned, else HTN_EUNSUPPORTED). The decode step
 * gathers its token row and its RoPE (cos | sin) row this way. Replaces
 * base.embed_tokens(token_ids), decode.py:81, plus the rotary row lookup of
 * decode.py:49-67 in one kernel (the reference runs them as separate ops). */
int htn_embed_gather_pair(const int64_t* ids_a, int64_t count_a, const void* table_a,
                          int64_t vocab_a, int64_t hidden_a, void* out_a,
                          const int64_t* ids_b, int64_t count_b, const void* table_b,
                          int64_t vocab_b, int64_t hidden_b, void* out_b, htn_stream_t stream);

/* ---------------------------------------------------------------- norms */

/* out = bf16(gain * bf16(x * rsqrt(mean(x^2) + eps))) per row.
 * Replaces rms_norm(x, weight, eps), kernels/rmsnorm.py:84. */
int htn_rms_norm(const void* x, int64_t x_row_stride, const void* gain, void* out,
                 int64_t rows, int64_t cols, float eps, htn_stream_t stream);

/* summed = bf16(x + residual); normalized = rms_norm(summed).
 * Replaces add_rms_norm(x, residual, weight, eps), kernels/rmsnorm.py:35. */
int htn_add_rms_norm(const void* x, const void* residual, const void* gain, void* summed,
                     void* normalized, int64_t rows, int64_t cols, float eps,
                     htn_stream_t stream);

/* out[r, c] = bf16(bf16(silu(gate[r, c])) * up[r, c]); out contiguous.
 * Replaces swiglu(gate, up), kernels/fused.py:171. */
int htn_swiglu(const void* gate, int64_t gate_row_stride, const void* up,
               int64_t up_row_stride, void* out, int64_t rows, int64_t cols,
               htn_stream_t stream);

/* ---------------------------------------------------------------- batch-one GEMV */

/* y[n] = bf16(sum_k x[k] * w[n, k]) for n < rows; w is [rows, k] row-major. */
int htn_gemv(const void* x, const void* w, void* y, int64_t rows, int64_t k,
             htn_stream_t stream);

/* RMSNorm prologue then projection: y = W . bf16(gain * bf16(x * inv)).
 * swiglu != 0: w holds gate rows [0, rows) then up rows [rows, 2 rows) and
 * y[n] = bf16(bf16(silu(bf16 gate_n)) * bf16 up_n).
 * Replaces norm_projection(x, gain, weight, eps, swiglu=...),
 * kernels/projection.py:36. */
int htn_gemv_norm(const void* x, const void* gain, float eps, const void* w, void* y,
                  int64_t rows, int64_t k, int swiglu, htn_stream_t stream);

/* y[n] = bf16(bf16(sum_k x[k] w[n, k]) + residual[n]).
 * Replaces output_projection_residual(x, weight, residual),
 * kernels/projection.py:70, and down_residual(x, w, residual),
 * kernels/down.py:27 (same rounding: projection rounded before the add). */
int htn_gemv_residual(const void* x, const void* w, const void* residual, void* y,
                      int64_t rows, int64_t k, htn_stream_t stream);

/* Greedy head: token = argmax_n bf16(W[n] . xn) with the lowest id on ties,
 * where xn = x, or rms_norm(x, gain, eps) when gain is not NULL (the final
 * norm fused in). Writes token_out[0]; when position_inc is not NULL it also
 * adds 1 to position_inc[0] (the decode step's position.add_(1)). Two
 * launches: the GEMV leaves one key per block in `scratch`
 * (HTN_HEAD_SCRATCH_BYTES), a one-block kernel reduces them.
 * Replaces greedy_token(x, w), kernels/greedy.py:45, and
 * lm_head(x).argmax(-1), decode.py:96-99. */
int htn_lm_head_argmax(const void* x, const void* gain, float eps, const void* w,
                       int64_t vocab, int64_t k, int64_t* token_out,
                       int64_t* position_inc, void* scratch, htn_stream_t stream);

/* htn_lm_head_argmax without the scratch argument: the per-block keys go to
 * a fixed device array of HTN_HEAD_SCRATCH_BYTES that the library holds on
 * every GPU it runs on until the process ends (its address is looked up once
 * per device, on the first call there). Allocates nothing, so it can be
 * called where hipMalloc cannot (under HIP graph capture, in serving loops
 * that forbid allocation). Same results and limits as htn_lm_head_argmax
 * (k <= 16384 and vocab <= 2^31, else HTN_EINVAL); the grid never writes
 * more keys than the array holds. All calls on one GPU share the array, so
 * calls that overlap on one GPU (concurrent streams) race; calls ordered on
 * one stream do not. No initial contents are needed: every call writes each
 * key it reads.
 * No counterpart in the reference: it exists for callers that cannot
 * allocate device memory. */
int htn_lm_head_argmax_noalloc(const void* x, const void* gain, float eps, const void* w,
                               int64_t vocab, int64_t k, int64_t* token_out,
                               int64_t* position_inc, htn_stream_t stream);
/* Bytes of the fixed key array above (HTN_HEAD_SCRATCH_BYTES). */
int64_t htn_head_scratch_capacity(void);

/* ---------------------------------------------------------------- 8-bit weights
 * Weight-only 8-bit twins of the four GEMVs above: w holds rows*k bytes in
 * `format` (HTN_WEIGHT_*), scales[n] is the fp32 scale of weight row n
 * (gate/up: 2*rows scales, gate rows first). Every dot product is
 *   y[n] = s_n * sum_k x[k] * w[n, k]   (fp32 accumulate, then the scale),
 * rounded to bf16 where the bf16 GEMV rounds its plain dot product, so the
 * norm prologue and the SwiGLU / residual / argmax epilogues keep the same
 * rounding boundaries. k must be a multiple of 16 and x, gain and w 16-byte
 * aligned (HTN_EUNSUPPORTED otherwise).
 * No reference counterpart: dryft decodes in bf16 only; these cover the
 * int8 / fp8 weight-only decode of the same projections (QKV, O, gate/up,
 * down, LM head). */
int htn_gemv_w8(const void* x, const void* w, const float* scales, int format, void* y,
                int64_t rows, int64_t k, htn_stream_t stream);
int htn_gemv_norm_w8(const void* x, const void* gain, float eps, const void* w,
                     const float* scales, int format, void* y, int64_t rows, int64_t k,
                     int swiglu, htn_stream_t stream);
int htn_gemv_residual_w8(const void* x, const void* w, const float* scales, int format,
                         const void* residual, void* y, int64_t rows, int64_t k,
                         htn_stream_t stream);
int htn_lm_head_argmax_w8(const void* x, const void* gain, float eps, const void* w,
                          const float* scales, int format, int64_t vocab, int64_t k,
                          int64_t* token_out, int64_t* position_inc, void* scratch,
                          htn_stream_t stream);

/* ---------------------------------------------------------------- 2..128 rows
 * Projection of `rows` (1..128) activation rows x[m, :k] (row stride
 * x_stride elements) by a row-major bf16 weight w[n, k] (2n rows, gate then
 * up, for HTN_EPI_SWIGLU), reading the weight once for all rows (MFMA tiles).
 * gain != NULL applies RMSNorm to each row first:
 *   x' = bf16(gain * bf16(x * rsqrt(mean(x^2) + eps))).
 * Epilogues (HTN_EPI_*): y[m, n] (row stride y_stride) as the batch-one GEMVs
 * round it, + residual[m, n] (row stride res_stride), SwiGLU, or tokens[m]
 * (int64 device array) = per-row argmax. k must be a multiple of 64, x
 * (with its stride), gain and w 16-byte aligned.
 * scratch: htn_gemm_rows_scratch_bytes(rows, n, k, epilogue, gain != NULL)
 * bytes (the normalised rows, K-split partials or per-strip argmax keys; 0
 * means none is needed).
 * Replaces the reference's multi-row decode projections: Projection._tile
 * (projections.py:168-183), gate_up_swiglu (kernels/gateup.py:40-58) and the
 * split down projection (kernels/split_down.py:85-101). */
int64_t htn_gemm_rows_scratch_bytes(int64_t rows, int64_t n, int64_t k, int epilogue, int norm);
int htn_gemm_rows(const void* x, int64_t x_stride, const void* gain, float eps, const void* w,
                  int64_t n, int64_t k, int64_t rows, int epilogue, const void* residual,
                  int64_t res_stride, void* y, int64_t y_stride, int64_t* tokens, void* scratch,
                  htn_stream_t stream);

/* The residual projection of htn_gemm_rows (HTN_EPI_RESIDUAL, no input norm)
 * fused with the next RMSNorm of its output:
 *   y[m, :]      = bf16(bf16(W x_m) + residual[m, :])      (row stride y_stride)
 *   normed[m, :] = bf16(gain * bf16(y[m, :] * rsqrt(mean(y[m, :]^2) + eps)))
 * normed is contiguous [rows, n]. When the projection splits K (its plan is
 * htn_gemm_rows'), the split finish computes both in one launch; otherwise,
 * and for rows wider than 8192 or unaligned pointers, the projection is
 * followed by htn_rms_norm. Both paths give the same bits.
 * scratch: htn_gemm_rows_scratch_bytes(rows, n, k, HTN_EPI_RESIDUAL_NORM, 0)
 * bytes.
 * Replaces the reference's split_down_residual_norm
 * (dryft/engine/kernels/split_down.py:85-101). */
int htn_gemm_rows_residual_norm(const void* x, int64_t x_stride, const void* w, int64_t n,
                                int64_t k, int64_t rows, const void* residual,
                                int64_t res_stride, void* y, int64_t y_stride, const void* gain,
                                float eps, void* normed, void* scratch, htn_stream_t stream);

/* The projection of many rows at once (a prompt's prefill: hundreds to
 * thousands of rows): y = x W^T as a tiled GEMM on the matrix cores, one
 * launch, 128 x 128 output tiles, both operands staged in LDS (weight tiles
 * reused from the L2 of one XCD by every row tile). Epilogues HTN_EPI_STORE,
 * HTN_EPI_RESIDUAL and HTN_EPI_SWIGLU as htn_gemm_rows (w holds 2n rows for
 * SwiGLU: gate rows, then up rows); no input RMSNorm (normalise the rows
 * first with htn_rms_norm). Rows are x[m, :k] with row stride x_stride; y
 * (and the residual) [rows, n] with row strides y_stride (res_stride). k must
 * be a multiple of 64 and at most 2^20, x_stride a multiple of 8 and
 * y_stride of 4, x and w 16-byte and y 8-byte aligned. fp32 accumulation
 * over k in 64-wide steps; bf16 rounding boundaries as htn_gemm_rows.
 * Replaces the reference's projections over the whole prompt in its prefill
 * forward (prefill.py:6-26 -> DecodeState.prefill, decode.py:156-166). */
int htn_gemm_tiles(const void* x, int64_t x_stride, const void* w, int64_t n, int64_t k,
                   int64_t rows, int epilogue, const void* residual, int64_t res_stride, void* y,
                   int64_t y_stride, void* scratch, htn_stream_t stream);

/* Scratch bytes htn_gemm_tiles uses for these sizes (0: none). When the tile
 * grid alone fills at most half of the blocks the CUs hold at once (prompts
 * of a few hundred rows), each tile's k range splits over up to 8 blocks whose fp32
 * partial sums go to `scratch` (16-byte aligned) and a second launch adds
 * them in split order; with scratch NULL every tile sums its whole k range.
 * The two orders of the fp32 sums may round an output 1 bf16 ulp apart. */
int64_t htn_gemm_tiles_scratch_bytes(int64_t rows, int64_t n, int64_t k, int epilogue);

/* y[m, n] = bf16(sum_k x[m, k] * w[n, k]) (fp32 accumulation) for every row
 * m < rows, through hipBLASLt: the plain product of a prefill projection,
 * whose epilogues (residual add with the next RMSNorm, SwiGLU) then run as
 * htn_add_rms_norm / htn_swiglu with the same bf16 rounding boundaries as
 * htn_gemm_tiles' fused ones. x, w, y and workspace 16-byte aligned, k and
 * the row strides multiples of 8; workspace holds
 * htn_gemm_library_workspace_bytes() bytes. HTN_EUNSUPPORTED when the
 * library offers no algorithm for the shape (htn_gemm_tiles covers it).
 * The first call for a shape outside stream capture also picks the
 * algorithm: it times the library's candidates whose output equals the
 * heuristic's first (bit for bit, on the call's operands), each with its
 * weights from HBM, and keeps the fastest if it beats the first by at least
 * 5%, so results never depend on the pick; that call allocates about 512 MB
 * plus a copy of y for the duration, and synchronises the stream. Calls
 * under capture before it use the heuristic's first algorithm.
 * Replaces, with those epilogue launches, the reference's prefill
 * projections (prefill.py:6-26 -> projections.py:168-183 over the prompt). */
int64_t htn_gemm_library_workspace_bytes(void);
int htn_gemm_library(const void* x, int64_t x_stride, const void* w, int64_t n, int64_t k,
                     int64_t rows, void* y, int64_t y_stride, void* workspace,
                     htn_stream_t stream);

/* SwiGLU of `rows` (1..32) activation rows x[m, :k] (row stride x_stride)
 * by the interleaved K-major weight w[k, 2 * width] (row-major, w[k, 2i] the
 * gate and w[k, 2i + 1] the up weight of output i):
 *   y[m, i] = bf16(bf16(silu(bf16(gate))) * bf16(up))   (row stride y_stride)
 * read in place, the weight once for all rows (MFMA tiles). k must be a
 * multiple of 32, width even, x (with its stride) 16-byte and w 8-byte
 * aligned.
 * scratch: htn_gate_up_swiglu_scratch_bytes(rows, width, k) bytes (K-split
 * partials; 0 means none is needed).
 * Replaces the reference's gate_up_swiglu (dryft/engine/kernels/gateup.py:40-58)
 * on its own weight layout. */
int64_t htn_gate_up_swiglu_scratch_bytes(int64_t rows, int64_t width, int64_t k);
int htn_gate_up_swiglu(const void* x, int64_t x_stride, const void* w, int64_t width, int64_t k,
                       int64_t rows, void* y, int64_t y_stride, void* scratch,
                       htn_stream_t stream);

/* Measurement helper with no reference counterpart: reads `bytes` (a
 * multiple of 16, 16-byte aligned) of src once with streaming 16-byte loads
 * and writes one XOR-folded word per block to out[0 .. htn_stream_read_blocks()),
 * so that benchmarks can quote a kernel's bandwidth against the measured
 * streaming-read ceiling beside the nominal HBM peak. */
int64_t htn_stream_read_blocks(void);
int htn_stream_read(const void* src, int64_t bytes, uint32_t* out, htn_stream_t stream);

/* out[r] = argmax over bf16 logits[r, :n] (lowest id on ties) for r < rows. */
int htn_argmax_bf16(const void* logits, int64_t rows, int64_t n, int64_t* out,
                    htn_stream_t stream);

/* ---------------------------------------------------------------- attention (D = 128) */

/* Per-head RMSNorm + RoPE of q and k, for tokens t < T of batch b < B:
 *   q[b, t, h, :] at q + b*q_sb + t*q_st + h*128 (likewise k, v);
 *   cos/sin row for token t at cos + rope_row(t)*rope_st, where
 *   rope_row(t) = positions[t] if rope_by_position else t; rows at or past
 *   rope_rows (the table length) are skipped, never read.
 * out_q is [B, T, Hq, 128] contiguous. When keys/values are not NULL the
 * normalised k and the raw v are written to cache slot positions[t] of the
 * [B, Hkv, cap, 128] caches; when out_k is not NULL the normalised k is also
 * written to out_k [B, T, Hkv, 128]. positions may be NULL when it is not
 * needed (no cache write and rope_by_position == 0).
 * Replaces norm_rope_cache(...), kernels/fused.py:70, and
 * norm_rope(...), kernels/fused.py:132. */
int htn_norm_rope_cache(const void* q, int64_t q_sb, int64_t q_st, const void* k,
                        int64_t k_sb, int64_t k_st, const void* v, int64_t v_sb,
                        int64_t v_st, const void* q_gain, const void* k_gain, float q_eps,
                        float k_eps, const void* cos, const void* sin, int64_t rope_st,
                        int64_t rope_rows, int rope_by_position, void* keys, void* values,
                        int64_t cap,
                        const int64_t* positions, void* out_q, void* out_k, int64_t B,
                        int64_t T, int64_t Hq, int64_t Hkv, htn_stream_t stream);

/* Bytes of scratch the attention entry points need for these sizes (for Q > 8,
 * the causal many-query kernel, only the counter region). The first
 * HTN_ATTENTION_COUNTER_BYTES hold arrival counters (32 KB) and the fused
 * output projection's row accumulators (64 KB): zero them once when the
 * buffer is allocated; every call leaves them zero. Calls sharing a scratch
 * buffer must be ordered (one stream). */
#define HTN_ATTENTION_COUNTER_BYTES 98304
/* Byte offset of the fused output projection's accumulators: one 64-bit
 * word per output row (at most 8192), zero between calls. */
#define HTN_ATTENTION_OUTPUT_ACC_BYTE 32768
/* Byte offset, inside the counter region, of a 32-bit count of in-kernel
 * merges that found a split of their (batch, kv head) pair on another XCD
 * than their own (dispatch not round-robin, so that split's partial may not
 * have been visible to the merge). It stays 0 on a correct run and, unlike the
 * arrival counters, is never reset by the kernels: the caller reads it (any
 * time after the calls it covers) and clears it. */
#define HTN_ATTENTION_XCD_MISMATCH_BYTE 8
/* Byte offset, inside the counter region, of a 32-bit count of fused
 * output-projection blocks (htn_prologue_attention_output) that could not use
 * their pair's attention partials (they ran on another XCD than the pair's
 * splits, or the splits had not arrived within the wait bound), plus row
 * partials outside the fixed-point accumulator's range (|partial| >= 2^24
 * with bf16 weights, 2^32 with 8-bit ones). 0 on a correct run; never reset
 * by the kernels (the caller reads and clears it). */
#define HTN_ATTENTION_OUTPUT_ERROR_BYTE 12
int64_t htn_attention_scratch_bytes(int64_t B, int64_t Hq, int64_t Q, int64_t cap);

/* Grouped-query attention over fixed-capacity caches with causality by
 * absolute position: query t of head h sees slots <= positions[t] of kv head
 * h / (Hq / Hkv); later slots are never read. q[b, h, t, :] at
 * q + b*q_sb + h*q_sh + t*q_st; out[b, h, t, :] at out + b*o_sb + h*o_sh +
 * t*o_st (element strides; dims contiguous), so a token-major [B, Q, Hq, 128]
 * output feeds the output projection without a transpose.
 * Split-KV: each split writes an unnormalised partial and its (max, sum) to
 * `scratch` (htn_attention_scratch_bytes). Workgroups are dispatched to the
 * XCDs round-robin, so the splits of one (batch, kv head) pair are laid on a
 * single XCD and the last of them to arrive merges the pair's rows from that
 * XCD's L2 in the same launch. Where the device's XCD count does not divide
 * 8, for more than 256 (batch, kv head) pairs, for the streaming long-context
 * kernel, or with the environment variable HTN_ATTENTION_MERGE_LAUNCH=1, a
 * second launch merges instead. One launch when the context fits one split.
 * More than 8 queries per sequence (a prompt's prefill): one causal launch,
 * no split and no scratch use; q must be 16-byte aligned with element strides
 * that are multiples of 8, out 8-byte aligned with strides that are multiples
 * of 4 (HTN_EUNSUPPORTED otherwise). It plays the part of the reference's
 * causal flash attention over the prompt (attention.py:92-98).
 * Replaces grouped_attention(q, k, v, positions), kernels/attention.py:213. */
int htn_grouped_attention(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                          const void* keys, const void* values, int64_t cap,
                          const int64_t* positions, void* out, int64_t o_sb, int64_t o_sh,
                          int64_t o_st, int64_t B, int64_t Hq, int64_t Hkv, int64_t Q,
                          void* scratch, htn_stream_t stream);

/* Single-token decode attention with the QK-norm/RoPE/cache append fused in:
 * q, the newest k and v come from the packed projection row
 * qkv[b, :] (row stride qkv_sb; k at k_off, v at v_off). The cos/sin row is
 * cos + rope_row*rope_st with rope_row = positions[0] if rope_by_position
 * else 0. Writes the newest k/v into slot positions[0] and returns
 * out [B, Hq, 128].
 * Replaces prologue_attention(...), kernels/attention.py:162. */
int htn_prologue_attention(const void* qkv, int64_t qkv_sb, int64_t k_off, int64_t v_off,
                           const void* q_gain, const void* k_gain, float q_eps, float k_eps,
                           const void* cos, const void* sin, int64_t rope_st,
                           int64_t rope_rows, int rope_by_position, void* keys, void* values,
                           int64_t cap,
                           const int64_t* positions, void* out, int64_t B, int64_t Hkv,
                           int64_t groups, void* scratch, htn_stream_t stream);

/* htn_prologue_attention, plus the weight of the projection that reads its
 * output (next_n x next_k, format 0 = bf16, HTN_WEIGHT_INT8 or
 * HTN_WEIGHT_FP8_E4M3; row scales are not read): while the attention runs,
 * blocks on CUs it leaves idle read up to 3 MB of those weights per XCD into
 * the L2 of the XCD whose GEMV blocks will multiply them (one-token GEMV
 * grid, equal block index mod 8). Results are identical to
 * htn_prologue_attention; only the following projection gets faster. Used
 * with the XCD-affine split grid only (otherwise no prefetch).
 * Replaces prologue_attention(...), kernels/attention.py:162, in the decode
 * step (the reference has no such prefetch). */
int htn_prologue_attention_prefetch(
    const void* qkv, int64_t qkv_sb, int64_t k_off, int64_t v_off, const void* q_gain,
    const void* k_gain, float q_eps, float k_eps, const void* cos, const void* sin,
    int64_t rope_st, int64_t rope_rows, int rope_by_position, void* keys, void* values,
    int64_t cap, const int64_t* positions, void* out, int64_t B, int64_t Hkv, int64_t groups,
    void* scratch, const void* next_w, int64_t next_n, int64_t next_k, int next_format,
    htn_stream_t stream);

/* htn_prologue_attention followed by the output projection with its
 * residual: out[b, :] = bf16(bf16(W_o a[b]) + residual[b, :]) (8-bit W_o:
 * bf16(bf16(scale_n * (W_o a)_n) + residual_n)), with a[b] the attention
 * rows [Hq * 128] and W_o [n, Hq * 128] row-major (o_format 0 bf16, or
 * HTN_WEIGHT_INT8 / HTN_WEIGHT_FP8_E4M3 with o_scale [n] fp32). For one
 * sequence on the XCD-affine split grid (in-kernel merge) the projection
 * runs in the attention launch: blocks on each kv head's XCD hold that head
 * group's columns of W_o in registers while the attention runs, merge its
 * rows when its last split arrives, and add their row sums, in 64-bit fixed
 * point, into one accumulator word per output row (integer addition makes
 * the total independent of the arrival order; the contribution that
 * completes a row rounds it as the reference does -- any summation order
 * of the projection is the reference's contract -- adds the residual and
 * clears the word). Projections under 16 MB or over 8192 rows, and shapes
 * the fused kernel does not cover, take the unfused path: the attention rows go to scratch
 * and the residual GEMV follows. scratch holds htn_attention_output_scratch_bytes
 * bytes, its first HTN_ATTENTION_COUNTER_BYTES zero when allocated (every
 * call leaves them zero; a call that counted an error at
 * HTN_ATTENTION_OUTPUT_ERROR_BYTE may not).
 * Replaces prologue_attention(...) (kernels/attention.py:162) followed by
 * output_projection_residual(a, W_o, residual) (kernels/projection.py:70),
 * the pair fused_layer.py:146-147 runs. */
int64_t htn_attention_output_scratch_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t cap,
                                           int64_t n);
/* Diagnostic: how many htn_prologue_attention_output calls of this process
 * ran the projection inside the attention launch (the rest took the
 * unfused path). */
int64_t htn_attention_output_fused_calls(void);
int htn_prologue_attention_output(
    const void* qkv, int64_t qkv_sb, int64_t k_off, int64_t v_off, const void* q_gain,
    const void* k_gain, float q_eps, float k_eps, const void* cos, const void* sin,
    int64_t rope_st, int64_t rope_rows, int rope_by_position, void* keys, void* values,
    int64_t cap, const int64_t* positions, int64_t B, int64_t Hkv, int64_t groups,
    const void* o_weight, const float* o_scale, int o_format, int64_t n,
    const void* residual, void* out, void* scratch, htn_stream_t stream);

/* Diagnostics and control of the in-kernel attention merge; no counterpart
 * in the reference. htn_xcc_ids writes, for each block b < blocks of a
 * one-dimensional grid, the XCD it ran on (hardware register XCC_ID), so a
 * test can confirm the round-robin dispatch the merge relies on (blocks with
 * equal index mod 8 share an XCD). The first attention call on a device
 * outside stream capture runs that check itself (a 2048-block grid, one
 * small allocation, synchronous) and merges in-kernel only if it holds.
 * htn_attention_merge_in_kernel returns 1 if the attention entry points merge
 * splits in-kernel on the current device (running the check if it has not
 * run). htn_attention_disable_in_kernel_merge switches the current device to
 * the separate merge launch for the rest of the process (launches captured
 * earlier keep the mode they were captured with); the host calls it when a
 * merge has counted a split from another XCD (the 32-bit word at byte
 * HTN_ATTENTION_XCD_MISMATCH_BYTE of the attention scratch). */
int htn_xcc_ids(int32_t* out, int64_t blocks, htn_stream_t stream);
int htn_attention_merge_in_kernel(void);
int htn_attention_disable_in_kernel_merge(void);

#ifdef __cplusplus
}
#endif

#endif /* HTN_DECODE_H */
