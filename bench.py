"""Batch-one Qwen3 greedy decode throughput on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--headline-only]

Headline workload: the Qwen3-8B shape (hidden 4096, 36 layers, 32 q / 8 kv
heads, head_dim 128, FFN 12288, vocab 151936, untied LM head), random-init
bf16 weights N(0, 0.02), a 2048-token uniform-random prompt, then W untimed
and K timed greedy decode steps (defaults K = 256, W = 3: context 2048 ->
2303). A step is one replay of the captured decode graph; the timed region
replays K steps back to back with weights, KV cache and token/position state
already resident in HBM. `value` is decode tok/s.

Also on the same line:
  roofline        the dominant kernel of that step by per-step time (RMSNorm +
                  gate/up GEMV + SwiGLU, 36 x 31 us of the ~2.9 ms step): launched
                  back to back in a captured graph over the 36 layers' 201 MB
                  weights (7.2 GB, far beyond the 256 MB Infinity Cache), timed
                  with HIP events on the capturing stream; achieved = algorithmic
                  bytes / average launch; traffic = counted HBM bytes per launch
                  from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes;
                  also the fraction of a device copy's measured bandwidth;
  decode_roofline bytes per generated token (every weight once + KV) x tok/s
                  against 8 TB/s;
  prefill_s, prefill_kernels
                  the captured batched prefill of the 2048-token prompt (replay
                  time) and its matrix-core work at 2048 rows (the four
                  projections -- hipBLASLt products with their row-wise
                  epilogue launches -- and the causal attention, each over 8
                  layers back to back in a graph): microseconds, TFLOP/s and
                  the fraction of the 2.5 PFLOP/s dense bf16 peak;
  cpu_baseline    the CPU oracle (torch eager, this host's cores) on a bounded
                  sample of the same workload: one batched prefill of the 2048-token
                  prompt, then 32 decode steps fed the GPU's tokens, reported as
                  decode tok/s, with the teacher-forced parity record of the
                  GPU's first 33 tokens against the oracle's logits (differing
                  steps classified as near-ties within 1e-3, explained by the
                  oracle's own evaluation orders, or unexplained);
  qwen3_0.6b      the Qwen3-0.6B shape (tied), prompt 512, 64 steps, with its own
                  dominant kernel (the decode attention at context 512) and the
                  teacher-forced record of all 64 tokens;
  per_op          the row-wise fused ops at 0.6B widths, 32768 rows and one row;
  qwen3_8b_int8 / qwen3_8b_fp8
                  the 8B shape with weight-only int8 / fp8-e4m3fn projections and
                  LM head (uniform integer weights in [-127, 127], per-row scales
                  U(0.001, 0.01)), 128 steps at context 8192 over a synthetic KV
                  cache (N(0,1) keys and values in slots 0..8191);
  speculative_4b_draft_0.6b
                  4B-shape target + 0.6B-shape draft (random bf16), k = 4 draft
                  tokens verified in one 5-row pass, context 4096 (synthetic KV):
                  tok/s, measured greedy acceptance, verify / step / draft times;
  batched_qwen3_8b  the 8B shape at batch 4 and 16, context 512;
  prompt_lookup_qwen3_8b
                  Engine.generate on the 8B shape with batch-one prompt-lookup
                  speculation (the reference's production mode) beside plain
                  decode, on a repetitive 512-token prompt, 128 tokens;
  cpu_qwen3_0.6b_prompt32
                  the CPU oracle's whole 64-step greedy decode of the 0.6B shape
                  after a 32-token prompt (the reference's CPU configuration),
                  timed, against the golden ids, beside the GPU's decode of the
                  same request and its teacher-forced record.
"""
import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from hackthenorth_amd import _lib  # noqa: E402
from hackthenorth_amd import decode as D  # noqa: E402
from hackthenorth_amd.kernels import projection as P  # noqa: E402
from hackthenorth_amd.kernels import rng as DR  # noqa: E402
from hackthenorth_amd.model import Qwen3Model, shape_config  # noqa: E402
from hackthenorth_amd.prefill import prefill  # noqa: E402

METRIC = "batch-1 decode tok/s at Qwen3 shapes + per-kernel HBM GB/s as % of peak"
# Per-kernel HBM bytes of the 8B decode step, from the committed rocprofv3
# FETCH_SIZE / WRITE_SIZE passes (calibrated against a copy of known size).
PMC_PROFILE = os.path.join(ROOT, "profiles", "decode_per_kernel_hbm_qwen3-8b.txt")
TRACE_PROFILE = os.path.join(ROOT, "profiles", "decode_qwen3-8b_bf16_kernel_stats.txt")
HBM_PEAK_GBS = 8000.0
PROMPT_SEED, PROMPT_STREAM = 1, 7
DOMINANT_ROLE = "RMSNorm + gate/up GEMV + SwiGLU"


def measured_traffic(role=DOMINANT_ROLE):
    """Counted HBM bytes per launch (read + write) of a role in the per-kernel table."""
    try:
        with open(PMC_PROFILE) as f:
            for line in f:
                if line.startswith(role + " "):
                    cols = line[len(role):].split()
                    return int(round((float(cols[3]) + float(cols[4])) * 1e6))
    except (OSError, ValueError, IndexError):
        pass
    return None


def trace_average_us(kernel_prefix):
    """Average dispatch duration of a kernel in the committed kernel-trace summary."""
    try:
        with open(TRACE_PROFILE) as f:
            for line in f:
                if line.startswith(kernel_prefix):
                    return float(line[len(kernel_prefix):].split()[1])
    except (OSError, ValueError, IndexError):
        pass
    return None


def kv_bytes_per_token(cfg, ctx):
    """KV read over ctx slots plus the appended slot, all layers (bf16)."""
    per_slot = 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * cfg.head_dim * 2
    return per_slot * (ctx + 1)


def run_decode(shape, prompt_len, steps, warmup, log, weight_format="bf16",
               synthetic_context=False, batch=1, model=None, record_steps=0):
    """Greedy decode of `steps` tokens after a prompt of `prompt_len` tokens.

    synthetic_context: instead of prefilling, fill every KV slot with N(0,1)
    values and start decoding at position prompt_len (the step's cost does not
    depend on the cached values; this keeps 8192-token contexts cheap to set up).
    record_steps: the untimed pass that copies the emitted ids out runs
    max(steps, record_steps) steps (more ids for the parity record than the
    timed steps give).
    """
    cfg = shape_config(shape, weight_format=weight_format)
    if model is None:
        model = Qwen3Model.random(cfg)
    prompt = DR.randint(prompt_len, cfg.vocab_size, PROMPT_SEED, PROMPT_STREAM)
    recorded = max(steps, record_steps)
    total = max(warmup + steps, recorded) + 1
    with torch.inference_mode():
        state = D.DecodeState(model, batch, prompt_len, total)
        t0 = time.perf_counter()
        if synthetic_context:
            DR.normal_(state.cache.storage.view(-1), 21, 77, 1.0)
            state.position.fill_(prompt_len)
            state.token.copy_(prompt[-batch:].view(batch, 1))
            first = state.token.clone()
            log(f"{shape} {weight_format}: synthetic {prompt_len}-slot KV cache")
        else:
            # First call: warm-up and capture of the prefill graph; second: a replay.
            prefill(model, state, prompt.view(1, -1))
            torch.cuda.synchronize()
            capture_s = time.perf_counter() - t0
            t0 = time.perf_counter()
            first = prefill(model, state, prompt.view(1, -1)).clone()
            torch.cuda.synchronize()
            log(f"{shape}: prefill of {prompt_len} tokens {time.perf_counter() - t0:.3f}s "
                f"(first call with warm-up and graph capture {capture_s:.2f}s)")
        prefill_s = time.perf_counter() - t0
        for _ in range(warmup):
            state.graph.replay()
        # Time exactly `steps` decode steps from the state right after prefill.
        state.position.fill_(prompt_len)
        state.token.copy_(first)
        torch.cuda.synchronize()
        start = time.perf_counter()
        for i in range(steps):
            state.graph.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - start
        # Token ids of the timed run (one more pass, copying each token out).
        state.position.fill_(prompt_len)
        state.token.copy_(first)
        tokens = torch.empty((recorded, batch), dtype=torch.int64, device=model.device)
        for i in range(recorded):
            state.graph.replay()
            tokens[i].copy_(state.token[:, 0])
        torch.cuda.synchronize()
    mean_ctx = prompt_len + (steps - 1) / 2.0
    # Bytes per step: every weight once, each sequence's KV; per token at batch one.
    bytes_per_token = (model.decode_weight_bytes() + batch * kv_bytes_per_token(cfg, mean_ctx)) / batch
    tok_s = batch * steps / elapsed
    toks = tokens.cpu()
    return dict(model=model, cfg=cfg, prompt=prompt.cpu().tolist(), first=int(first[0, 0]),
                prefill_s=prefill_s,
                tokens=(toks[:, 0] if batch == 1 else toks).tolist(), elapsed=elapsed, tok_s=tok_s,
                ms_per_step=1e3 * elapsed / steps, bytes_per_token=bytes_per_token,
                decode_frac=bytes_per_token * tok_s / (HBM_PEAK_GBS * 1e9))


def run_batched(shape, ctx, steps, batches, log):
    """Batched greedy decode (B sequences per captured step, synthetic KV at
    context `ctx`): aggregate tok/s per batch size, one model for all."""
    model = Qwen3Model.random(shape_config(shape))
    out = {"workload": f"{shape} bf16 batched greedy decode, {steps} steps at context {ctx} "
                       "(synthetic N(0,1) KV), one captured HIP graph per step: multi-row MFMA "
                       "projections and per-sequence attention", "by_batch": {}}
    for b in batches:
        r = run_decode(shape, ctx, steps, 2, log, synthetic_context=True, batch=b, model=model)
        out["by_batch"][str(b)] = {"tok_s": round(r["tok_s"], 1),
                                   "ms_per_step": round(r["ms_per_step"], 4),
                                   "per_sequence_tok_s": round(r["tok_s"] / b, 1)}
        log(f"{shape} batch {b}: {r['tok_s']:.1f} tok/s aggregate, {r['ms_per_step']:.3f} ms/step")
        del r
        torch.cuda.empty_cache()
    return out


def graph_ms(graph, reps=20):
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps


def run_draft_speculation(ctx, steps, k, log):
    """4B target + 0.6B draft at context `ctx` over synthetic KV caches."""
    from hackthenorth_amd.draft import DraftSpeculator
    target = Qwen3Model.random(shape_config("qwen3-4b"))
    draft = Qwen3Model.random(shape_config("qwen3-0.6b"))
    spec = DraftSpeculator(target, draft, ctx, steps + 1, draft_tokens=k)
    prompt = DR.randint(ctx, target.config.vocab_size, PROMPT_SEED, PROMPT_STREAM)
    first = int(prompt[-1])
    with torch.inference_mode():
        for st in (spec.target_state, spec.draft_state):
            DR.normal_(st.cache.storage.view(-1), 21, 78, 1.0)
        ts, ds = spec.target_state, spec.draft_state
        # Component times at this context.
        ts.position.fill_(ctx)
        verify_ms = graph_ms(ts.verify_graph)
        ts.position.fill_(ctx)
        step_ms = graph_ms(ts.graph)
        ds.position.fill_(ctx)
        draft_ms = graph_ms(spec.draft_graph)
        list(spec.continue_from(first, ctx, 8))  # warm-up
        spec.reset_stats()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        tokens = [t[0] for t in spec.continue_from(first, ctx, steps)]
        elapsed = time.perf_counter() - t0
    alpha = spec.acceptance
    cycle_ms = 1e3 * elapsed / max(spec.cycles, 1)

    def projected(a):  # tokens per cycle at per-token acceptance a, measured cycle time
        per_cycle = (1 - a ** (k + 1)) / (1 - a) if a < 1 else k + 1
        return round(per_cycle / (cycle_ms / 1e3), 1)

    log(f"speculation 4b+0.6b k={k}: {steps / elapsed:.1f} tok/s, acceptance {alpha:.3f}, "
        f"verify {verify_ms:.3f} ms, target step {step_ms:.3f} ms, draft k steps {draft_ms:.3f} ms")
    return {"workload": f"Qwen3-4B-shape target + Qwen3-0.6B-shape draft (random bf16), k={k} "
                        f"draft tokens, {k + 1}-row verify pass, context {ctx} (synthetic KV), "
                        f"{steps} tokens",
            "tok_s": round(steps / elapsed, 2), "acceptance": round(alpha, 4),
            "cycles": spec.cycles, "tokens_per_cycle": round(steps / max(spec.cycles, 1), 3),
            "cycle_ms": round(cycle_ms, 4), "verify_pass_ms": round(verify_ms, 4),
            "target_step_ms": round(step_ms, 4), "draft_k_steps_ms": round(draft_ms, 4),
            "verify_over_step": round(verify_ms / step_ms, 3),
            "target_only_tok_s": round(1e3 / step_ms, 1),
            "projected_tok_s_at_acceptance": {str(a): projected(a) for a in (0.5, 0.7, 0.9)},
            "first_tokens": tokens[:8]}


def graph_launch_us(calls, device, replays=1):
    """Average duration of one launch of `calls` (callables, each one kernel
    launch sequence) captured back to back in a graph, timed with HIP events
    recorded on the capturing stream around the replay."""
    stream = torch.cuda.Stream(device=device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        for fn in calls[:4]:
            fn()
    torch.cuda.current_stream(device).wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.graph(graph, stream=stream):
        for fn in calls:
            fn()
    with torch.cuda.stream(stream):
        graph.replay()
        stream.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1e3 / (replays * len(calls))


def dominant_kernel(model, rounds=4):
    """Fused RMSNorm + gate/up GEMV + SwiGLU, one launch per layer, rotating
    through all layers' weights `rounds` times, back to back in a graph."""
    cfg = model.config
    layers = model.layers
    x = DR.normal_(torch.empty((1, 1, cfg.hidden_size), dtype=torch.bfloat16,
                               device=model.device), 3, 99, 1.0)
    gain = layers[0].post_attention_layernorm.weight
    calls = [(lambda w=layers[i % len(layers)].gate_up_weight:
              P.norm_projection(x, gain, w, 1e-6, swiglu=True))
             for i in range(rounds * len(layers))]
    avg_us = graph_launch_us(calls, model.device)
    k, n2 = cfg.hidden_size, 2 * cfg.intermediate_size
    algorithmic = n2 * k * 2 + k * 2 * 2 + cfg.intermediate_size * 2  # W + x + gain + y
    return dict(name="gemv_vec<norm, swiglu> (RMSNorm + gate/up GEMV + SwiGLU)",
                instance="void htn::gemv_vec<1, 2, 8, true, 2, 0>(htn::GemvArgs)",
                avg_us=avg_us, bytes=algorithmic, achieved=algorithmic / avg_us / 1e3,
                launches=len(calls), weights_rotated_bytes=len(layers) * n2 * k * 2)


def attention_kernel(model, ctx, rounds=4):
    """The decode step's attention launch (QK-norm + RoPE + KV append +
    split-KV GQA attention + merge, with the O-weight prefetch of the step) at
    position `ctx`, one launch per layer over every layer's cache, back to back
    in a graph. Algorithmic bytes: the K/V rows of slots 0..ctx, the packed
    q/k/v row in, the attention row out, the RoPE row and the two gains."""
    from hackthenorth_amd.kernels.attention import prologue_attention
    cfg = model.config
    c = cfg
    cap = ctx + 1
    dev = model.device
    cache = D.KVCache(model, 1, cap)
    DR.normal_(cache.storage.view(-1), 21, 79, 1.0)
    rotary = D.RotaryTable(model, cap)
    position = torch.tensor([ctx], dtype=torch.int64, device=dev)
    rope = rotary.step_row(position)
    q_width, k_width, _ = c.widths
    packed = DR.normal_(torch.empty((1, 1, sum(c.widths)), dtype=torch.bfloat16, device=dev),
                        5, 98, 1.0)
    groups = c.num_attention_heads // c.num_key_value_heads
    layers = model.layers
    calls = [(lambda i=i % len(layers): prologue_attention(
        packed, layers[i].q_norm, layers[i].k_norm, rope[0], rope[1], cache.keys[i],
        cache.values[i], position, c.num_key_value_heads, groups, q_width, q_width + k_width,
        next_weight=layers[i].o_weight)) for i in range(rounds * len(layers))]
    avg_us = graph_launch_us(calls, dev)
    kv = 2 * c.num_key_value_heads * (ctx + 1) * c.head_dim * 2
    io = sum(c.widths) * 2 + q_width * 2 + 2 * c.head_dim * 2 + 2 * c.head_dim * 2
    algorithmic = kv + io
    del cache
    return dict(name="prologue attention (QK-norm + RoPE + KV append + split-KV GQA + merge)",
                avg_us=avg_us, bytes=algorithmic, achieved=algorithmic / avg_us / 1e3,
                context=ctx, launches=len(calls))


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak


def prefill_kernels(model, rows=2048, layers=8):
    """The batched prefill's matrix-core work at `rows` prompt tokens: each
    projection as the prefill runs it (the plain product through hipBLASLt,
    then the row-wise epilogue launch: none for QKV, SwiGLU for gate/up, the
    residual add with the next RMSNorm for O and down) and the causal
    attention, launched over `layers` layers' weights back to back in a graph,
    timed with HIP events. Work per projection: 2 M N K flops (N: weight rows,
    gate and up both counted), causal attention 4 Hq D T (T + 1) / 2."""
    from hackthenorth_amd.kernels import rows as RW
    from hackthenorth_amd.kernels.attention import grouped_attention
    c = model.config
    dev = model.device
    h = c.hidden_size
    x = DR.normal_(torch.empty((rows, h), dtype=torch.bfloat16, device=dev), 5, 90, 1.0)
    res = DR.normal_(torch.empty((rows, h), dtype=torch.bfloat16, device=dev), 5, 91, 1.0)
    q_width = c.num_attention_heads * c.head_dim
    inter = c.intermediate_size
    a = DR.normal_(torch.empty((rows, q_width), dtype=torch.bfloat16, device=dev), 5, 92, 1.0)
    m = DR.normal_(torch.empty((rows, inter), dtype=torch.bfloat16, device=dev), 5, 93, 1.0)
    ls = model.layers[:layers]
    out = {}
    for name, fn, n, k in (
            ("qkv", lambda l: RW.projection_rows(x, l.qkv_weight), sum(c.widths), h),
            ("o_residual", lambda l: RW.residual_norm_rows(
                a, l.o_weight, res, l.post_attention_layernorm.weight, 1e-6), h, q_width),
            ("gate_up_swiglu", lambda l: RW.swiglu_rows(x, l.gate_up_weight), 2 * inter, h),
            ("down_residual", lambda l: RW.residual_norm_rows(
                m, l.down_weight, res, l.input_layernorm.weight, 1e-6), h, inter)):
        us = graph_launch_us([lambda l=l: fn(l) for l in ls], dev)
        tflops = 2.0 * rows * n * k / us / 1e6
        out[name] = {"us": round(us, 2), "tflops": round(tflops, 1),
                     "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "n": n, "k": k}
    cache = D.KVCache(model, 1, rows)
    DR.normal_(cache.storage.view(-1), 21, 94, 1.0)
    q = DR.normal_(torch.empty((1, c.num_attention_heads, rows, c.head_dim), dtype=torch.bfloat16,
                               device=dev), 5, 95, 1.0)
    pos = torch.arange(rows, device=dev)
    o = torch.empty((1, rows, c.num_attention_heads, c.head_dim), dtype=torch.bfloat16, device=dev)
    us = graph_launch_us([lambda i=i: grouped_attention(q, cache.keys[i], cache.values[i], pos,
                                                        out=o.transpose(1, 2))
                          for i in range(layers)], dev)
    tflops = 4.0 * c.num_attention_heads * c.head_dim * rows * (rows + 1) / 2 / us / 1e6
    out["attention_prefill"] = {"us": round(us, 2), "tflops": round(tflops, 1),
                                "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}
    del cache, x, res, a, m, q, o
    return {"rows": rows, "peak_tflops": MFMA_BF16_PEAK_TFLOPS, **out}


def prefill_kernels_no_grad(model, rows=2048):
    with torch.inference_mode():
        return prefill_kernels(model, rows)


def copy_peak(nbytes=2 << 30, reps=5):
    """Device-to-device copy bandwidth (bytes read + written per second, GB/s)."""
    src = DR.normal_(torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda"), 9, 9, 1.0)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    end.synchronize()
    sec = start.elapsed_time(end) / 1e3 / reps
    del src, dst
    return 2 * nbytes / sec / 1e9


def read_peak(nbytes=2 << 30, reps=5):
    """Streaming-read bandwidth (htn_stream_read over nbytes, GB/s): the
    practical ceiling of read-dominated kernels such as the GEMVs."""
    src = DR.normal_(torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda"), 9, 9, 1.0)
    out = torch.empty(int(_lib.load().htn_stream_read_blocks()), dtype=torch.int32, device="cuda")
    st = _lib.stream()
    _lib.call("htn_stream_read", _lib.ptr(src), nbytes, _lib.ptr(out), st)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        _lib.call("htn_stream_read", _lib.ptr(src), nbytes, _lib.ptr(out), st)
    end.record()
    end.synchronize()
    sec = start.elapsed_time(end) / 1e3 / reps
    del src, out
    return nbytes / sec / 1e9


def per_op_microbench(reps=10, latency_launches=200):
    """The row-wise fused ops at Qwen3-0.6B widths (bf16 activations N(0,1)):
    bandwidth over 32768 rows (algorithmic bytes / average launch time; the
    inputs are re-read every repetition, and 0.3-0.6 GB working sets exceed the
    256 MB Infinity Cache), and the batch-one latency of one row (the decode
    step's case) as the average of `latency_launches` back-to-back launches in
    a graph."""
    from hackthenorth_amd.kernels import embed as E
    from hackthenorth_amd.kernels import fused as F
    from hackthenorth_amd.kernels import rmsnorm as N
    from hackthenorth_amd.model import Norm
    rows, H, I, Hq, Hkv, Dh, V = 32768, 1024, 3072, 16, 8, 128, 151936
    dev = torch.device("cuda")

    def randn(shape, stream):
        t = torch.empty(shape, dtype=torch.bfloat16, device=dev)
        return DR.normal_(t, 11, stream, 1.0)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / 1e3 / reps

    def one_row_us(fn):
        return graph_launch_us([fn] * latency_launches, dev)

    out = {}
    x, r, g = randn((rows, H), 1), randn((rows, H), 2), randn((H,), 3)
    t = timed(lambda: N.add_rms_norm(x, r, g, 1e-6))
    t1 = one_row_us(lambda: N.add_rms_norm(x[:1], r[:1], g, 1e-6))
    out["add_rms_norm"] = (rows * H * 2 * 4 + H * 2, t, f"[{rows}, {H}]", t1)
    del x, r
    gate, up = randn((rows, I), 4), randn((rows, I), 5)
    t = timed(lambda: F.swiglu(gate, up))
    t1 = one_row_us(lambda: F.swiglu(gate[:1], up[:1]))
    out["swiglu"] = (rows * I * 2 * 3, t, f"[{rows}, {I}]", t1)
    del gate, up
    packed = randn((1, rows, (Hq + 2 * Hkv) * Dh), 6)
    q, k, v = (u.view(1, rows, -1, Dh) for u in packed.split((Hq * Dh, Hkv * Dh, Hkv * Dh), -1))
    qn, kn = Norm(randn((Dh,), 7), 1e-6), Norm(randn((Dh,), 8), 1e-6)
    cos, sin = (u.to(dev)[None] for u in D.rope_tables(shape_config("qwen3-0.6b"), rows))
    keys = torch.zeros((1, Hkv, rows, Dh), dtype=torch.bfloat16, device=dev)
    values = torch.zeros_like(keys)
    positions = torch.arange(rows, device=dev)
    t = timed(lambda: F.norm_rope_cache(q, k, v, qn, kn, cos, sin, keys, values, positions))
    t1 = one_row_us(lambda: F.norm_rope_cache(q[:, :1], k[:, :1], v[:, :1], qn, kn, cos[:, :1],
                                              sin[:, :1], keys, values, positions[:1]))
    per_token = (Hq + 2 * Hkv) * Dh * 2 * 2 + 2 * Dh * 2 + 8
    out["qk_norm_rope_kv_append"] = (rows * per_token, t,
                                     f"{rows} tokens x ({Hq} q + {Hkv} kv heads)", t1)
    del packed, keys, values
    table = randn((V, H), 9)
    ids = DR.randint(rows, V, 1, 8, device=dev)
    t = timed(lambda: E.embed_gather(ids, table))
    t1 = one_row_us(lambda: E.embed_gather(ids[:1], table))
    out["embed_gather"] = (rows * (H * 2 * 2 + 8), t, f"{rows} ids of [{V}, {H}]", t1)
    return {name: {"shape": shape, "bytes": b, "us": round(sec * 1e6, 2),
                   "GBs": round(b / sec / 1e9, 1),
                   "frac_of_peak": round(b / sec / 1e9 / HBM_PEAK_GBS, 4),
                   "one_row_us": round(t1, 3)}
            for name, (b, sec, shape, t1) in out.items()}


def oracle_weights(model):
    """The device model's weights as the oracle's CPU dictionary (bit-identical
    to oracle.qwen3.generate_weights for the same seed, which the GPU tests
    check; copying them is far faster than regenerating 8B weights in numpy)."""
    w = {"embed": model.embed_weight.cpu(), "norm": model.norm.weight.cpu()}
    w["lm_head"] = (w["embed"] if model.lm_head_weight is model.embed_weight
                    else model.lm_head_weight.cpu())
    for i, layer in enumerate(model.layers):
        for kind, t in layer.tensors().items():
            w[f"{i}.{kind}"] = t.cpu()
        w[f"{i}.ln1"] = layer.input_layernorm.weight.cpu()
        w[f"{i}.ln2"] = layer.post_attention_layernorm.weight.cpu()
        w[f"{i}.q_norm"] = layer.q_norm.weight.cpu()
        w[f"{i}.k_norm"] = layer.k_norm.weight.cpu()
    return w


def cpu_threads():
    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    return threads


def cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            return next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        return ""


def explain_record(record, oracle, prompt, tokens, primary):
    """Explain the record's differing steps (if any) against the oracle's other
    evaluation orders of the same sequence: `primary` names the order the
    record was made in ("stepwise": prompt pass then one token at a time;
    "batched": one causal pass over prompt + tokens); the others are made
    only when a step needs them."""
    from oracle import parity as OP
    from oracle import qwen3 as Q
    if record.pending():
        o64 = Q.Oracle(oracle.shape, oracle.weights, oracle.capacity, acc=torch.float64)
        makers = {"float64": lambda: o64.teacher_forced_logits(prompt, tokens)}
        if primary == "stepwise":
            makers["batched"] = lambda: oracle.teacher_forced_logits(prompt, tokens)
        else:
            makers["stepwise"] = lambda: oracle.stepwise_logits(prompt, tokens)
        record.explain(OP.Orders(**makers).callables())
    return record.summary()


def cpu_baseline(model, shape_name, prompt, gpu_tokens, decode_steps=32):
    """The CPU oracle on this host's cores over a bounded sample of the
    workload: one batched prefill of the whole prompt, then `decode_steps`
    decode steps fed the GPU's own tokens (teacher forcing), which also gives
    the parity record of those tokens against the oracle's logits (differing
    steps explained against the oracle's other evaluation orders)."""
    from oracle import parity as OP
    from oracle import qwen3 as Q
    cpu_threads()
    shape = Q.SHAPES[shape_name]
    t0 = time.perf_counter()
    weights = oracle_weights(model)
    tokens = gpu_tokens[:decode_steps + 1]
    oracle = Q.Oracle(shape, weights, capacity=len(prompt) + decode_steps + 1)
    setup_s = time.perf_counter() - t0
    timer = {}
    record = OP.teacher_forced(oracle, prompt, tokens, OP.NEAR_TIE, timer=timer)
    summary = explain_record(record, oracle, prompt, tokens, "stepwise")
    del oracle, weights
    return {"value": decode_steps / timer["decode_s"], "unit": "tok/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"CPU oracle (torch eager, fp32 accumulation with the reference's bf16 "
                      f"rounding boundaries) on the same {shape_name} workload and weights: one "
                      f"batched prefill of the {len(prompt)}-token prompt "
                      f"({timer['prefill_s']:.1f} s) then {decode_steps} decode steps at context "
                      f"{len(prompt)}-{len(prompt) + decode_steps - 1} fed the GPU's tokens; "
                      f"value = tok/s over those decode steps",
            "prefill_s": round(timer["prefill_s"], 3),
            "prefill_tok_s": round(len(prompt) / timer["prefill_s"], 1),
            "decode_s": round(timer["decode_s"], 3), "setup_s": round(setup_s, 1),
            "teacher_forced": summary,
            "cpu_model": cpu_model_name(), "os_cpu_count": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0))}


def cfg1_cpu_and_gpu(log, steps=64, prompt_len=32):
    """The Qwen3-0.6B shape with a 32-token prompt and 64 greedy steps: the CPU
    oracle's whole free-running decode timed on this host (prefill and
    per-token decode reported apart, after one warm-up step), its ids against
    the committed golden ids, and the GPU's captured decode of the same
    request with its teacher-forced parity record."""
    from oracle import parity as OP
    from oracle import qwen3 as Q
    threads = cpu_threads()
    shape = Q.SHAPES["0.6b"]
    model = Qwen3Model.random(shape_config("qwen3-0.6b"))
    prompt = Q.prompt_ids(prompt_len, shape.vocab)
    with torch.inference_mode():
        state = D.DecodeState(model, 1, prompt_len, steps)
        first = prefill(model, state, torch.tensor([prompt], device="cuda"))[:, 0].tolist()
        gpu = [t[0] for t in D.stream_decode(state, first, steps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        first = prefill(model, state, torch.tensor([prompt], device="cuda"))[:, 0].tolist()
        again = [t[0] for t in D.stream_decode(state, first, steps)]
        gpu_s = time.perf_counter() - t0
    weights = oracle_weights(model)
    del state, model
    torch.cuda.empty_cache()
    oracle = Q.Oracle(shape, weights, capacity=prompt_len + steps)
    # One warm-up step (a prefill of the prompt and one decode step), then the
    # timed decode: the prompt pass, then 63 single-token steps.
    cache = Q.new_cache(shape, oracle.capacity)
    tok, _, _ = oracle.forward(torch.tensor([prompt]), cache, torch.arange(prompt_len))
    oracle.forward(tok.view(1, 1), cache, torch.tensor([prompt_len]))
    cache = Q.new_cache(shape, oracle.capacity)
    t0 = time.perf_counter()
    tok, _, _ = oracle.forward(torch.tensor([prompt]), cache, torch.arange(prompt_len))
    t1 = time.perf_counter()
    cpu = [int(tok[0, 0])]
    for i in range(1, steps):
        tok, _, _ = oracle.forward(torch.tensor([[cpu[-1]]]), cache,
                                   torch.tensor([prompt_len + i - 1]))
        cpu.append(int(tok[0, 0]))
    t2 = time.perf_counter()
    golden_path = os.path.join(ROOT, "tests", "golden", "qwen3_0.6b_decode.json")
    with open(golden_path) as f:
        fixture = json.load(f)
    golden, golden_gaps = fixture["tokens"], fixture["top2_gap_fp32"]
    logits = oracle.teacher_forced_logits(prompt, gpu)
    record = OP.TokenRecord()
    for i, t in enumerate(gpu):
        record.add(i, logits[i], t)
    summary = explain_record(record, oracle, prompt, gpu, "batched")
    parts = next((i for i, (a, b) in enumerate(zip(cpu, golden)) if a != b), None)
    log(f"cfg1 0.6B CPU oracle: {(steps - 1) / (t2 - t1):.2f} tok/s decode; GPU "
        f"{steps / gpu_s:.1f} tok/s end to end; CPU ids equal to golden "
        f"{sum(a == b for a, b in zip(cpu, golden))}/{steps}")
    return {"workload": f"Qwen3-0.6B-shape bf16 (tied), {prompt_len}-token prompt, {steps} "
                        f"greedy steps (the reference's torch-eager CPU configuration)",
            "cpu": {"decode_tok_s": round((steps - 1) / (t2 - t1), 2),
                    "prefill_s": round(t1 - t0, 3), "decode_s": round(t2 - t1, 3),
                    "cores": threads, "kind": "port",
                    "ids_equal_to_golden": sum(a == b for a, b in zip(cpu, golden)),
                    # The golden ids were written by the same oracle on another
                    # CPU; its BLAS sums in another order, so the free-running
                    # ids may part at a near-tie (the fixture's top-2 gap there).
                    "first_step_off_golden": parts,
                    "golden_top2_gap_there": (round(golden_gaps[parts], 6)
                                              if parts is not None else None),
                    "cpu_model": cpu_model_name()},
            "gpu": {"end_to_end_tok_s": round(steps / gpu_s, 1),
                    "repeat_identical": again == gpu,
                    "ids_equal_to_cpu_oracle": sum(a == b for a, b in zip(gpu, cpu)),
                    "teacher_forced": summary}}


def run_prompt_lookup(log, shape="qwen3-8b", prompt_len=512, steps=128, seed_len=64):
    """Batch-one prompt-lookup speculation (the reference's production mode,
    dryft/engine/engine.py:224-249) through Engine.generate, beside the same
    request without speculation. The prompt is the model's own text: a
    64-token random seed and its greedy continuation (plain decode) up to
    `prompt_len` tokens, so the lookup proposes from n-grams the model itself
    produced (a random-init model's greedy text turns repetitive, as language
    models' often does). Reported: end-to-end tok/s of each mode (prefill
    included, after a warm-up request that captures the graphs), the
    verifier's passes, proposals and acceptance, and whether both modes emit
    the same ids."""
    import tempfile
    from hackthenorth_amd.engine import Engine
    from hackthenorth_amd.model import write_random_model_dir
    vocab = shape_config(shape).vocab_size
    seed = DR.randint(seed_len, vocab, PROMPT_SEED, PROMPT_STREAM + 1).cpu().tolist()
    out = {"workload": f"{shape} bf16, Engine.generate of {steps} tokens after a "
                       f"{prompt_len}-token prompt (a {seed_len}-token random seed and the "
                       "model's own greedy continuation), prompt-lookup speculation (draft "
                       "width 7, 8-row verify graph) against plain decode"}
    with tempfile.TemporaryDirectory() as tmp:
        path = write_random_model_dir(os.path.join(tmp, "m"), shape, seed=0)
        ids = {}
        for mode in ("plain", "prompt_lookup"):
            engine = Engine(path, speculative=mode == "prompt_lookup")
            if mode == "plain":
                prompt = seed + [t[0] for t in engine.generate([seed], prompt_len - seed_len)]
                out["prompt_distinct_ids"] = len(set(prompt))
            list(engine.generate([prompt], steps))  # warm-up: captures
            engine.reset_stats()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            got = [t[0] for t in engine.generate([prompt], steps)]
            elapsed = time.perf_counter() - t0
            ids[mode] = got
            stats = dict(engine.stats)
            if stats["proposed"]:
                stats["acceptance"] = round(stats["accepted"] / stats["proposed"], 4)
            out[mode] = {"tok_s": round(steps / elapsed, 2), "seconds": round(elapsed, 4),
                         **stats}
            del engine
            torch.cuda.empty_cache()
    out["speedup"] = round(out["prompt_lookup"]["tok_s"] / out["plain"]["tok_s"], 4)
    out["ids_identical"] = sum(a == b for a, b in zip(ids["plain"], ids["prompt_lookup"]))
    log(f"prompt lookup {shape}: {out['prompt_lookup']['tok_s']:.1f} vs plain "
        f"{out['plain']['tok_s']:.1f} tok/s ({out['speedup']:.3f}x), "
        f"{out['prompt_lookup']['verify_passes']} verify passes")
    return out


def pmc_pass(shape="qwen3-0.6b", weight_format="bf16"):
    """Short, graph-free workload for rocprofv3 --pmc passes (counter collection
    is per dispatch, so every kernel is launched eagerly): 8 decode steps of the
    shape's workload (0.6B at context 512, 8B at context 2048 over a synthetic
    cache; the 8B 8-bit formats at context 8192, as their bench lines), one
    launch of the dominant kernel per layer over the layers' weights, and a
    256 MiB device copy (reads and writes exactly 256 MiB) that calibrates the
    byte counters."""
    cfg = shape_config(shape, weight_format=weight_format)
    model = Qwen3Model.random(cfg)
    ctx = 512 if shape == "qwen3-0.6b" else (2048 if weight_format == "bf16" else 8192)
    cap = ctx + 8
    with torch.inference_mode():
        cache = D.KVCache(model, 1, cap)
        if ctx > 512:
            DR.normal_(cache.storage.view(-1), 21, 77, 1.0)
        rotary = D.RotaryTable(model, cap)
        token = torch.zeros((1, 1), dtype=torch.int64, device=model.device)
        for i in range(8):
            pos = torch.tensor([ctx + i], dtype=torch.int64, device=model.device)
            token = D.forward(model, token, cache, pos, rotary=rotary)
        x = torch.empty((1, 1, cfg.hidden_size), dtype=torch.bfloat16, device=model.device)
        DR.normal_(x, 3, 99, 1.0)
        gain = model.layers[0].post_attention_layernorm.weight
        for layer in model.layers:
            P.norm_projection(x, gain, layer.gate_up_weight, 1e-6, swiglu=True)
        src = torch.empty(128 << 20, dtype=torch.bfloat16, device="cuda")
        dst = torch.empty_like(src)
        DR.normal_(src, 9, 9, 1.0)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
    k, n2 = cfg.hidden_size, 2 * cfg.intermediate_size
    print(json.dumps({"pmc_pass": True, "weight_format": weight_format, "context": ctx,
                      "calibration_copy_bytes": src.numel() * 2,
                      "dominant_kernel_bytes": n2 * k * (2 if weight_format == "bf16" else 1)
                      + k * 4 + cfg.intermediate_size * 2}),
          flush=True)


def pmc_pass_rows(workload):
    """Graph-free multi-row workloads for the same counter passes: "prefill"
    runs the 8B 2048-token prompt's batched forward twice (the first call of
    each library GEMM shape picks its algorithm; the second pass is the one
    to read), "rows" eight batched decode steps of 16 sequences at context
    512 (the multi-row MFMA projections and the per-sequence attention),
    "verify" eight 5-row verify passes of the 4B shape at context 4096 (the
    speculative target's pass); all end with the 256 MiB calibration copy."""
    cfg = shape_config("qwen3-4b" if workload == "verify" else "qwen3-8b")
    model = Qwen3Model.random(cfg)
    dev = model.device
    with torch.inference_mode():
        if workload == "prefill":
            rows, batch = 2048, 1
            cache = D.KVCache(model, 1, rows + 8)
            rotary = D.RotaryTable(model, rows + 8)
            ids = DR.randint(rows, cfg.vocab_size, 5, 1, device=dev).view(1, rows)
            pos = torch.arange(rows, dtype=torch.int64, device=dev)
            for _ in range(2):
                D.forward(model, ids, cache, pos, rotary=rotary)
        elif workload == "verify":
            rows, batch, ctx = 5, 1, 4096
            cache = D.KVCache(model, 1, ctx + 48)
            DR.normal_(cache.storage.view(-1), 21, 79, 1.0)
            rotary = D.RotaryTable(model, ctx + 48)
            ids = torch.zeros((1, rows), dtype=torch.int64, device=dev)
            for i in range(8):
                pos = torch.arange(ctx + 5 * i, ctx + 5 * i + rows, dtype=torch.int64, device=dev)
                D.forward(model, ids, cache, pos, last_only=False, rotary=rotary)
        else:
            rows, batch, ctx = 16, 16, 512
            cache = D.KVCache(model, batch, ctx + 8)
            DR.normal_(cache.storage.view(-1), 21, 78, 1.0)
            rotary = D.RotaryTable(model, ctx + 8)
            ids = torch.zeros((batch, 1), dtype=torch.int64, device=dev)
            for i in range(8):
                pos = torch.full((1,), ctx + i, dtype=torch.int64, device=dev)
                ids = D.forward(model, ids, cache, pos, rotary=rotary)
        src = torch.empty(128 << 20, dtype=torch.bfloat16, device="cuda")
        dst = torch.empty_like(src)
        DR.normal_(src, 9, 9, 1.0)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps({"pmc_pass": True, "workload": workload, "rows": rows, "batch": batch,
                      "calibration_copy_bytes": src.numel() * 2}), flush=True)


def decode_line(res):
    """The common keys of a decode result."""
    return {"tok_s": round(res["tok_s"], 2), "ms_per_step": round(res["ms_per_step"], 4),
            "bytes_per_token": res["bytes_per_token"],
            "roofline_frac": round(res["decode_frac"], 4),
            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / res["bytes_per_token"], 1)}


def section_0p6b(args, log):
    """The Qwen3-0.6B decode (prompt 512, 64 steps) with its dominant kernel:
    the decode attention (28 x ~7.7 us per step against 28 x ~5 us for the
    gate/up GEMV in the step's kernel trace)."""
    r = run_decode("qwen3-0.6b", 512, 64, args.warmup, log)
    att = attention_kernel(r["model"], 512)
    log(f"qwen3-0.6b: {r['tok_s']:.1f} tok/s; attention {att['avg_us']:.2f} us/launch")
    parity = None
    if not args.no_cpu_baseline:
        # Every one of the 64 tokens (the first from the prefill) teacher-forced.
        from oracle import parity as OP
        from oracle import qwen3 as Q
        cpu_threads()
        oracle = Q.Oracle(Q.SHAPES["0.6b"], oracle_weights(r["model"]), 512 + 64)
        tokens = [r["first"]] + r["tokens"][:63]
        logits = oracle.teacher_forced_logits(r["prompt"], tokens)
        record = OP.TokenRecord()
        for i, t in enumerate(tokens):
            record.add(i, logits[i], t)
        parity = explain_record(record, oracle, r["prompt"], tokens, "batched")
        del oracle
    out = {"workload": "Qwen3-0.6B-shape bf16 (tied), prompt 512, 64 greedy steps "
                       "(context 512-575)", **decode_line(r),
           "dominant_kernel": {"kernel": att["name"], "avg_launch_us": round(att["avg_us"], 3),
                               "bytes_per_launch": att["bytes"], "context": att["context"],
                               "achieved_GBs": round(att["achieved"], 1),
                               "frac": round(att["achieved"] / HBM_PEAK_GBS, 4)},
           "first_tokens": [r["first"]] + r["tokens"][:15]}
    if parity is not None:
        out["teacher_forced"] = parity
    del r
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--headline-only", action="store_true",
                    help="the 8B headline line only (no secondary sections, no CPU baseline)")
    ap.add_argument("--cpu-decode-steps", type=int, default=32)
    ap.add_argument("--secondary", default="all",
                    help="comma-separated keys of the secondary sections to run after the "
                         "headline (default all; 'none' for none)")
    ap.add_argument("--quiet", action="store_true")
    ap.add_argument("--pmc-shape", default="qwen3-8b", choices=("qwen3-0.6b", "qwen3-8b"),
                    help="model shape of the --pmc-pass workload")
    ap.add_argument("--prefill-tiles", action="store_true",
                    help="prompt projections on this library's tiled GEMM instead of hipBLASLt")
    ap.add_argument("--pmc-format", default="bf16", choices=("bf16", "int8", "fp8_e4m3"),
                    help="projection weight format of the --pmc-pass workload (8B only)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="short workload for rocprofv3 counter passes (no JSON bench line)")
    ap.add_argument("--pmc-workload", default="decode",
                    choices=("decode", "prefill", "rows", "verify"),
                    help="workload of --pmc-pass: decode steps (default), the 8B 2048-token "
                         "prefill, 8B batched decode at 16 rows, or the 4B 5-row verify pass")
    ap.add_argument("--section", default="all",
                    choices=("all", "qwen3-0.6b", "qwen3-8b-int8", "qwen3-8b-fp8", "speculative",
                             "batched", "per-op", "prefill", "cfg1", "prompt-lookup"),
                    help="run one secondary workload alone and print its JSON (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the batch-one decode path on exactly one GPU; "
              "multi-GPU runs are not part of this build", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        sys.exit(2)

    if args.prefill_tiles:
        from hackthenorth_amd.kernels import rows as RW
        RW.LIBRARY = False
    if args.pmc_pass:
        if args.pmc_workload == "decode":
            pmc_pass(args.pmc_shape, args.pmc_format)
        else:
            pmc_pass_rows(args.pmc_workload)
        return

    def log(msg):
        if not args.quiet:
            print(msg, file=sys.stderr, flush=True)

    if args.section != "all":
        if args.section == "qwen3-0.6b":
            out = section_0p6b(args, log)
        elif args.section == "speculative":
            out = run_draft_speculation(4096, 128, 4, log)
        elif args.section == "batched":
            out = run_batched("qwen3-8b", 512, 32, (1, 4, 16), log)
        elif args.section == "per-op":
            out = {"per_op": per_op_microbench()}
        elif args.section == "cfg1":
            out = cfg1_cpu_and_gpu(log)
        elif args.section == "prompt-lookup":
            out = {"qwen3_8b": run_prompt_lookup(log),
                   "qwen3_0.6b": run_prompt_lookup(log, shape="qwen3-0.6b")}
        elif args.section == "prefill":
            model = Qwen3Model.random(shape_config("qwen3-8b"))
            with torch.inference_mode():
                out = {"prefill_kernels": prefill_kernels(model, args.prompt)}
        else:
            fmt = "int8" if args.section.endswith("int8") else "fp8_e4m3"
            r = run_decode("qwen3-8b", 8192, 128, args.warmup, log, weight_format=fmt,
                           synthetic_context=True)
            out = decode_line(r)
        print(json.dumps({"section": args.section, **out}), flush=True)
        return

    # Headline: Qwen3-8B shape, bf16, prompt 2048, K timed greedy steps.
    res = run_decode("qwen3-8b", args.prompt, args.steps, args.warmup, log,
                     record_steps=0 if args.no_cpu_baseline else args.cpu_decode_steps)
    log(f"qwen3-8b: {res['tok_s']:.1f} tok/s, {res['ms_per_step']:.3f} ms/step "
        f"({100 * res['decode_frac']:.1f}% of the bytes roofline)")
    dom = dominant_kernel(res["model"])
    log(f"dominant kernel: {dom['avg_us']:.2f} us/launch, {dom['achieved']:.0f} GB/s")
    copy_gbs = copy_peak()
    read_gbs = read_peak()
    log(f"device copy: {copy_gbs:.0f} GB/s (read + write), streaming read: {read_gbs:.0f} GB/s")
    trace_us = trace_average_us(dom["instance"])
    line = {
        "metric": METRIC, "value": round(res["tok_s"], 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init N(0,0.02) bf16 weights and uniform prompt ids from the "
                "counter RNG (seed 0 weights, seed 1 prompt)",
        "config": {"workload": f"Qwen3-8B-shape bf16 batch-1 greedy decode (hidden 4096, 36 "
                               f"layers, 32 q / 8 kv heads, FFN 12288, vocab 151936, untied), "
                               f"prompt {args.prompt}, {args.steps} timed steps (context "
                               f"{args.prompt}-{args.prompt + args.steps - 1}), one captured "
                               f"HIP graph per step",
                   "batch": 1, "prompt_tokens": args.prompt, "decode_steps": args.steps},
        "roofline": {"bound": "hbm", "achieved": round(dom["achieved"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["achieved"] / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": dom["name"], "instance": dom["instance"],
                     "avg_launch_us": round(dom["avg_us"], 3),
                     "bytes_per_launch": dom["bytes"], "launches_timed": dom["launches"],
                     "weights_rotated_bytes": dom["weights_rotated_bytes"],
                     "trace_avg_us": trace_us,
                     "trace_frac": (round(dom["bytes"] / trace_us / 1e3 / HBM_PEAK_GBS, 4)
                                    if trace_us else None),
                     "copy_peak_GBs": round(copy_gbs, 1),
                     "frac_of_copy_peak": round(dom["achieved"] / copy_gbs, 4),
                     "read_peak_GBs": round(read_gbs, 1),
                     "frac_of_read_peak": round(dom["achieved"] / read_gbs, 4)},
        "decode_roofline": {"bytes_per_token": res["bytes_per_token"],
                            "achieved_GBs": round(res["bytes_per_token"] * res["tok_s"] / 1e9, 1),
                            "frac": round(res["decode_frac"], 4),
                            "frac_of_copy_peak": round(
                                res["bytes_per_token"] * res["tok_s"] / 1e9 / copy_gbs, 4),
                            "frac_of_read_peak": round(
                                res["bytes_per_token"] * res["tok_s"] / 1e9 / read_gbs, 4),
                            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / res["bytes_per_token"], 1)},
        "prefill_s": round(res["prefill_s"], 3),
        "prefill_tok_s": round(args.prompt / res["prefill_s"], 1),
        "prefill_kernels": prefill_kernels_no_grad(res["model"], args.prompt),
        "first_tokens": [res["first"]] + res["tokens"][:15],
    }
    if not args.no_cpu_baseline and not args.headline_only:
        try:
            line["cpu_baseline"] = cpu_baseline(res["model"], "8b", res["prompt"],
                                                [res["first"]] + res["tokens"],
                                                args.cpu_decode_steps)
            tf = line["cpu_baseline"]["teacher_forced"]
            log(f"cpu baseline: {line['cpu_baseline']['value']:.2f} tok/s decode, prefill "
                f"{line['cpu_baseline']['prefill_s']:.1f} s; teacher-forced "
                f"{tf['identical']}/{tf['checked']} identical, {tf['near_tie']} near-ties, "
                f"{tf['oracle_noise']} oracle noise, {tf['unexplained']} unexplained")
        except Exception as exc:  # report, do not lose the headline line
            line["cpu_baseline"] = {"error": repr(exc)}
    del res["model"]
    torch.cuda.empty_cache()
    if not args.headline_only:
        sections = [("qwen3_0.6b", lambda: section_0p6b(args, log)),
                    ("per_op", per_op_microbench)]
        for fmt in ("int8", "fp8_e4m3"):
            sections.append((f"qwen3_8b_{fmt.split('_')[0]}",
                             lambda fmt=fmt: {"workload": f"Qwen3-8B-shape, weight-only {fmt} "
                                              "projections and LM head, bf16 activations and KV, "
                                              "128 greedy steps at context 8192-8319 (synthetic "
                                              "N(0,1) KV cache)",
                                              **decode_line(run_decode(
                                                  "qwen3-8b", 8192, 128, args.warmup, log,
                                                  weight_format=fmt, synthetic_context=True))}))
        sections.append(("speculative_4b_draft_0.6b",
                         lambda: run_draft_speculation(4096, 128, 4, log)))
        sections.append(("batched_qwen3_8b",
                         lambda: run_batched("qwen3-8b", 512, 32, (4, 16), log)))
        sections.append(("prompt_lookup_qwen3_8b", lambda: run_prompt_lookup(log)))
        sections.append(("prompt_lookup_qwen3_0.6b",
                         lambda: run_prompt_lookup(log, shape="qwen3-0.6b")))
        if not args.no_cpu_baseline:
            sections.append(("cpu_qwen3_0.6b_prompt32", lambda: cfg1_cpu_and_gpu(log)))
        wanted = None if args.secondary == "all" else set(args.secondary.split(","))
        for key, fn in sections:
            if wanted is not None and key not in wanted:
                continue
            try:
                line[key] = fn()
            except Exception as exc:  # report, do not lose the headline line
                line[key] = {"error": repr(exc)}
            torch.cuda.empty_cache()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
