"""Batch-one Qwen3 greedy decode throughput on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-8b]

Default workload: the Qwen3-0.6B shape (hidden 1024, 28 layers, 16 q / 8 kv
heads, head_dim 128, FFN 3072, vocab 151936, tied), random-init bf16
weights N(0, 0.02), a 512-token uniform-random prompt, then K greedy decode
steps (K = 64: context 512 -> 575). A step is one replay of the captured
decode graph; the timed region replays K steps back to back with weights,
KV cache and token/position state already resident in HBM.

Also reported on the same line:
  roofline      the dominant kernel (the fused RMSNorm + gate/up GEMV + SwiGLU,
                one launch per layer), timed alone with HIP events on its stream
                over rotating per-layer weights (28 x 12.6 MB, more than the
                256 MB Infinity Cache), as algorithmic bytes / launch time;
  decode_roofline  bytes per generated token / step time against 8 TB/s;
  cpu_baseline  the CPU oracle (torch eager, this host's cores) on a bounded
                sample of the same workload: batched prompt prefill + 8 greedy
                decode steps, reported as decode tok/s;
  qwen3_8b      the Qwen3-8B shape (untied), prompt 2048, 256 greedy steps;
  qwen3_8b_int8 / qwen3_8b_fp8
                the Qwen3-8B shape with weight-only int8 / fp8-e4m3fn projections
                and LM head (uniform integer weights in [-127, 127], per-row
                scales U(0.001, 0.01)), decoding 128 steps at context 8192 over a
                synthetic KV cache (N(0,1) keys and values in slots 0..8191);
  speculative_4b_draft_0.6b
                Qwen3-4B-shape target with a Qwen3-0.6B-shape draft (both random
                bf16), k = 4 draft tokens verified in one 5-row pass, context 4096
                (synthetic KV caches): tok/s, measured greedy acceptance, and the
                verify pass / draft step / single target step times.
"""
import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from hackthenorth_amd import decode as D  # noqa: E402
from hackthenorth_amd.kernels import projection as P  # noqa: E402
from hackthenorth_amd.kernels import rng as DR  # noqa: E402
from hackthenorth_amd.model import Qwen3Model, shape_config  # noqa: E402

METRIC = "batch-1 decode tok/s at Qwen3 shapes + per-kernel HBM GB/s as % of peak"
# HBM bytes per launch of the dominant kernel, from the committed rocprofv3
# FETCH_SIZE / WRITE_SIZE passes (calibrated against a copy of known size).
PMC_PROFILE = os.path.join(ROOT, "profiles", "gemv_gateup_swiglu_qwen3-0.6b_pmc.txt")
HBM_PEAK_GBS = 8000.0
PROMPT_SEED, PROMPT_STREAM = 1, 7


def measured_traffic():
    try:
        with open(PMC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def kv_bytes_per_token(cfg, ctx):
    """KV read over ctx slots plus the appended slot, all layers (bf16)."""
    per_slot = 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * cfg.head_dim * 2
    return per_slot * (ctx + 1)


def run_decode(shape, prompt_len, steps, warmup, log, weight_format="bf16",
               synthetic_context=False, batch=1, model=None):
    """Greedy decode of `steps` tokens after a prompt of `prompt_len` tokens.

    synthetic_context: instead of prefilling, fill every KV slot with N(0,1)
    values and start decoding at position prompt_len (the step's cost does not
    depend on the cached values; this keeps 8192-token contexts cheap to set up).
    """
    cfg = shape_config(shape, weight_format=weight_format)
    if model is None:
        model = Qwen3Model.random(cfg)
    prompt = DR.randint(prompt_len, cfg.vocab_size, PROMPT_SEED, PROMPT_STREAM)
    total = warmup + steps + 1
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
            first = state.prefill(model, prompt.view(1, -1)).clone()
            torch.cuda.synchronize()
            log(f"{shape}: prefill of {prompt_len} tokens (step by step) "
                f"{time.perf_counter() - t0:.2f}s")
        for _ in range(warmup):
            state.graph.replay()
        # Time exactly `steps` decode steps from the state right after prefill.
        state.position.fill_(prompt_len)
        state.token.copy_(first)
        tokens = torch.empty((steps, batch), dtype=torch.int64, device=model.device)
        torch.cuda.synchronize()
        start = time.perf_counter()
        for i in range(steps):
            state.graph.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - start
        # Token ids of the timed run (one more pass, copying each token out).
        state.position.fill_(prompt_len)
        state.token.copy_(first)
        for i in range(steps):
            state.graph.replay()
            tokens[i].copy_(state.token[:, 0])
        torch.cuda.synchronize()
    mean_ctx = prompt_len + (steps - 1) / 2.0
    # Bytes per step: every weight once, each sequence's KV; per token at batch one.
    bytes_per_token = (model.decode_weight_bytes() + batch * kv_bytes_per_token(cfg, mean_ctx)) / batch
    tok_s = batch * steps / elapsed
    toks = tokens.cpu()
    return dict(model=model, cfg=cfg, prompt=prompt.cpu().tolist(), first=int(first[0, 0]),
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


def dominant_kernel(model, launches=280):
    """Fused norm + gate/up + SwiGLU GEMV over the layers' weights (one launch per
    layer, rotating through all of them), captured in a graph so the launches run
    back to back, timed with HIP events on the capturing stream."""
    cfg = model.config
    layers = model.layers
    x = torch.empty((1, 1, cfg.hidden_size), dtype=torch.bfloat16, device=model.device)
    DR.normal_(x, 3, 99, 1.0)
    gain = layers[0].post_attention_layernorm.weight
    stream = torch.cuda.Stream(device=model.device)
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for layer in layers[:4]:
            P.norm_projection(x, gain, layer.gate_up_weight, 1e-6, swiglu=True)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(launches):
            P.norm_projection(x, gain, layers[i % len(layers)].gate_up_weight, 1e-6, swiglu=True)
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        graph.replay()
        end.record(stream)
    end.synchronize()
    avg_s = start.elapsed_time(end) / 1e3 / launches
    k, n2 = cfg.hidden_size, 2 * cfg.intermediate_size
    algorithmic = n2 * k * 2 + k * 2 * 2 + cfg.intermediate_size * 2  # W + x + gain + y
    achieved = algorithmic / avg_s / 1e9
    return dict(name="gemv_vec<norm, swiglu> (RMSNorm + gate/up GEMV + SwiGLU)",
                avg_us=avg_s * 1e6, bytes=algorithmic, achieved=achieved)


def per_op_microbench(reps=10):
    """Bandwidth of the row-wise fused ops at Qwen3-0.6B widths over 32768 rows
    (bf16 activations N(0,1)): algorithmic bytes / average launch time."""
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

    out = {}
    x, r, g = randn((rows, H), 1), randn((rows, H), 2), randn((H,), 3)
    t = timed(lambda: N.add_rms_norm(x, r, g, 1e-6))
    out["add_rms_norm"] = (rows * H * 2 * 4 + H * 2, t, f"[{rows}, {H}]")
    del x, r
    gate, up = randn((rows, I), 4), randn((rows, I), 5)
    t = timed(lambda: F.swiglu(gate, up))
    out["swiglu"] = (rows * I * 2 * 3, t, f"[{rows}, {I}]")
    del gate, up
    packed = randn((1, rows, (Hq + 2 * Hkv) * Dh), 6)
    q, k, v = (u.view(1, rows, -1, Dh) for u in packed.split((Hq * Dh, Hkv * Dh, Hkv * Dh), -1))
    qn, kn = Norm(randn((Dh,), 7), 1e-6), Norm(randn((Dh,), 8), 1e-6)
    cos, sin = (u.to(dev)[None] for u in D.rope_tables(shape_config("qwen3-0.6b"), rows))
    keys = torch.zeros((1, Hkv, rows, Dh), dtype=torch.bfloat16, device=dev)
    values = torch.zeros_like(keys)
    positions = torch.arange(rows, device=dev)
    t = timed(lambda: F.norm_rope_cache(q, k, v, qn, kn, cos, sin, keys, values, positions))
    per_token = (Hq + 2 * Hkv) * Dh * 2 * 2 + 2 * Dh * 2 + 8
    out["qk_norm_rope_kv_append"] = (rows * per_token, t, f"{rows} tokens x ({Hq} q + {Hkv} kv heads)")
    del packed, keys, values
    table = randn((V, H), 9)
    ids = DR.randint(rows, V, 1, 8, device=dev)
    t = timed(lambda: E.embed_gather(ids, table))
    out["embed_gather"] = (rows * (H * 2 * 2 + 8), t, f"{rows} ids of [{V}, {H}]")
    return {name: {"shape": shape, "bytes": b, "us": round(sec * 1e6, 2),
                   "GBs": round(b / sec / 1e9, 1), "frac_of_peak": round(b / sec / 1e9 / HBM_PEAK_GBS, 4)}
            for name, (b, sec, shape) in out.items()}


def cpu_baseline(prompt, steps_gpu_tokens, first_gpu, decode_steps=8):
    from oracle import qwen3 as Q
    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    shape = Q.SHAPES["0.6b"]
    weights = Q.generate_weights(shape, seed=0)
    oracle = Q.Oracle(shape, weights, capacity=len(prompt) + decode_steps + 1)
    cache = Q.new_cache(shape, oracle.capacity)
    ids = torch.tensor([prompt], dtype=torch.int64)
    t0 = time.perf_counter()
    tok, _, _ = oracle.forward(ids, cache, torch.arange(len(prompt)))
    prefill_s = time.perf_counter() - t0
    tokens = [int(tok[0, 0])]
    t0 = time.perf_counter()
    for i in range(decode_steps):
        pos = torch.tensor([len(prompt) + i])
        tok, _, _ = oracle.forward(torch.tensor([[tokens[-1]]]), cache, pos)
        tokens.append(int(tok[0, 0]))
    decode_s = time.perf_counter() - t0
    agree = tokens[0] == first_gpu and tokens[1:] == steps_gpu_tokens[:decode_steps]
    cpu_name = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu_name = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {"value": decode_steps / decode_s, "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"CPU oracle (torch eager, bf16 rounding of the reference path) on the same "
                      f"0.6B workload: one batched prefill of the {len(prompt)}-token prompt "
                      f"({prefill_s:.1f}s) then {decode_steps} greedy decode steps at ctx "
                      f"{len(prompt)}-{len(prompt) + decode_steps - 1}; tok/s over the decode steps",
            "prefill_s": round(prefill_s, 3), "tokens_match_gpu": bool(agree),
            "cpu_tokens": tokens, "gpu_tokens": [first_gpu] + list(steps_gpu_tokens[:decode_steps]),
            "cpu_model": cpu_name, "os_cpu_count": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0))}


def pmc_pass(shape="qwen3-0.6b"):
    """Short, graph-free workload for rocprofv3 --pmc passes (counter collection
    is per dispatch, so every kernel is launched eagerly): 8 decode steps of the
    shape's workload (0.6B at context 512, 8B at context 2048 over a synthetic
    cache), one launch of the dominant kernel per layer over the layers'
    weights, and a 256 MiB device copy (reads and writes exactly 256 MiB) that
    calibrates the byte counters."""
    cfg = shape_config(shape)
    model = Qwen3Model.random(cfg)
    ctx = 512 if shape == "qwen3-0.6b" else 2048
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
    print(json.dumps({"pmc_pass": True, "calibration_copy_bytes": src.numel() * 2,
                      "dominant_kernel_bytes": n2 * k * 2 + k * 4 + cfg.intermediate_size * 2}),
          flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-8b", action="store_true")
    ap.add_argument("--quiet", action="store_true")
    ap.add_argument("--pmc-shape", default="qwen3-0.6b", choices=("qwen3-0.6b", "qwen3-8b"),
                    help="model shape of the --pmc-pass workload")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="short workload for rocprofv3 counter passes (no JSON bench line)")
    ap.add_argument("--section", default="all",
                    choices=("all", "qwen3-8b", "qwen3-8b-int8", "qwen3-8b-fp8", "speculative",
                             "batched", "per-op"),
                    help="run one secondary workload alone and print its JSON (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the batch-one decode path on exactly one GPU; "
              "multi-GPU runs are not part of this build", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        sys.exit(2)

    if args.pmc_pass:
        pmc_pass(args.pmc_shape)
        return

    def log(msg):
        if not args.quiet:
            print(msg, file=sys.stderr, flush=True)

    if args.section != "all":
        if args.section == "qwen3-8b":
            r = run_decode("qwen3-8b", 2048, 256, args.warmup, log)
            out = {k: r[k] for k in ("tok_s", "ms_per_step", "bytes_per_token", "decode_frac")}
        elif args.section == "speculative":
            out = run_draft_speculation(4096, 128, 4, log)
        elif args.section == "batched":
            out = run_batched("qwen3-8b", 512, 32, (1, 4, 16), log)
        elif args.section == "per-op":
            out = {"per_op": per_op_microbench()}
        else:
            fmt = "int8" if args.section.endswith("int8") else "fp8_e4m3"
            r = run_decode("qwen3-8b", 8192, 128, args.warmup, log, weight_format=fmt,
                           synthetic_context=True)
            out = {k: r[k] for k in ("tok_s", "ms_per_step", "bytes_per_token", "decode_frac")}
        print(json.dumps({"section": args.section, **out}), flush=True)
        return

    res = run_decode("qwen3-0.6b", args.prompt, args.steps, args.warmup, log)
    log(f"qwen3-0.6b: {res['tok_s']:.1f} tok/s, {res['ms_per_step']:.3f} ms/step")
    dom = dominant_kernel(res["model"])
    log(f"dominant kernel: {dom['avg_us']:.2f} us/launch, {dom['achieved']:.0f} GB/s")
    line = {
        "metric": METRIC, "value": round(res["tok_s"], 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init N(0,0.02) bf16 weights and uniform prompt ids from the "
                "counter RNG (seed 0 weights, seed 1 prompt)",
        "config": {"workload": "Qwen3-0.6B-shape bf16 batch-1 greedy decode, prompt "
                               f"{args.prompt}, {args.steps} steps (context {args.prompt}-"
                               f"{args.prompt + args.steps - 1}), captured HIP graph per step",
                   "batch": 1, "prompt_tokens": args.prompt, "decode_steps": args.steps},
        "roofline": {"bound": "hbm", "achieved": round(dom["achieved"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["achieved"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": dom["name"], "avg_launch_us": round(dom["avg_us"], 3),
                     "bytes_per_launch": dom["bytes"]},
        "decode_roofline": {"bytes_per_token": res["bytes_per_token"],
                            "achieved_GBs": round(res["bytes_per_token"] * res["tok_s"] / 1e9, 1),
                            "frac": round(res["decode_frac"], 4),
                            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / res["bytes_per_token"], 1)},
        "first_tokens": [res["first"]] + res["tokens"][:15],
    }
    del res["model"]
    torch.cuda.empty_cache()
    line["per_op"] = per_op_microbench()
    torch.cuda.empty_cache()
    if not args.no_8b:
        try:
            r8 = run_decode("qwen3-8b", 2048, 256, args.warmup, log)
            del r8["model"]
            torch.cuda.empty_cache()
            line["qwen3_8b"] = {"workload": "Qwen3-8B-shape bf16, prompt 2048, 256 greedy steps",
                                "tok_s": round(r8["tok_s"], 2),
                                "ms_per_step": round(r8["ms_per_step"], 4),
                                "bytes_per_token": r8["bytes_per_token"],
                                "roofline_frac": round(r8["decode_frac"], 4),
                                "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / r8["bytes_per_token"], 1)}
            log(f"qwen3-8b: {r8['tok_s']:.1f} tok/s ({100 * r8['decode_frac']:.1f}% of roofline)")
        except Exception as exc:  # report, do not lose the headline line
            line["qwen3_8b"] = {"error": repr(exc)}
        for fmt in ("int8", "fp8_e4m3"):
            key = "qwen3_8b_" + fmt.split("_")[0]
            try:
                rq = run_decode("qwen3-8b", 8192, 128, args.warmup, log, weight_format=fmt,
                                synthetic_context=True)
                del rq["model"]
                torch.cuda.empty_cache()
                line[key] = {"workload": f"Qwen3-8B-shape, weight-only {fmt} projections and LM "
                                         "head, bf16 activations and KV, 128 greedy steps at "
                                         "context 8192-8319 (synthetic N(0,1) KV cache)",
                             "tok_s": round(rq["tok_s"], 2),
                             "ms_per_step": round(rq["ms_per_step"], 4),
                             "bytes_per_token": rq["bytes_per_token"],
                             "roofline_frac": round(rq["decode_frac"], 4),
                             "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / rq["bytes_per_token"], 1)}
                log(f"qwen3-8b {fmt}: {rq['tok_s']:.1f} tok/s "
                    f"({100 * rq['decode_frac']:.1f}% of roofline)")
            except Exception as exc:
                line[key] = {"error": repr(exc)}
    if not args.no_8b:
        try:
            line["speculative_4b_draft_0.6b"] = run_draft_speculation(4096, 128, 4, log)
        except Exception as exc:
            line["speculative_4b_draft_0.6b"] = {"error": repr(exc)}
        torch.cuda.empty_cache()
        try:
            line["batched_qwen3_8b"] = run_batched("qwen3-8b", 512, 32, (4, 16), log)
        except Exception as exc:
            line["batched_qwen3_8b"] = {"error": repr(exc)}
        torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(res["prompt"], res["tokens"], res["first"])
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
