"""Parity at the benchmark configurations: the HIP path against the CPU oracle
at the shapes and contexts the bench measures.

  * Qwen3-8B shape, bf16, context 2048: two decoder layers on identical inputs
    and identical caches (teacher-forced per layer), through the decode step's
    own kernels (fused prologue attention with the O-weight prefetch);
  * the same for int8 and fp8-e4m3fn weight-only layers at context 8192;
  * the 8B LM head with its greedy argmax over all 151936 rows;
  * Qwen3-4B shape: a 5-row verify pass at context 4096 (eager and captured);
  * Qwen3-0.6B shape: 64 greedy steps after a 512-token prompt, every
    emitted token checked against the oracle's logits along the emitted
    sequence (the reference judge's replay, dryft/agent/benchmark_gpu.py:139-152);
  * batched decode through Engine.generate (4 and 16 prompts) and draft-model
    speculation, each emitted sequence checked the same way.

Layer weights come from the counter RNG on both sides (the oracle regenerates
them in numpy), so every layer is checked against independently generated
weights. Caches at long contexts hold N(0,1) values in the slots before the
query (the kernels' cost and numerics do not depend on how they were written);
the oracle gets a copy of the same cache.

Bars: per layer, every element within HIDDEN_ULPS bf16 ulps of max(|expected|,
the layer's rms) and cosine >= 0.9999 (parity_helpers.check_hidden); appended
cache rows within one bf16 ulp; greedy ids equal to the oracle's pick, or a
near-tie within the north star's 1e-3, or a step where the oracle's own
evaluation orders (token-by-token instead of one causal pass, float64 instead
of float32 between the same bf16 roundings) disagree at least as much
(oracle/parity.py); each test prints the classification of every differing
step. The LM-head test admits near-ties only: one GEMV's logits carry no
accumulated noise.
"""
import dataclasses
import json
import os

import pytest
import torch

from oracle import parity as OP
from oracle import qwen3 as Q
from oracle import rng as ORNG
from parity_helpers import check_hidden, check_record, record_sequence
from hackthenorth_amd import decode as D
from hackthenorth_amd.draft import DraftSpeculator
from hackthenorth_amd.engine import Engine
from hackthenorth_amd.kernels import rng as DR
from hackthenorth_amd.kernels.greedy import greedy_head
from hackthenorth_amd.prefill import prefill
from hackthenorth_amd.model import (STREAM_LM_HEAD, STREAM_LM_HEAD_SCALE, Qwen3Model,
                                    shape_config, write_random_model_dir)
from hackthenorth_amd.quant import QuantizedWeight

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = {"tiny": "tiny", "0.6b": "qwen3-0.6b", "4b": "qwen3-4b", "8b": "qwen3-8b"}


def within_one_ulp(label, actual, expected):
    a = actual.detach().cpu().float().reshape(-1)
    e = expected.detach().cpu().float().reshape(-1)
    ulp = torch.pow(2.0, torch.floor(torch.log2(e.abs().clamp_min(1e-30))) - 7)
    bad = (a - e).abs() > torch.maximum(ulp, torch.full_like(ulp, 1e-6))
    print(f"{label}: {int(bad.sum())} of {a.numel()} beyond one bf16 ulp", flush=True)
    assert not bool(bad.any())


def synthetic_cache(model, capacity, filled, seed_stream):
    """A KVCache whose slots [0, filled) hold N(0,1) values (zeros after)."""
    cache = D.KVCache(model, 1, capacity)
    DR.normal_(cache.storage.view(-1), 21, seed_stream, 1.0)
    cache.storage[..., filled:, :].zero_()
    return cache


def oracle_cache(cache):
    return Q.Cache(cache.storage[:, 0].cpu().clone(), cache.storage[:, 1].cpu().clone())


@pytest.mark.parametrize("fmt,ctx", [("bf16", 2048), ("int8", 8192), ("fp8_e4m3", 8192)])
def test_8b_layers_at_benchmark_context_match_oracle(fmt, ctx):
    layers = 2
    oshape = dataclasses.replace(Q.SHAPES["8b"], layers=layers, vocab=16)
    cfg = shape_config("qwen3-8b", num_hidden_layers=layers, vocab_size=16, weight_format=fmt)
    model = Qwen3Model.random(cfg)
    oracle = Q.Oracle(oshape, Q.generate_weights(oshape, seed=0, weight_format=fmt), ctx + 1)
    with torch.inference_mode():
        cache = synthetic_cache(model, ctx + 1, ctx, 80)
        ocache = oracle_cache(cache)
        rotary = D.RotaryTable(model, ctx + 1)
        pos = torch.tensor([ctx], dtype=torch.int64, device="cuda")
        rope = rotary.step_row(pos)
        h = DR.normal_(torch.empty((1, cfg.hidden_size), dtype=torch.bfloat16, device="cuda"),
                       7, 11, 1.0)
        for layer in range(layers):
            mine = D.decode_layer(model, layer, h, cache, pos, rotary, rope)
            expected = oracle.layer(layer, h.cpu().view(1, 1, -1), ocache, torch.tensor([ctx]))
            check_hidden(f"8b {fmt} ctx {ctx} layer {layer}", mine, expected)
            for kv in (0, 1):
                within_one_ulp(f"8b {fmt} ctx {ctx} layer {layer} {'kv'[kv]} row",
                               cache.storage[layer, kv, 0, :, ctx],
                               (ocache.keys if kv == 0 else ocache.values)[layer][0, :, ctx])
            h = mine


@pytest.mark.parametrize("fmt", ["bf16", "int8", "fp8_e4m3"])
def test_8b_lm_head_argmax_matches_oracle(fmt):
    """Final RMSNorm + [151936 x 4096] head + greedy argmax, several rows."""
    vocab, hidden = 151936, 4096
    dev = torch.device("cuda")
    if fmt == "bf16":
        w = DR.normal_(torch.empty((vocab, hidden), dtype=torch.bfloat16, device=dev), 0,
                       STREAM_LM_HEAD, 0.02)
        wf, scale = w.cpu().float(), None
    else:
        w = QuantizedWeight.empty(vocab, hidden, fmt, dev)
        w.randomize_(0, STREAM_LM_HEAD, STREAM_LM_HEAD_SCALE)
        codes = w.data.cpu().numpy().reshape(-1)
        wf = torch.from_numpy(ORNG.w8_values(codes, fmt)).view(vocab, hidden)
        scale = w.scale.cpu()
    gain = DR.normal_(torch.empty((hidden,), dtype=torch.bfloat16, device=dev), 4, 9, 1.0)
    record = OP.TokenRecord()
    normed = []
    with torch.inference_mode():
        for row in range(6):
            x = DR.normal_(torch.empty((hidden,), dtype=torch.bfloat16, device=dev), 30 + row,
                           1, 1.0)
            token = torch.empty((1,), dtype=torch.int64, device=dev)
            greedy_head(x, gain, 1e-6, w, token)
            xn = Q.rms_norm(x.cpu(), gain.cpu(), 1e-6)
            normed.append(xn)
            logits = xn.float() @ wf.T
            if scale is not None:
                logits = logits * scale
            record.add(row, logits, int(token))

    def float64(step):
        logits = normed[step].double() @ wf.double().T
        return logits if scale is None else logits * scale.double()

    summary = check_record(record, f"8b LM head {fmt}", {"float64": float64})
    # One GEMV: a differing id must be a near-tie, not accumulated noise.
    assert summary["oracle_noise"] == 0, summary


def test_4b_verify_rows_at_context_4096_match_oracle():
    layers, ctx, rows = 2, 4096, 5
    oshape = dataclasses.replace(Q.SHAPES["4b"], layers=layers)
    cfg = shape_config("qwen3-4b", num_hidden_layers=layers)
    model = Qwen3Model.random(cfg)
    oracle = Q.Oracle(oshape, Q.generate_weights(oshape, seed=0), ctx + rows)
    ids = Q.prompt_ids(rows, oshape.vocab, seed=9)
    with torch.inference_mode():
        cache = synthetic_cache(model, ctx + rows, ctx, 81)
        ocache = oracle_cache(cache)
        rotary = D.RotaryTable(model, ctx + rows)
        positions = torch.arange(ctx, ctx + rows, device="cuda")
        record = []
        got = D.forward(model, torch.tensor([ids], device="cuda"), cache, positions,
                        last_only=False, rotary=rotary, record=record)[0].cpu()
        clean = oracle_cache(cache)
        _, logits, _ = oracle.forward(torch.tensor([ids]), ocache, torch.arange(ctx, ctx + rows),
                                      last_only=False)
        # Per layer on identical inputs: the oracle's layer l gets the HIP
        # rows that entered the HIP's layer l, and a cache holding the same
        # earlier slots.
        per_layer = Q.Cache(clean.keys.clone(), clean.values.clone())
        h = oracle.weights["embed"][torch.tensor([ids])]
        opos = torch.arange(ctx, ctx + rows)
        for layer in range(layers):
            expected = oracle.layer(layer, h, per_layer, opos)
            check_hidden(f"4b verify rows ctx {ctx} layer {layer}", record[layer], expected)
            for kv, name in ((0, "k"), (1, "v")):
                mine = cache.storage[layer, kv, 0, :, ctx:ctx + rows]
                ref = (per_layer.keys if kv == 0 else per_layer.values)[layer][0, :, ctx:ctx + rows]
                check_hidden(f"4b verify rows layer {layer} new {name} rows", mine, ref)
            h = record[layer].cpu()
        tokens = OP.TokenRecord()
        for i, t in enumerate(got.tolist()):
            tokens.add(i, logits[0, i], t)

        def stepwise():
            c = Q.Cache(clean.keys.clone(), clean.values.clone())
            return torch.stack([oracle.forward(torch.tensor([[t]]), c, torch.tensor([ctx + i]))[1]
                                [0, 0] for i, t in enumerate(ids)])

        def float64():
            o64 = Q.Oracle(oshape, oracle.weights, ctx + rows, acc=torch.float64)
            c = Q.Cache(clean.keys.clone(), clean.values.clone())
            return o64.forward(torch.tensor([ids]), c, torch.arange(ctx, ctx + rows),
                               last_only=False)[1][0]

        check_record(tokens, "4b 5-row verify",
                     OP.Orders(stepwise=stepwise, float64=float64).callables())
        # The captured verify graph gives the eager pass's bits.
        state = D.DecodeState(model, 1, ctx, 4, speculative=True, draft_tokens=rows - 1)
        state.cache.storage[..., :ctx, :].copy_(cache.storage[..., :ctx, :])
        state.verify_input.copy_(torch.tensor([ids], device="cuda"))
        state.position.fill_(ctx)
        state.verify_graph.replay()
        assert state.verify_output[0].cpu().tolist() == got.tolist()


def test_0p6b_decode_at_context_512_teacher_forced():
    shape = Q.SHAPES["0.6b"]
    prompt_len, steps = 512, 64
    prompt = Q.prompt_ids(prompt_len, shape.vocab)
    model = Qwen3Model.random(shape_config("qwen3-0.6b"))
    from hackthenorth_amd.kernels import attention as A
    A.xcd_merge_mismatches(reset=True)
    with torch.inference_mode():
        state = D.DecodeState(model, 1, prompt_len, steps)
        first = state.prefill(model, torch.tensor([prompt], device="cuda"))[:, 0].tolist()
        emitted = [t[0] for t in D.stream_decode(state, first, steps)]
    # Every in-kernel split merge of the 64 captured steps saw its pair's
    # splits on its own XCD.
    assert A.xcd_merge_mismatches() == 0
    oracle = Q.Oracle(shape, Q.generate_weights(shape, seed=0), prompt_len + steps)
    record_sequence(oracle, prompt, emitted, "0.6b ctx 512, 64 steps")


def test_8b_full_depth_decode_teacher_forced():
    """All 36 layers of the 8B shape (random weights, full vocabulary): a
    256-token prompt through the batched prefill (library products), then 16
    steps of the captured decode graph (fused attention + output projection),
    every emitted token teacher-forced against the oracle's 36-layer pass."""
    shape = Q.SHAPES["8b"]
    prompt_len, steps = 256, 16
    prompt = Q.prompt_ids(prompt_len, shape.vocab)
    model = Qwen3Model.random(shape_config("qwen3-8b"))
    from hackthenorth_amd.kernels import attention as A
    A.xcd_merge_mismatches(reset=True)
    with torch.inference_mode():
        state = D.DecodeState(model, 1, prompt_len, steps)
        first = prefill(model, state, torch.tensor([prompt], device="cuda"))[:, 0].tolist()
        emitted = [t[0] for t in D.stream_decode(state, first, steps)]
    assert A.xcd_merge_mismatches() == 0
    del state, model
    torch.cuda.empty_cache()
    oracle = Q.Oracle(shape, Q.generate_weights(shape, seed=0), prompt_len + steps)
    record_sequence(oracle, prompt, emitted, "8b full depth, prompt 256, 16 steps")


def test_8b_prefill_2048_matches_oracle_batched_forward():
    """The captured batched prefill of a 2048-token prompt (two 8B layers):
    per layer on identical inputs, every prompt slot's K/V and every row of
    the layer output against the oracle's batched layer; the first token
    against the oracle's whole forward; the graph's caches and token equal
    to the eager pass's; a replay on a second prompt equal to the eager pass
    on that prompt."""
    layers, length = 2, 2048
    oshape = dataclasses.replace(Q.SHAPES["8b"], layers=layers, vocab=64)
    cfg = shape_config("qwen3-8b", num_hidden_layers=layers, vocab_size=64)
    model = Qwen3Model.random(cfg)
    oracle = Q.Oracle(oshape, Q.generate_weights(oshape, seed=0), length + 1)
    prompts = [Q.prompt_ids(length, oshape.vocab, seed=s) for s in (1, 2)]
    with torch.inference_mode():
        state = D.DecodeState(model, 1, length, 2)
        first = prefill(model, state, torch.tensor([prompts[0]], device="cuda"))
        assert int(state.position) == length
        # The same pass eagerly, with every layer's output rows recorded.
        cache = D.KVCache(model, 1, length + 1)
        rows = []
        eager_first = D.forward(model, torch.tensor([prompts[0]], device="cuda"), cache,
                                torch.arange(length, device="cuda"), rotary=state.rotary,
                                record=rows)
        assert torch.equal(eager_first, first)
        assert torch.equal(cache.storage[..., :length, :], state.cache.storage[..., :length, :])
        ocache = Q.new_cache(oshape, length + 1)
        positions = torch.arange(length)
        h = oracle.weights["embed"][torch.tensor([prompts[0]])]
        for layer in range(layers):
            expected = oracle.layer(layer, h, ocache, positions)
            check_hidden(f"prefill 2048 layer {layer} output rows", rows[layer], expected)
            for kv, name in ((0, "k"), (1, "v")):
                mine = state.cache.storage[layer, kv, 0, :, :length]
                ref = (ocache.keys if kv == 0 else ocache.values)[layer][0, :, :length]
                check_hidden(f"prefill 2048 layer {layer} {name} cache", mine, ref)
            h = rows[layer].cpu()
        _, logits, _ = oracle.forward(torch.tensor([prompts[0]]), Q.new_cache(oshape, length + 1),
                                      positions)
        record = OP.TokenRecord()
        record.add(0, logits[0, 0], int(first[0, 0]))
        o64 = Q.Oracle(oshape, oracle.weights, length + 1, acc=torch.float64)
        check_record(record, "8b prefill 2048 first token", {
            "float64": lambda step: o64.forward(torch.tensor([prompts[0]]),
                                                Q.new_cache(oshape, length + 1),
                                                torch.arange(length))[1][0, 0]})
        replayed = int(prefill(model, state, torch.tensor([prompts[1]], device="cuda"))[0, 0])
        kv_replay = state.cache.storage[..., :length, :].clone()
        eager = int(state.prefill(model, torch.tensor([prompts[1]], device="cuda"))[0, 0])
        assert replayed == eager
        assert torch.equal(kv_replay, state.cache.storage[..., :length, :])


def golden(name):
    with open(os.path.join(GOLDEN, f"{name}.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("draft_seed,k", [(0, 4), (5, 4), (0, 1)])
def test_draft_speculation_emits_oracle_greedy_ids(draft_seed, k):
    """Draft-model speculation on the tiny golden prompt: every emitted token
    checked against the oracle's logits along the emitted sequence, and
    compared with the oracle's own greedy decode (the golden ids)."""
    meta = golden("tiny_decode")
    prompt, steps = meta["prompt"], len(meta["tokens"])
    target = Qwen3Model.random(shape_config("tiny", seed=0), seed=0)
    draft = Qwen3Model.random(shape_config("tiny", seed=draft_seed), seed=draft_seed)
    spec = DraftSpeculator(target, draft, len(prompt), steps, draft_tokens=k)
    got = [t[0] for t in spec.generate(prompt, steps)]
    shape = Q.SHAPES["tiny"]
    oracle = Q.Oracle(shape, Q.generate_weights(shape, seed=0), len(prompt) + steps)
    record_sequence(oracle, prompt, got, f"tiny draft seed {draft_seed} k {k} (acceptance "
                                         f"{spec.acceptance:.2f})")
    same = sum(a == b for a, b in zip(got, meta["tokens"]))
    print(f"{same}/{steps} ids equal to the oracle's free-running greedy decode", flush=True)


@pytest.mark.parametrize("draft_name", ["self", "0.6b"])
def test_4b_full_depth_draft_speculation_teacher_forced(draft_name):
    """Draft-model speculation with the 4B target at full depth (36 layers,
    full vocabulary), k = 4: a copy of the target as its own draft (most
    proposals accepted, so the verify pass's later rows emit tokens; the
    draft's one-row steps and the verify pass's rows round apart at
    random-weight near-ties, which rejects the rest) and the 0.6B shape as
    the draft (proposals rejected, the verify pass's first row emits); every
    emitted token teacher-forced against the oracle's 4B pass."""
    shape = Q.SHAPES["4b"]
    prompt_len, steps = 64, 24
    prompt = Q.prompt_ids(prompt_len, shape.vocab)
    target = Qwen3Model.random(shape_config("qwen3-4b"))
    draft = Qwen3Model.random(shape_config("qwen3-4b" if draft_name == "self" else "qwen3-0.6b"))
    spec = DraftSpeculator(target, draft, prompt_len, steps, draft_tokens=4)
    got = [t[0] for t in spec.generate(prompt, steps)]
    acceptance = spec.acceptance
    del spec, target, draft
    torch.cuda.empty_cache()
    if draft_name == "self":
        assert acceptance > 0.5, acceptance
    oracle = Q.Oracle(shape, Q.generate_weights(shape, seed=0), prompt_len + steps)
    record_sequence(oracle, prompt, got, f"4b full depth, {draft_name} draft, k 4 (acceptance "
                                         f"{acceptance:.2f})")


@pytest.mark.parametrize("shape_name,batch,prompt_len,steps",
                         [("tiny", 4, 9, 16), ("tiny", 16, 9, 16), ("0.6b", 4, 32, 16)])
def test_engine_generate_batched_teacher_forced(tmp_path, shape_name, batch, prompt_len, steps):
    shape = Q.SHAPES[shape_name]
    path = write_random_model_dir(str(tmp_path / shape_name), NAMES[shape_name], seed=0)
    engine = Engine(path, speculative=False)
    prompts = [Q.prompt_ids(prompt_len, shape.vocab, seed=20 + b) for b in range(batch)]
    outs = list(engine.generate(prompts, steps))
    assert len(outs) == steps and all(len(o) == batch for o in outs)
    oracle = Q.Oracle(shape, Q.generate_weights(shape, seed=0), prompt_len + steps)
    for b in range(batch):
        record_sequence(oracle, prompts[b], [o[b] for o in outs],
                        f"{shape_name} batch {batch}, sequence {b}, {steps} steps")
