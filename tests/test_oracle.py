"""Pin the CPU oracle before trusting it.

  * against the installed transformers Qwen3 (same formulas as the reference's
    pinned 4.51.3) on identical weights: RoPE tables bit-equal, greedy ids
    equal, logits close;
  * against literal known answers from the reference tests (halfway rounding,
    greedy tie, residual-sum exactness, RMSNorm cast placement);
  * against invariants: fixed-cache decode equals full-prefix recompute
    (dryft/tests/test_decode.py:92-115), masked NaN slots are never read;
  * against the committed golden fixtures it wrote.
A planted mistake (a dropped bf16 rounding, a wrong rotate_half sign, a
transposed projection) fails at least one of these; see
test_planted_mistakes_are_caught.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import qwen3 as Q

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BF16 = torch.bfloat16


def tiny():
    shape = Q.SHAPES["tiny"]
    return shape, Q.generate_weights(shape, seed=0)


def hf_model(shape, weights):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen3Config(
        vocab_size=shape.vocab, hidden_size=shape.hidden, intermediate_size=shape.ffn,
        num_hidden_layers=shape.layers, num_attention_heads=shape.q_heads,
        num_key_value_heads=shape.kv_heads, head_dim=shape.head_dim,
        tie_word_embeddings=shape.tied, rope_theta=shape.theta, rms_norm_eps=shape.eps)
    cfg._attn_implementation = "eager"
    model = transformers.Qwen3ForCausalLM(cfg).eval()
    inv_freq = model.model.rotary_emb.inv_freq.clone()   # keep the fp32 buffer
    model = model.to(BF16)
    model.model.rotary_emb.inv_freq = inv_freq
    d = shape.head_dim
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(weights["embed"])
        if not shape.tied:
            model.lm_head.weight.copy_(weights["lm_head"])
        for l, layer in enumerate(model.model.layers):
            q, k, v = weights[f"{l}.qkv"].split((shape.q_heads * d, shape.kv_heads * d,
                                                 shape.kv_heads * d))
            layer.self_attn.q_proj.weight.copy_(q)
            layer.self_attn.k_proj.weight.copy_(k)
            layer.self_attn.v_proj.weight.copy_(v)
            layer.self_attn.o_proj.weight.copy_(weights[f"{l}.o"])
            g, u = weights[f"{l}.gate_up"].chunk(2)
            layer.mlp.gate_proj.weight.copy_(g)
            layer.mlp.up_proj.weight.copy_(u)
            layer.mlp.down_proj.weight.copy_(weights[f"{l}.down"])
    return model


def test_rope_tables_equal_transformers_rotary_module():
    shape, weights = tiny()
    model = hf_model(shape, weights)
    cos, sin = model.model.rotary_emb(model.model.embed_tokens.weight[:1].unsqueeze(0),
                                      torch.arange(300)[None])
    ocos, osin = Q.rope_tables(300, shape.head_dim, shape.theta)
    assert torch.equal(cos[0], ocos) and torch.equal(sin[0], osin)


def test_greedy_decode_matches_transformers():
    shape, weights = tiny()
    model = hf_model(shape, weights)
    prompt = Q.prompt_ids(7, shape.vocab)
    oracle = Q.Oracle(shape, weights, capacity=40)
    tokens, logits, _ = oracle.greedy_decode(prompt, 16)
    ids = torch.tensor([prompt])
    with torch.no_grad():
        for i, tok in enumerate(tokens):
            ref = model(ids, use_cache=False).logits[0, -1].float()
            # transformers' eager attention rounds scores and probabilities to
            # bf16; the oracle keeps them fp32, so logits agree to ~1e-2.
            torch.testing.assert_close(logits[i], ref, atol=3e-2, rtol=0)
            top = torch.topk(ref, 2).values
            if float(top[0] - top[1]) > 3e-2:
                assert int(ref.argmax()) == tok
            ids = torch.cat([ids, torch.tensor([[tok]])], 1)


def test_halfway_projection_rounds_before_residual():
    # dryft/tests/test_fused_kernels.py:179-187
    x = torch.ones(1, 1, 33, dtype=BF16)
    w = torch.zeros(3, 33, dtype=BF16)
    w[:, 0] = 1
    w[:, 1] = 1 / 256
    assert bool((Q.output_residual(x, w, -torch.ones(1, 1, 3, dtype=BF16)) == 0).all())


def test_greedy_tie_picks_lowest_id():
    # dryft/tests/test_fused_kernels.py:169-173
    w = torch.zeros(1000, 64, dtype=BF16)
    w[3] = 1
    w[-1] = 1
    logits = Q.linear(torch.ones(3, 64, dtype=BF16), w)
    assert Q.greedy(logits).tolist() == [3, 3, 3]


def test_add_rms_norm_sum_exact_and_cast_placement():
    x = Q.normal_bf16(3, 1, (4, 2560), 1.0)
    r = Q.normal_bf16(3, 2, (4, 2560), 1.0)
    g = Q.normal_bf16(3, 3, (2560,), 1.0)
    s, n = Q.add_rms_norm(x, r, g, 1e-6)
    assert torch.equal(s, x + r)  # torch's bf16 add rounds once, like the kernel
    # The gain multiplies the *rounded* normalized value (rmsnorm.py:70-79):
    v = s.float()
    inv = torch.rsqrt(v.square().mean(-1, keepdim=True) + 1e-6)
    fused_once = (g.float() * (v * inv)).to(BF16)
    assert torch.equal(n, (g * (v * inv).to(BF16)))
    assert not torch.equal(n, fused_once)  # the two formulas differ on this input


def test_attention_never_reads_masked_slots_and_matches_dense_softmax():
    q = Q.normal_bf16(4, 1, (1, 8, 3, 128), 1.0)
    k = Q.normal_bf16(4, 2, (1, 2, 50, 128), 1.0)
    v = Q.normal_bf16(4, 3, (1, 2, 50, 128), 1.0)
    positions = torch.tensor([10, 11, 12])
    out = Q.attention(q, k, v, positions)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 13:] = float("nan")
    v2[:, :, 13:] = float("nan")
    assert torch.equal(Q.attention(q, k2, v2, positions), out)
    # Dense reference with repeat_interleave (dryft/tests/test_fused_kernels.py:396-401).
    kk, vv = k.float().repeat_interleave(4, 1), v.float().repeat_interleave(4, 1)
    mask = torch.arange(50)[None, :] <= positions[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), kk, vv, attn_mask=mask)
    torch.testing.assert_close(out.float(), ref, atol=1e-2, rtol=1e-2)


def test_fixed_cache_decode_equals_full_prefix_recompute():
    # dryft/tests/test_decode.py:92-115, with stale +-1000 storage.
    shape, weights = tiny()
    oracle = Q.Oracle(shape, weights, capacity=12)
    prompt = Q.prompt_ids(5, shape.vocab, seed=9)
    cache = Q.new_cache(shape, 12, fill=1000.0)
    tok, _, _ = oracle.forward(torch.tensor([prompt]), cache, torch.arange(5))
    seq = list(prompt)
    for step in range(6):
        full = Q.new_cache(shape, 12, fill=-1000.0)
        expect, _, _ = oracle.forward(torch.tensor([seq]), full, torch.arange(len(seq)))
        assert int(tok) == int(expect)
        seq.append(int(tok))
        tok, _, _ = oracle.forward(tok.view(1, 1), cache, torch.tensor([len(seq) - 1]))


def test_planted_mistakes_are_caught(monkeypatch):
    """A dropped rounding or a flipped rotate_half sign changes the oracle's outputs."""
    x = Q.normal_bf16(5, 1, (1, 1, 4, 128), 1.0)
    g = Q.normal_bf16(5, 2, (128,), 1.0)
    cos, sin = Q.rope_tables(8, 128, 1e6)
    good = Q.norm_rope(x, g, cos[5], sin[5], 1e-6)
    n = Q.rms_norm(x, g, 1e-6).float()
    flipped = torch.cat((n[..., 64:], -n[..., :64]), -1)
    bad = ((n * cos[5].float()).to(BF16).float() + (flipped * sin[5].float()).to(BF16).float()).to(BF16)
    assert not torch.equal(good, bad)
    w = Q.normal_bf16(5, 3, (48, 64), 0.02)
    xr = Q.normal_bf16(5, 4, (64,), 1.0)
    r = Q.normal_bf16(5, 5, (48,), 1.0)
    unrounded = ((xr.float() @ w.float().T) + r.float()).to(BF16)
    assert not torch.equal(Q.output_residual(xr, w, r), unrounded)


def test_oracle_reproduces_tiny_golden():
    with open(os.path.join(GOLDEN, "tiny_decode.json")) as f:
        meta = json.load(f)
    shape, weights = tiny()
    tokens, _, records = Q.Oracle(shape, weights, capacity=meta["capacity"]).greedy_decode(
        meta["prompt"], len(meta["tokens"]), record_steps=3)
    assert tokens == meta["tokens"]
    hidden = np.load(os.path.join(GOLDEN, "tiny_decode_hidden.npz"))["hidden"]
    for s, step in enumerate(records):
        for l, h in enumerate(step):
            exp = torch.from_numpy(hidden[s, l].view(np.int16)).view(BF16)
            torch.testing.assert_close(h.reshape(-1), exp, atol=1e-2, rtol=1e-2)


def test_oracle_reproduces_qwen3_06b_golden_prefix():
    with open(os.path.join(GOLDEN, "qwen3_0.6b_decode.json")) as f:
        meta = json.load(f)
    shape = Q.SHAPES["0.6b"]
    oracle = Q.Oracle(shape, Q.generate_weights(shape, seed=0), capacity=meta["capacity"])
    tokens, _, _ = oracle.greedy_decode(meta["prompt"], 4)
    assert tokens == meta["tokens"][:4]


def test_ops_fixture_reproduces():
    data = np.load(os.path.join(GOLDEN, "ops.npz"))

    def t(name, shape):
        return torch.from_numpy(data[name].view(np.int16)).view(BF16).reshape(shape)

    x, r, gain = t("add_x", (4, 1024)), t("add_r", (4, 1024)), t("add_gain", (1024,))
    s, n = Q.add_rms_norm(x, r, gain, 1e-6)
    assert torch.equal(s, t("add_sum", (4, 1024)))
    torch.testing.assert_close(n, t("add_norm", (4, 1024)), atol=1e-2, rtol=1e-2)
    w, xr = t("proj_w", (40, 1024)), t("proj_x", (1024,))
    torch.testing.assert_close(Q.linear(xr, w), t("proj_y", (40,)), atol=1e-2, rtol=1e-2)


def test_float64_order_keeps_the_bf16_boundaries_and_differs_only_by_rounding():
    """The float64 evaluation is the same formula: with inputs whose products
    and sums are exact in both types it is bit-equal to the float32 one, and
    on a model its logits stay within the float32 rounding noise."""
    # Exact case: small integers times powers of two sum exactly in fp32.
    x = torch.tensor([[1.0, 2.0, -3.0, 0.5]], dtype=BF16)
    w = torch.tensor([[0.25, 1.0, 2.0, -4.0], [1.0, 1.0, 1.0, 1.0]], dtype=BF16)
    shape = Q.Shape(hidden=4, layers=0, q_heads=1, kv_heads=1, head_dim=128, ffn=4,
                    vocab=2, tied=False)
    weights = {"lm_head": w, "embed": w, "norm": torch.ones(4, dtype=BF16)}
    o32 = Q.Oracle(shape, weights, 4)
    o64 = Q.Oracle(shape, weights, 4, acc=torch.float64)
    assert torch.equal(o32._linear(x, "lm_head"), o64._linear(x, "lm_head"))
    assert o64._dot(x, "lm_head").dtype == torch.float64
    # A dropped bf16 rounding is not a different order: rms_norm keeps it.
    v = Q.normal_bf16(6, 1, (3, 256), 1.0)
    g = Q.normal_bf16(6, 2, (256,), 1.0)
    n64 = Q.rms_norm(v, g, 1e-6, torch.float64)
    vv = v.double()
    unrounded = (g.double() * vv * torch.rsqrt(vv.square().mean(-1, keepdim=True) + 1e-6))
    assert torch.equal(n64, (g.double() * (vv * torch.rsqrt(
        vv.square().mean(-1, keepdim=True) + 1e-6)).to(BF16).double()).to(BF16))
    assert not torch.equal(n64, unrounded.to(BF16))
    # Whole model: float64 and float32 logits agree to the noise of fp32
    # summation order through two bf16-rounded layers.
    shape, weights = tiny()
    prompt = Q.prompt_ids(9, shape.vocab, seed=4)
    l32 = Q.Oracle(shape, weights, 16).teacher_forced_logits(prompt, [1, 2, 3])
    l64 = Q.Oracle(shape, weights, 16, acc=torch.float64).teacher_forced_logits(prompt,
                                                                               [1, 2, 3])
    torch.testing.assert_close(l64, l32, atol=2e-2, rtol=0)
    with pytest.raises(ValueError):
        Q.Oracle(shape, weights, 16, acc=torch.float16)


def test_stepwise_logits_equal_the_decode_loop():
    """stepwise_logits is the oracle's own decode loop: the logits it returns
    are those greedy_decode computes when fed the same tokens."""
    shape, weights = tiny()
    oracle = Q.Oracle(shape, weights, capacity=20)
    prompt = Q.prompt_ids(6, shape.vocab, seed=5)
    tokens, logits, _ = oracle.greedy_decode(prompt, 5)
    stepwise = oracle.stepwise_logits(prompt, tokens)
    for i in range(5):
        assert torch.equal(stepwise[i], logits[i])
    batched = oracle.teacher_forced_logits(prompt, tokens)
    torch.testing.assert_close(batched, stepwise, atol=2e-2, rtol=0)
