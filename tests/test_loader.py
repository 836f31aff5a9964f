"""Checkpoint loading (Qwen3Model.from_pretrained, Engine(model_path)) from a
Hugging Face-style directory: config.json plus safetensors shards with the
Hugging Face tensor names.

The reference loads such a directory with transformers and repacks q/k/v and
gate/up at load time (dryft/engine/engine.py:42-48,64-67,
dryft/engine/attention.py:54-63). The round trip writes the oracle's seeded
weights under those names (split back into q/k/v and gate/up, in two shards),
loads them, and checks the packed tensors bit for bit; on the GPU the loaded
model decodes the golden ids of the seeded model.
"""
import json
import os

import pytest
import torch
from safetensors.torch import save_file

from oracle import qwen3 as Q
from hackthenorth_amd.model import Qwen3Model, shape_config

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def hf_tensors(shape, w):
    """Hugging Face names for the oracle's packed weights."""
    d = shape.head_dim
    q, kv = shape.q_heads * d, shape.kv_heads * d
    out = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["norm"]}
    if not shape.tied:
        out["lm_head.weight"] = w["lm_head"]
    for l in range(shape.layers):
        p = f"model.layers.{l}."
        qkv, gu = w[f"{l}.qkv"], w[f"{l}.gate_up"]
        out[p + "self_attn.q_proj.weight"] = qkv[:q]
        out[p + "self_attn.k_proj.weight"] = qkv[q:q + kv]
        out[p + "self_attn.v_proj.weight"] = qkv[q + kv:]
        out[p + "self_attn.o_proj.weight"] = w[f"{l}.o"]
        out[p + "mlp.gate_proj.weight"] = gu[:shape.ffn]
        out[p + "mlp.up_proj.weight"] = gu[shape.ffn:]
        out[p + "mlp.down_proj.weight"] = w[f"{l}.down"]
        out[p + "input_layernorm.weight"] = w[f"{l}.ln1"]
        out[p + "post_attention_layernorm.weight"] = w[f"{l}.ln2"]
        out[p + "self_attn.q_norm.weight"] = w[f"{l}.q_norm"]
        out[p + "self_attn.k_norm.weight"] = w[f"{l}.k_norm"]
    return {k: v.contiguous() for k, v in out.items()}


def write_checkpoint(path, name, shape, w):
    """config.json in the Hugging Face Qwen3 layout (no random_init) and two shards."""
    os.makedirs(path, exist_ok=True)
    cfg = shape_config(name).to_dict()
    cfg.pop("random_init", None)
    cfg.update(architectures=["Qwen3ForCausalLM"], model_type="qwen3", torch_dtype="bfloat16")
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    tensors = hf_tensors(shape, w)
    names = sorted(tensors)
    half = len(names) // 2
    for i, part in enumerate((names[:half], names[half:])):
        save_file({k: tensors[k] for k in part},
                  os.path.join(path, f"model-0000{i + 1}-of-00002.safetensors"))
    return path


def packed_pairs(model, w, shape):
    pairs = [("embed", model.embed_weight, w["embed"]), ("norm", model.norm.weight, w["norm"]),
             ("lm_head", model.lm_head_weight, w["lm_head"])]
    for l, layer in enumerate(model.layers):
        for kind, t in layer.tensors().items():
            pairs.append((f"{l}.{kind}", t, w[f"{l}.{kind}"]))
        pairs += [(f"{l}.ln1", layer.input_layernorm.weight, w[f"{l}.ln1"]),
                  (f"{l}.ln2", layer.post_attention_layernorm.weight, w[f"{l}.ln2"]),
                  (f"{l}.q_norm", layer.q_norm.weight, w[f"{l}.q_norm"]),
                  (f"{l}.k_norm", layer.k_norm.weight, w[f"{l}.k_norm"])]
    return pairs


def test_safetensors_round_trip_packs_bit_for_bit(tmp_path):
    shape = Q.SHAPES["tiny"]
    w = Q.generate_weights(shape, seed=0)
    # Gains that are not all ones, so a gain loaded into the wrong slot shows.
    for l in range(shape.layers):
        for i, g in enumerate(("ln1", "ln2", "q_norm", "k_norm")):
            w[f"{l}.{g}"] = Q.normal_bf16(40 + l, i, w[f"{l}.{g}"].shape, 1.0)
    w["norm"] = Q.normal_bf16(41, 9, w["norm"].shape, 1.0)
    path = write_checkpoint(str(tmp_path / "ckpt"), "tiny", shape, w)
    model = Qwen3Model.from_pretrained(path, device="cpu")
    assert model.config.random_init is None
    for name, actual, expected in packed_pairs(model, w, shape):
        assert actual.shape == expected.shape, name
        assert torch.equal(actual.view(torch.int16), expected.view(torch.int16)), name


def test_tied_checkpoint_shares_the_embedding(tmp_path):
    shape = Q.SHAPES["tiny"]
    import dataclasses
    tied = dataclasses.replace(shape, tied=True)
    w = Q.generate_weights(tied, seed=0)
    path = write_checkpoint(str(tmp_path / "tied"), "tiny", tied, w)
    with open(os.path.join(path, "config.json")) as f:
        cfg = json.load(f)
    cfg["tie_word_embeddings"] = True
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    model = Qwen3Model.from_pretrained(path, device="cpu")
    assert model.lm_head_weight is model.embed_weight
    assert torch.equal(model.lm_head_weight.view(torch.int16), w["embed"].view(torch.int16))


@pytest.mark.gpu
def test_engine_from_checkpoint_decodes_the_seeded_model(tmp_path):
    from hackthenorth_amd.engine import Engine
    with open(os.path.join(GOLDEN, "tiny_decode.json")) as f:
        meta = json.load(f)
    shape = Q.SHAPES["tiny"]
    w = Q.generate_weights(shape, seed=meta["seed"])
    path = write_checkpoint(str(tmp_path / "ckpt"), "tiny", shape, w)
    engine = Engine(path, speculative=False)
    random_init = Qwen3Model.random(shape_config("tiny", seed=meta["seed"]), seed=meta["seed"])
    for name, actual, expected in packed_pairs(engine.model, w, shape):
        assert torch.equal(actual.cpu().view(torch.int16), expected.view(torch.int16)), name
    for (_, loaded, _), (_, seeded, _) in zip(packed_pairs(engine.model, w, shape),
                                              packed_pairs(random_init, w, shape)):
        assert torch.equal(loaded.view(torch.int16), seeded.view(torch.int16))
    steps = len(meta["tokens"])
    got = [t[0] for t in engine.generate([meta["prompt"]], steps)]
    for i, (a, e) in enumerate(zip(got, meta["tokens"])):
        if a != e:
            assert meta["top2_gap_fp32"][i] < 2e-2, (i, a, e)
            break
    print(f"checkpoint decode: {sum(a == e for a, e in zip(got, meta['tokens']))}/{steps} "
          "ids equal to the golden decode", flush=True)
