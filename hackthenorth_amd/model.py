"""Qwen3 decoder weights on the device, in the layouts the decode kernels read.

The reference loads a Hugging Face checkpoint with transformers and repacks it
at load time: q/k/v rows concatenated into one QKV weight
(dryft/engine/attention.py:56-63) and gate/up rows concatenated
(dryft/engine/engine.py:42-48). This module keeps those packed row-major
layouts without transformers:

  qkv_weight      [(Hq + 2 Hkv) * 128, H]   q rows, then k rows, then v rows
  o_weight        [H, Hq * 128]
  gate_up_weight  [2 I, H]                  gate rows, then up rows
  down_weight     [H, I]
  embed_weight    [V, H]; lm_head_weight is the same tensor when tied

Weights come either from a checkpoint directory (config.json + *.safetensors
with the Hugging Face tensor names) or, for the synthetic benchmark shapes,
from a seeded device-side generator (config.json carrying "random_init").

With weight_format "int8" or "fp8_e4m3" the four projections of every layer
and the LM head are QuantizedWeight objects (one byte per weight plus an fp32
scale per row); the embedding table and the norm gains stay bf16.
"""
import glob
import json
import os
from dataclasses import dataclass, field, asdict

import torch

from .kernels import rng
from .quant import FORMATS, QuantizedWeight

# Generator stream ids per tensor; the test oracle regenerates the same
# weights from the same ids and seed.
STREAM_EMBED = 1
STREAM_LM_HEAD = 2
STREAM_LM_HEAD_SCALE = 3
_LAYER_KINDS = {"qkv": 0, "o": 1, "gate_up": 2, "down": 3}
SCALE_STREAM_OFFSET = 8  # 8-bit weights: row scales of a tensor use its stream + 8


def layer_stream(layer, kind):
    return 100 + 16 * layer + _LAYER_KINDS[kind]


def _nbytes(t):
    return t.nbytes() if isinstance(t, QuantizedWeight) else t.numel() * t.element_size()


@dataclass
class Qwen3Config:
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int
    tie_word_embeddings: bool
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    random_init: dict = field(default=None)
    weight_format: str = "bf16"   # or "int8" / "fp8_e4m3" (weight-only, per-row scales)

    @classmethod
    def from_dict(cls, d):
        keys = cls.__dataclass_fields__.keys()
        c = {k: d[k] for k in keys if k in d}
        if "rope_theta" not in c and isinstance(d.get("rope_parameters"), dict):
            c["rope_theta"] = d["rope_parameters"].get("rope_theta", 1e6)
        if "head_dim" not in c:
            c["head_dim"] = d["hidden_size"] // d["num_attention_heads"]
        return cls(**c)

    def to_dict(self):
        return {k: v for k, v in asdict(self).items() if v is not None}

    @property
    def quantized(self):
        if self.weight_format != "bf16" and self.weight_format not in FORMATS:
            raise ValueError(f"unknown weight_format {self.weight_format!r}")
        return self.weight_format != "bf16"

    @property
    def widths(self):
        d = self.head_dim
        return (self.num_attention_heads * d, self.num_key_value_heads * d,
                self.num_key_value_heads * d)


# Benchmark shapes (random-init weights N(0, 0.02), RMSNorm gains 1).
SHAPES = {
    "tiny": dict(hidden_size=256, num_hidden_layers=2, num_attention_heads=4,
                 num_key_value_heads=2, head_dim=128, intermediate_size=384, vocab_size=97,
                 tie_word_embeddings=False),
    "qwen3-0.6b": dict(hidden_size=1024, num_hidden_layers=28, num_attention_heads=16,
                       num_key_value_heads=8, head_dim=128, intermediate_size=3072,
                       vocab_size=151936, tie_word_embeddings=True),
    "qwen3-4b": dict(hidden_size=2560, num_hidden_layers=36, num_attention_heads=32,
                     num_key_value_heads=8, head_dim=128, intermediate_size=9728,
                     vocab_size=151936, tie_word_embeddings=True),
    "qwen3-8b": dict(hidden_size=4096, num_hidden_layers=36, num_attention_heads=32,
                     num_key_value_heads=8, head_dim=128, intermediate_size=12288,
                     vocab_size=151936, tie_word_embeddings=False),
}


def shape_config(name, seed=0, std=0.02, **overrides):
    d = dict(SHAPES[name], rope_theta=1e6, rms_norm_eps=1e-6,
             random_init={"seed": seed, "std": std})
    d.update(overrides)
    return Qwen3Config.from_dict(d)


class Norm:
    """An RMSNorm gain with the attributes the fused ops read (.weight, .variance_epsilon)."""

    def __init__(self, weight, eps):
        self.weight = weight
        self.variance_epsilon = eps


class Layer:
    def __init__(self, config, index, device):
        c = config
        d = c.head_dim
        opts = dict(dtype=torch.bfloat16, device=device)
        self.layer_idx = index

        def weight(rows, cols):
            if c.quantized:
                return QuantizedWeight.empty(rows, cols, c.weight_format, device)
            return torch.empty((rows, cols), **opts)

        self.qkv_weight = weight(sum(c.widths), c.hidden_size)
        self.o_weight = weight(c.hidden_size, c.num_attention_heads * d)
        self.gate_up_weight = weight(2 * c.intermediate_size, c.hidden_size)
        self.down_weight = weight(c.hidden_size, c.intermediate_size)
        self.input_layernorm = Norm(torch.ones(c.hidden_size, **opts), c.rms_norm_eps)
        self.post_attention_layernorm = Norm(torch.ones(c.hidden_size, **opts), c.rms_norm_eps)
        self.q_norm = Norm(torch.ones(d, **opts), c.rms_norm_eps)
        self.k_norm = Norm(torch.ones(d, **opts), c.rms_norm_eps)

    def tensors(self):
        return {"qkv": self.qkv_weight, "o": self.o_weight, "gate_up": self.gate_up_weight,
                "down": self.down_weight}


class Qwen3Model:
    """Device-resident Qwen3 weights plus the config (the decode path's `model`)."""

    def __init__(self, config, device="cuda"):
        self.config = config
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.dtype = torch.bfloat16
        opts = dict(dtype=torch.bfloat16, device=self.device)
        c = config
        self.embed_weight = torch.empty((c.vocab_size, c.hidden_size), **opts)
        if c.quantized:
            # The LM head streams 8-bit rows; the gather table stays bf16 even when tied.
            self.lm_head_weight = QuantizedWeight.empty(c.vocab_size, c.hidden_size,
                                                        c.weight_format, self.device)
        else:
            self.lm_head_weight = (self.embed_weight if c.tie_word_embeddings
                                   else torch.empty((c.vocab_size, c.hidden_size), **opts))
        self.norm = Norm(torch.ones(c.hidden_size, **opts), c.rms_norm_eps)
        self.layers = [Layer(c, i, self.device) for i in range(c.num_hidden_layers)]

    @property
    def widths(self):
        return self.config.widths

    def weight_bytes(self):
        """Bytes of all weight tensors resident in HBM."""
        total = self.embed_weight.numel() * 2
        if self.lm_head_weight is not self.embed_weight:
            total += _nbytes(self.lm_head_weight)
        for layer in self.layers:
            total += sum(_nbytes(t) for t in layer.tensors().values())
        return total

    def decode_weight_bytes(self):
        """Weight bytes one decode step must read: every projection and the LM
        head once, plus the single embedding row and the norm gains."""
        c = self.config
        total = _nbytes(self.lm_head_weight) + c.hidden_size * 2 * 2
        for layer in self.layers:
            total += sum(_nbytes(t) for t in layer.tensors().values())
            total += (2 * c.hidden_size + 2 * c.head_dim) * 2
        return total

    # ------------------------------------------------------------------ init

    def randomize(self, seed=0, std=0.02):
        """Fill every projection with the seeded device generator; gains stay 1.

        bf16: N(0, std). 8-bit formats: uniform integers in [-127, 127] (fp8:
        their e4m3fn rounding) with row scales U(0.001, 0.01); the embedding
        table is N(0, std) bf16 either way.
        """
        rng.normal_(self.embed_weight, seed, STREAM_EMBED, std)
        if isinstance(self.lm_head_weight, QuantizedWeight):
            self.lm_head_weight.randomize_(seed, STREAM_LM_HEAD, STREAM_LM_HEAD_SCALE)
        elif self.lm_head_weight is not self.embed_weight:
            rng.normal_(self.lm_head_weight, seed, STREAM_LM_HEAD, std)
        for i, layer in enumerate(self.layers):
            for kind, t in layer.tensors().items():
                st = layer_stream(i, kind)
                if isinstance(t, QuantizedWeight):
                    t.randomize_(seed, st, st + SCALE_STREAM_OFFSET)
                else:
                    rng.normal_(t, seed, st, std)
        return self

    @classmethod
    def random(cls, config, seed=0, std=0.02, device="cuda"):
        return cls(config, device).randomize(seed, std)

    def load_state(self, tensors):
        """Copy Hugging Face-named tensors into the packed layouts (8-bit formats:
        quantized per row on the way in)."""
        with torch.no_grad():
            self.embed_weight.copy_(tensors["model.embed_tokens.weight"])
            if self.lm_head_weight is not self.embed_weight:
                _assign(self.lm_head_weight, tensors["lm_head.weight"])
            self.norm.weight.copy_(tensors["model.norm.weight"])
            for i, layer in enumerate(self.layers):
                p = f"model.layers.{i}."
                _assign(layer.qkv_weight, torch.cat([tensors[p + f"self_attn.{n}_proj.weight"]
                                                     for n in ("q", "k", "v")]))
                _assign(layer.o_weight, tensors[p + "self_attn.o_proj.weight"])
                _assign(layer.gate_up_weight, torch.cat([tensors[p + f"mlp.{n}_proj.weight"]
                                                         for n in ("gate", "up")]))
                _assign(layer.down_weight, tensors[p + "mlp.down_proj.weight"])
                layer.input_layernorm.weight.copy_(tensors[p + "input_layernorm.weight"])
                layer.post_attention_layernorm.weight.copy_(
                    tensors[p + "post_attention_layernorm.weight"])
                layer.q_norm.weight.copy_(tensors[p + "self_attn.q_norm.weight"])
                layer.k_norm.weight.copy_(tensors[p + "self_attn.k_norm.weight"])
        return self

    @classmethod
    def from_pretrained(cls, model_path, device="cuda"):
        """Load config.json plus safetensors shards, or random-init when the
        config carries {"random_init": {"seed": s, "std": sigma}}."""
        with open(os.path.join(model_path, "config.json")) as f:
            raw = json.load(f)
        config = Qwen3Config.from_dict(raw)
        model = cls(config, device)
        shards = sorted(glob.glob(os.path.join(model_path, "*.safetensors")))
        if shards:
            from safetensors.torch import load_file
            tensors = {}
            for shard in shards:
                tensors.update(load_file(shard, device="cpu"))
            if config.tie_word_embeddings:
                tensors.setdefault("lm_head.weight", tensors["model.embed_tokens.weight"])
            return model.load_state({k: v.to(torch.bfloat16) for k, v in tensors.items()})
        if config.random_init:
            r = config.random_init
            return model.randomize(int(r.get("seed", 0)), float(r.get("std", 0.02)))
        raise FileNotFoundError(f"{model_path}: no *.safetensors and no random_init in config.json")


def _assign(dst, src):
    if isinstance(dst, QuantizedWeight):
        q = QuantizedWeight.quantize(src.to(dst.device), dst.format)
        dst.data.copy_(q.data)
        dst.scale.copy_(q.scale)
    else:
        dst.copy_(src)


def write_random_model_dir(path, shape="qwen3-0.6b", seed=0, std=0.02, weight_format="bf16"):
    """Write a checkpoint directory whose weights are regenerated from the seed."""
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(shape_config(shape, seed, std, weight_format=weight_format).to_dict(), f,
                  indent=1)
    return path
