"""CPU restatement of the reference's batch-one Qwen3 decode -- TEST INFRASTRUCTURE ONLY.

This is the checker that the HIP library is compared against. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it; the
product path (hackthenorth_amd/) never does.

It restates, in plain PyTorch on the CPU, the torch-eager path the reference
runs: dryft/engine/decode.py:78-99 (forward: embed -> layers -> final norm on
the last row -> lm_head -> argmax) over the Qwen3 decoder layer of
transformers 4.51.3 (dryft/requirements.txt:11), with the bf16 rounding
boundaries the reference kernels keep:

  RMSNorm           dryft/engine/kernels/rmsnorm.py:64-81
                    y = bf16(gain * bf16(x * rsqrt(mean(x^2) + eps)))
  residual add      dryft/engine/kernels/rmsnorm.py:25-26   bf16(a + b)
  projection        dryft/engine/kernels/projection.py:25   bf16(sum fp32(x*w))
  O + residual      dryft/engine/kernels/projection.py:64-67 bf16(bf16(W a) + r)
  gate/up SwiGLU    dryft/engine/kernels/projection.py:26-32
                    bf16(bf16(silu(bf16 g)) * bf16 u)
  down + residual   dryft/engine/kernels/down.py:21-24       bf16(bf16(sum) + r)
  QK-norm + RoPE    dryft/engine/kernels/fused.py:17-30
                    n = bf16(g * bf16(x*inv)); out = bf16(bf16(n*cos) + bf16(rot(n)*sin))
  RoPE table        dryft/engine/decode.py:49-67 (the model's default rotary
                    module: inv_freq = 1/theta^(arange(0,D,2)/D) in fp32,
                    angle = fp32(pos * inv_freq), cos/sin rounded to bf16)
  attention         dryft/engine/kernels/attention.py:38-58 -- GQA, head h uses
                    kv head h // groups, scores fp32 scaled by D^-1/2, fp32
                    softmax over slots <= the query's absolute position, fp32
                    P.V, output rounded to bf16. The reference kernel also
                    rounds the block-relative exponentials to bf16 before P.V;
                    that rounding depends on its tiling and is covered by the
                    attention tolerance instead of being restated.
  greedy head       dryft/engine/kernels/greedy.py:27-29,41 and decode.py:99 --
                    logits rounded to bf16, argmax with the lowest id on ties.

8-bit weight-only variants (no reference counterpart: dryft decodes in bf16)
replace every projection and the LM head by y = bf16(s_n * sum_k x_k w_nk)
with exact int8 / fp8-e4m3fn weight values and fp32 row scales s_n; all other
roundings are unchanged.

The 8-bit linear is pinned in tests/test_oracle.py: with unit scales it
equals the bf16 linear of the same (bf16-exact) weight values, a scale
multiplies the output before the rounding (checked against a hand example),
and the generator's codes decode to the integer draws.

Parity pinned: tests/test_oracle.py checks this module against the installed
transformers Qwen3 implementation on identical weights (same formulas as
4.51.3), against hand-computed known answers copied from the reference tests
(halfway rounding, greedy tie, add_rms_norm sum), and against the
fixed-cache == full-prefix-recompute invariant of dryft/tests/test_decode.py:92-115.
"""
from dataclasses import dataclass, field

import numpy as np
import torch

from . import rng

BF16 = torch.bfloat16


@dataclass(frozen=True)
class Shape:
    hidden: int
    layers: int
    q_heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    tied: bool
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def qkv_rows(self):
        return (self.q_heads + 2 * self.kv_heads) * self.head_dim


SHAPES = {
    # Test-sized decoder with the real head width (the HIP kernels need D=128).
    "tiny": Shape(hidden=256, layers=2, q_heads=4, kv_heads=2, head_dim=128,
                  ffn=384, vocab=97, tied=False),
    "0.6b": Shape(hidden=1024, layers=28, q_heads=16, kv_heads=8, head_dim=128,
                  ffn=3072, vocab=151936, tied=True),
    "4b": Shape(hidden=2560, layers=36, q_heads=32, kv_heads=8, head_dim=128,
                ffn=9728, vocab=151936, tied=True),
    "8b": Shape(hidden=4096, layers=36, q_heads=32, kv_heads=8, head_dim=128,
                ffn=12288, vocab=151936, tied=False),
}

# Stream ids of the weight generator; the product's model loader uses the
# same ids so both sides regenerate identical weights from one seed.
STREAM_EMBED = 1
STREAM_LM_HEAD = 2
STREAM_LM_HEAD_SCALE = 3
SCALE_STREAM_OFFSET = 8
W8_FORMATS = ("int8", "fp8_e4m3")


def layer_stream(layer, kind):
    return 100 + 16 * layer + {"qkv": 0, "o": 1, "gate_up": 2, "down": 3}[kind]


def bf16_from_bits(bits, shape):
    return torch.from_numpy(bits.view(np.int16)).view(BF16).reshape(shape)


def normal_bf16(seed, stream, shape, std):
    count = int(np.prod(shape))
    return bf16_from_bits(rng.normal_bf16_bits(seed, stream, count, std), shape)


def w8_weight(seed, stream, scale_stream, shape, fmt):
    """(exact float32 weight values, float32 row scales U(0.001, 0.01))."""
    count = int(np.prod(shape))
    codes = rng.w8_codes(seed, stream, count, fmt)
    values = torch.from_numpy(rng.w8_values(codes, fmt)).reshape(shape)
    scale = torch.from_numpy(rng.uniform_f32(seed, scale_stream, shape[0], 0.001, 0.01))
    return values, scale


def generate_weights(shape, seed=0, std=0.02, weight_format="bf16"):
    """Random-init weights N(0, std) (Irwin-Hall approximation), gains 1.

    weight_format "int8" / "fp8_e4m3": the projections and the LM head are
    uniform integers in [-127, 127] (fp8: their e4m3fn rounding) held as exact
    float32 values, with row scales under "<name>.scale"; the embedding table
    stays N(0, std) bf16.
    """
    s = shape
    w = {"embed": normal_bf16(seed, STREAM_EMBED, (s.vocab, s.hidden), std)}
    if weight_format not in W8_FORMATS + ("bf16",):
        raise ValueError(weight_format)

    def put(name, stream, dims, scale_stream=None):
        if weight_format == "bf16":
            w[name] = normal_bf16(seed, stream, dims, std)
            return
        if scale_stream is None:
            scale_stream = stream + SCALE_STREAM_OFFSET
        w[name], w[name + ".scale"] = w8_weight(seed, stream, scale_stream, dims, weight_format)

    if s.tied and weight_format == "bf16":
        w["lm_head"] = w["embed"]
    else:
        put("lm_head", STREAM_LM_HEAD, (s.vocab, s.hidden), STREAM_LM_HEAD_SCALE)
    w["norm"] = torch.ones(s.hidden, dtype=BF16)
    for l in range(s.layers):
        put(f"{l}.qkv", layer_stream(l, "qkv"), (s.qkv_rows, s.hidden))
        put(f"{l}.o", layer_stream(l, "o"), (s.hidden, s.q_heads * s.head_dim))
        put(f"{l}.gate_up", layer_stream(l, "gate_up"), (2 * s.ffn, s.hidden))
        put(f"{l}.down", layer_stream(l, "down"), (s.hidden, s.ffn))
        for g in ("ln1", "ln2"):
            w[f"{l}.{g}"] = torch.ones(s.hidden, dtype=BF16)
        for g in ("q_norm", "k_norm"):
            w[f"{l}.{g}"] = torch.ones(s.head_dim, dtype=BF16)
    return w


# ---------------------------------------------------------------- per-op math

def rms_norm(x, gain, eps, acc=torch.float32):
    """dryft/engine/kernels/rmsnorm.py:64-81. `acc` is the arithmetic type
    between the bf16 roundings (float32 as the reference; float64 gives a
    second, independently rounded evaluation of the same formula)."""
    v = x.to(acc)
    inv = torch.rsqrt(v.square().mean(-1, keepdim=True) + eps)
    return (gain.to(acc) * (v * inv).to(BF16).to(acc)).to(BF16)


def add_rms_norm(x, residual, gain, eps):
    """dryft/engine/kernels/rmsnorm.py:16-32: (bf16 sum, rms_norm(sum))."""
    summed = (x.float() + residual.float()).to(BF16)
    return summed, rms_norm(summed, gain, eps)


def linear(x, weight):
    """bf16(sum fp32(x * w)) -- dryft/engine/kernels/projection.py:25."""
    return (x.float() @ weight.float().T).to(BF16)


def linear_w8(x, values, scale):
    """bf16(s_n * sum fp32(x * w)) for exact 8-bit weight values and fp32 row scales."""
    return ((x.float() @ values.float().T) * scale.float()).to(BF16)


def silu_mul(gate, up, acc=torch.float32):
    """dryft/engine/kernels/fused.py:160-168 and projection.py:26-32."""
    g = gate.to(acc)
    act = (g * torch.sigmoid(g)).to(BF16)
    return (act.to(acc) * up.to(acc)).to(BF16)


def output_residual(x, weight, residual):
    """dryft/engine/kernels/projection.py:56-67."""
    return (linear(x, weight).float() + residual.float()).to(BF16)


def rope_tables(capacity, head_dim, theta):
    """Default rotary embedding rows for positions 0..capacity-1 (decode.py:49-67)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64)
                                .float() / head_dim))
    positions = torch.arange(capacity, dtype=torch.int64).float()
    freqs = positions[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(BF16), emb.sin().to(BF16)


def norm_rope(x, gain, cos, sin, eps, acc=torch.float32):
    """Per-head RMSNorm then RoPE with rotate_half (kernels/fused.py:17-30).

    x [..., T, H, D]; cos/sin broadcastable to [..., T, 1, D].
    """
    n = rms_norm(x, gain, eps, acc).to(acc)
    half = x.shape[-1] // 2
    rot = torch.cat((-n[..., half:], n[..., :half]), dim=-1)
    left = (n * cos.to(acc)).to(BF16).to(acc)
    right = (rot * sin.to(acc)).to(BF16).to(acc)
    return (left + right).to(BF16)


def attention(q, keys, values, positions, acc=torch.float32):
    """GQA over a fixed-capacity cache (kernels/attention.py:13-63 semantics).

    q [B, Hq, Q, D] bf16; keys/values [B, Hkv, cap, D]; positions [Q] absolute.
    Slots after a query's position are never read (they may hold NaN).
    """
    d = q.shape[-1]
    groups = q.shape[1] // keys.shape[1]
    # Slots after the last query position are never touched (they may hold NaN).
    last = int(positions.max()) + 1
    k = keys[:, :, :last].to(acc).repeat_interleave(groups, dim=1)
    v = values[:, :, :last].to(acc).repeat_interleave(groups, dim=1)
    scores = (q.to(acc) @ k.transpose(-1, -2)) * (d ** -0.5)
    visible = torch.arange(last)[None, :] <= positions[:, None]
    scores = scores.masked_fill(~visible[None, None], float("-inf"))
    p = torch.softmax(scores, dim=-1)
    return (p @ v).to(BF16)


def greedy(logits_bf16):
    """Argmax over bf16 logits with the lowest id on ties (greedy.py:41)."""
    return torch.argmax(logits_bf16.float(), dim=-1)


# ---------------------------------------------------------------- model

@dataclass
class Cache:
    keys: torch.Tensor     # [L, B, Hkv, cap, D]
    values: torch.Tensor


def new_cache(shape, capacity, batch=1, fill=0.0):
    dims = (shape.layers, batch, shape.kv_heads, capacity, shape.head_dim)
    return Cache(torch.full(dims, fill, dtype=BF16), torch.full(dims, fill, dtype=BF16))


@dataclass
class Oracle:
    """The reference's forward over `weights`.

    `acc` is the arithmetic type between the bf16 rounding boundaries:
    float32, as the reference computes, or float64, which evaluates the same
    formula with every product and sum rounded differently (the roundings to
    bf16 stay where they are). The two give two legitimate evaluation orders
    of one model; where they pick different greedy tokens, the choice is
    within the formula's own rounding noise.
    """
    shape: Shape
    weights: dict
    capacity: int
    acc: torch.dtype = torch.float32
    cos: torch.Tensor = field(init=False)
    sin: torch.Tensor = field(init=False)
    f32: dict = field(init=False)

    def __post_init__(self):
        s = self.shape
        if self.acc not in (torch.float32, torch.float64):
            raise ValueError("acc must be torch.float32 or torch.float64")
        self.cos, self.sin = rope_tables(self.capacity, s.head_dim, s.theta)
        # fp32 copies of the bf16 weights: products of bf16 are exact in fp32.
        # The float64 evaluation converts each weight when it is used instead
        # (a resident copy would take four times the bf16 bytes).
        self.f32 = ({k: v.float() for k, v in self.weights.items() if v.dim() == 2}
                    if self.acc == torch.float32 else {})

    def _dot(self, x, name):
        """Dot products in `acc`, times the row scales of an 8-bit weight."""
        w = self.f32[name] if self.acc == torch.float32 else self.weights[name].to(self.acc)
        y = x.to(self.acc) @ w.T
        scale = self.weights.get(name + ".scale")
        return y if scale is None else y * scale.to(self.acc)

    def _linear(self, x, name):
        return self._dot(x, name).to(BF16)

    def layer(self, l, h, cache, positions):
        """Decoder layer l on hidden rows h [B, T, H] at absolute `positions`.

        Writes the layer's K/V for the new tokens into cache slots `positions`
        (decode.py:35-46) and returns the layer output [B, T, H].
        """
        s = self.shape
        w = self.weights
        b, t = h.shape[:2]
        d = s.head_dim
        acc = self.acc
        cos = self.cos[positions][None, :, None, :]      # [1, T, 1, D]
        sin = self.sin[positions][None, :, None, :]
        n = rms_norm(h, w[f"{l}.ln1"], s.eps, acc)
        qkv = self._linear(n, f"{l}.qkv")
        q, k, v = qkv.split((s.q_heads * d, s.kv_heads * d, s.kv_heads * d), -1)
        q = norm_rope(q.view(b, t, s.q_heads, d), w[f"{l}.q_norm"], cos, sin, s.eps, acc)
        k = norm_rope(k.view(b, t, s.kv_heads, d), w[f"{l}.k_norm"], cos, sin, s.eps, acc)
        v = v.reshape(b, t, s.kv_heads, d)
        cache.keys[l][:, :, positions] = k.transpose(1, 2)
        cache.values[l][:, :, positions] = v.transpose(1, 2)
        a = attention(q.transpose(1, 2), cache.keys[l], cache.values[l], positions, acc)
        a = a.transpose(1, 2).reshape(b, t, s.q_heads * d)
        r = (self._linear(a, f"{l}.o").to(acc) + h.to(acc)).to(BF16)
        m = rms_norm(r, w[f"{l}.ln2"], s.eps, acc)
        gu = self._linear(m, f"{l}.gate_up")
        act = silu_mul(gu[..., :s.ffn], gu[..., s.ffn:], acc)
        return (self._linear(act, f"{l}.down").to(acc) + r.to(acc)).to(BF16)

    def forward(self, ids, cache, positions, last_only=True, record=None, keep=None):
        """ids [B, T] int64, positions [T] absolute; returns (tokens, logits_f32, logits_bf16).

        Writes K/V of the new tokens into cache slots `positions` (decode.py:35-46).
        `record`, when a list, receives the bf16 hidden state after every layer.
        `keep` (with last_only=False) limits the head to the last `keep` rows.
        """
        s = self.shape
        w = self.weights
        h = w["embed"][ids]                              # [B, T, H]
        for l in range(s.layers):
            h = self.layer(l, h, cache, positions)
            if record is not None:
                record.append(h.clone())
        rows = h[:, -1:] if last_only else (h[:, -keep:] if keep else h)
        x = rms_norm(rows, w["norm"], s.eps, self.acc)
        logits = self._dot(x, "lm_head")
        logits_bf16 = logits.to(BF16)
        return greedy(logits_bf16), logits.float(), logits_bf16

    def greedy_decode(self, prompt, steps, record_steps=0):
        """Prefill the prompt, then `steps` greedy tokens (first from the prefill).

        Returns (tokens, per-step fp32 logits, per-step hidden-state records).
        """
        ids = torch.as_tensor(prompt, dtype=torch.int64).view(1, -1)
        p = ids.shape[1]
        cache = new_cache(self.shape, self.capacity)
        tokens, logits, records = [], [], []
        rec = [] if record_steps > 0 else None
        tok, lf, _ = self.forward(ids, cache, torch.arange(p), record=rec)
        if rec is not None:
            records.append([r[:, -1:] for r in rec])
        tokens.append(int(tok[0, 0]))
        logits.append(lf[0, 0])
        for step in range(1, steps):
            pos = torch.tensor([p + step - 1])
            rec = [] if step < record_steps else None
            tok, lf, _ = self.forward(torch.tensor([[tokens[-1]]]), cache, pos, record=rec)
            if rec is not None:
                records.append(rec)
            tokens.append(int(tok[0, 0]))
            logits.append(lf[0, 0])
        return tokens, logits, records

    def teacher_forced_logits(self, prompt, generated):
        """fp32 logits predicting each generated token, from one causal pass."""
        seq = list(prompt) + list(generated[:-1])
        ids = torch.tensor([seq], dtype=torch.int64)
        cache = new_cache(self.shape, max(self.capacity, len(seq)))
        _, lf, _ = self.forward(ids, cache, torch.arange(len(seq)), last_only=False,
                                keep=len(generated))
        return lf[0]

    def stepwise_logits(self, prompt, generated):
        """The same logits as teacher_forced_logits in another evaluation order:
        one causal pass over the prompt, then each generated token fed alone
        against the cache (the decode loop's order, decode.py:126-138)."""
        ids = torch.as_tensor(prompt, dtype=torch.int64).view(1, -1)
        p = ids.shape[1]
        cache = new_cache(self.shape, max(self.capacity, p + len(generated)))
        _, lf, _ = self.forward(ids, cache, torch.arange(p))
        out = [lf[0, 0]]
        for i in range(1, len(generated)):
            _, lf, _ = self.forward(torch.tensor([[int(generated[i - 1])]]), cache,
                                    torch.tensor([p + i - 1]))
            out.append(lf[0, 0])
        return torch.stack(out)


def prompt_ids(count, vocab, seed=1, stream=7):
    return [int(v) for v in rng.randint(seed, stream, count, vocab)]
