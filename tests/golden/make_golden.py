"""Write the committed golden fixtures from the CPU oracle.

  python tests/golden/make_golden.py            # all fixtures
  python tests/golden/make_golden.py tiny       # one of: tiny, 0.6b, ops

Fixtures hold only inputs and expected outputs; weights are regenerated from
the seed by the counter-based generator on both sides. The reference holds
no stored vectors for this path (its tests compare against live
transformers), so these are produced by the oracle, which
tests/test_oracle.py pins against the installed transformers Qwen3 on the
same weights and against the reference's literal known answers.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import qwen3 as Q  # noqa: E402
from oracle import rng  # noqa: E402


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def decode_fixture(name, shape_name, prompt_len, steps, record_steps, seed=0):
    shape = Q.SHAPES[shape_name]
    weights = Q.generate_weights(shape, seed=seed)
    prompt = Q.prompt_ids(prompt_len, shape.vocab)
    oracle = Q.Oracle(shape, weights, capacity=prompt_len + steps - 1)
    tokens, logits, records = oracle.greedy_decode(prompt, steps, record_steps=record_steps)
    gaps = []
    for lf in logits:
        top = torch.topk(lf, 2).values
        gaps.append(float(top[0] - top[1]))
    meta = dict(shape=shape_name, seed=seed, std=0.02, prompt_seed=1, prompt_stream=7,
                prompt=prompt, tokens=tokens, top2_gap_fp32=gaps,
                capacity=prompt_len + steps - 1)
    with open(os.path.join(HERE, f"{name}.json"), "w") as f:
        json.dump(meta, f)
    if record_steps:
        hidden = np.stack([np.stack([bits(h.reshape(-1)) for h in step]) for step in records])
        np.savez_compressed(os.path.join(HERE, f"{name}_hidden.npz"), hidden=hidden)
    print(name, tokens[:16], "min gap", min(gaps))


def ops_fixture():
    """Small per-op vectors (inputs from the counter RNG, outputs from the oracle)."""
    out = {}
    g = lambda stream, shape, std=1.0: Q.normal_bf16(3, stream, shape, std)  # noqa: E731
    x, r, gain = g(1, (4, 1024)), g(2, (4, 1024)), g(3, (1024,))
    s, n = Q.add_rms_norm(x, r, gain, 1e-6)
    out.update(add_x=x, add_r=r, add_gain=gain, add_sum=s, add_norm=n)
    w = g(4, (40, 1024), 0.02)
    xr = g(5, (1024,))
    out.update(proj_w=w, proj_x=xr, proj_y=Q.linear(xr, w))
    gu = g(6, (2 * 24, 1024), 0.02)
    normed = Q.rms_norm(xr, gain, 1e-6)
    y = Q.linear(normed, gu)
    out.update(swiglu_w=gu, swiglu_y=Q.silu_mul(y[:24], y[24:]))
    cos, sin = Q.rope_tables(16, 128, 1e6)
    qh = g(7, (1, 3, 4, 128))
    qn = g(8, (128,))
    out.update(rope_x=qh, rope_gain=qn, rope_out=Q.norm_rope(qh, qn, cos[[5, 9, 15]][None, :, None],
                                                              sin[[5, 9, 15]][None, :, None], 1e-6))
    np.savez_compressed(os.path.join(HERE, "ops.npz"), **{k: bits(v) for k, v in out.items()})
    print("ops", sorted(out))


def main(which):
    if which in ("all", "tiny"):
        decode_fixture("tiny_decode", "tiny", prompt_len=7, steps=24, record_steps=3)
    if which in ("all", "ops"):
        ops_fixture()
    if which in ("all", "0.6b"):
        decode_fixture("qwen3_0.6b_decode", "0.6b", prompt_len=32, steps=64, record_steps=2)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "all")
