"""Teacher-forced greedy-token parity records -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker of the HIP decode: nothing in the product path
imports it.

The reference's greedy head compares logits rounded to bf16 and takes the
lowest id among equal maxima (dryft/engine/kernels/greedy.py:3-4,27-29,41).
Two measures say how close the oracle's decision is to a tie, for a token g
that the HIP path emitted:

  deficit(l, g)   max_j l_j - l_g over the oracle's fp32 logits (0 when g is
                  the oracle's pick, or ties with it in fp32);
  margin(l, g)    the smallest delta such that some perturbation of the fp32
                  logits by at most delta per entry makes g the bf16 greedy
                  pick: g is raised by delta and every other logit lowered by
                  delta (the perturbation that helps g most), then the bf16
                  rule is applied. Because the rule rounds to bf16 (one ulp is
                  0.0156 for logits in [2, 4)), two logits that round alike
                  are tied whatever their fp32 gap, so margin <= deficit and
                  a flip across a bf16 rounding boundary has a small margin.

A differing token passes a bar b when its deficit is below b, or when its
margin is below b / 2: moving the two logits of a pair by d / 2 each closes a
gap of d, so a margin of b / 2 is the per-logit form of a pairwise gap b, with
the bf16 rounding of the decision rule taken into account.

The reference's own judge compares by the fp32 deficit with a 2.0-logit bar
(dryft/agent/benchmark_gpu.py:132-157).
"""
import torch

BF16 = torch.bfloat16


def greedy_bf16(logits):
    """argmax over bf16-rounded logits, lowest id on ties (greedy.py:41)."""
    return int(torch.argmax(logits.float().to(BF16).float()))


def deficit(logits, token):
    lf = logits.float()
    return max(0.0, float(lf.max() - lf[token]))


def _wins(lf, token, delta):
    moved = (lf - delta).to(BF16).float()
    moved[token] = (lf[token] + delta).to(BF16).float()
    return int(torch.argmax(moved)) == token


def margin(logits, token, iterations=48):
    """Smallest per-entry fp32 perturbation that makes `token` the bf16 greedy pick."""
    lf = logits.float().clone()
    if greedy_bf16(lf) == token:
        return 0.0
    lo, hi = 0.0, deficit(lf, token) + 1.0
    while not _wins(lf, token, hi):
        hi *= 2.0
    for _ in range(iterations):
        mid = 0.5 * (lo + hi)
        if _wins(lf, token, mid):
            hi = mid
        else:
            lo = mid
    return hi


class TokenRecord:
    """Per-step comparison of emitted tokens with the oracle's teacher-forced logits."""

    def __init__(self, bar):
        self.bar = bar
        self.steps = []

    def add(self, step, logits, token):
        oracle_token = greedy_bf16(logits)
        d = deficit(logits, token) if token != oracle_token else 0.0
        m = margin(logits, token) if token != oracle_token else 0.0
        self.steps.append(dict(step=step, token=int(token), oracle=oracle_token,
                               deficit=d, margin=m))

    def summary(self):
        diff = [s for s in self.steps if s["token"] != s["oracle"]]
        return {
            "checked": len(self.steps),
            "identical": len(self.steps) - len(diff),
            "deficit_over_1e-3": sum(s["deficit"] >= 1e-3 for s in diff),
            "margin_over_1e-3": sum(s["margin"] >= 1e-3 for s in diff),
            "over_bar": sum(s["deficit"] >= self.bar and s["margin"] >= self.bar / 2
                            for s in diff),
            "bar": self.bar,
            "max_deficit": max([s["deficit"] for s in diff], default=0.0),
            "max_margin": max([s["margin"] for s in diff], default=0.0),
            "differing_steps": [{k: (round(v, 6) if isinstance(v, float) else v)
                                 for k, v in s.items()} for s in diff],
        }

    def line(self, name):
        s = self.summary()
        return (f"{name}: {s['identical']}/{s['checked']} teacher-forced ids identical to the "
                f"oracle's; max deficit {s['max_deficit']:.4g}, max bf16 margin "
                f"{s['max_margin']:.4g}, deficits >= 1e-3: {s['deficit_over_1e-3']}, "
                f"margins >= 1e-3: {s['margin_over_1e-3']}, over the {self.bar:g} bar "
                f"(deficit >= bar and margin >= bar / 2): {s['over_bar']}")


def teacher_forced(oracle, prompt, tokens, bar, cache=None, timer=None):
    """Prefill `prompt` in one causal pass, then feed the emitted `tokens` one at
    a time; record how each emitted token compares with the oracle's logits.

    tokens[0] is the token emitted after the prompt, tokens[i] the one after
    tokens[i - 1]. `timer`, when a dict, receives "prefill_s" and "decode_s"
    (wall time of the prefill and of the len(tokens) - 1 decode steps).
    """
    import time
    from . import qwen3 as Q
    record = TokenRecord(bar)
    if cache is None:
        cache = Q.new_cache(oracle.shape, oracle.capacity)
    ids = torch.as_tensor(prompt, dtype=torch.int64).view(1, -1)
    t0 = time.perf_counter()
    _, lf, _ = oracle.forward(ids, cache, torch.arange(ids.shape[1]))
    t1 = time.perf_counter()
    record.add(0, lf[0, 0], tokens[0])
    for i in range(1, len(tokens)):
        pos = torch.tensor([ids.shape[1] + i - 1])
        _, lf, _ = oracle.forward(torch.tensor([[tokens[i - 1]]]), cache, pos)
        record.add(i, lf[0, 0], tokens[i])
    t2 = time.perf_counter()
    if timer is not None:
        timer["prefill_s"] = t1 - t0
        timer["decode_s"] = t2 - t1
    return record
