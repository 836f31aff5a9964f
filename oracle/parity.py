"""Teacher-forced greedy-token parity records -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker of the HIP decode: nothing in the product path
imports it.

The reference's greedy head compares logits rounded to bf16 and takes the
lowest id among equal maxima (dryft/engine/kernels/greedy.py:3-4,27-29,41).
The reference's judge replays the emitted sequence teacher-forced and checks
each position's emitted token against the replay's logits
(dryft/agent/benchmark_gpu.py:139-152; its bar is a 2.0-logit deficit).

Every emitted token g is compared with the oracle's logits l (the primary
evaluation order) at its position and classified:

  identical     g is the oracle's bf16 greedy pick;
  near_tie      deficit(l, g) < NEAR_TIE (1e-3), or margin(l, g) < NEAR_TIE / 2:
                the logits tie within 1e-3, counting the bf16 rounding of the
                decision rule;
  oracle_noise  the oracle itself, evaluated in another legitimate order (a
                token-by-token decode instead of one causal pass, float64
                instead of float32 arithmetic between the same bf16 roundings),
                picks g here; or the smallest gap l[a] - l[g] (a = the
                primary's fp32 argmax) over the orders is no larger than the
                orders' spread of that gap here (g is no farther from the
                nearest legitimate evaluation than those evaluations are from
                each other); or g's deficit is no larger than the largest
                deficit (against the primary) of a token that one of the
                other orders picks somewhere along the same sequence (the
                oracle itself emits tokens that far from the primary's
                argmax). The measured noise grows with depth: the oracle's
                own orders part at deficits of about 0.01 logits on the
                28-layer 0.6B shape and about 0.1 on the 36-layer 8B shape;
  unexplained   anything else. A parity check passes only with none.

  deficit(l, g)   max_j l_j - l_g over the fp32 logits (0 when g is the fp32 max);
  margin(l, g)    the smallest delta such that some perturbation of the fp32
                  logits by at most delta per entry makes g the bf16 greedy
                  pick: g is raised by delta and every other logit lowered by
                  delta (the perturbation that helps g most), then the bf16
                  rule is applied. Two logits that round to the same bf16 value
                  tie whatever their fp32 gap, so a flip across a bf16 rounding
                  boundary can have a margin far below its deficit, and a token
                  that is the fp32 argmax but loses the bf16 tie-break has a
                  deficit of 0 and a positive margin.
"""
import time

import torch

BF16 = torch.bfloat16
NEAR_TIE = 1e-3


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


def classify(logits, token, others, bar=NEAR_TIE, noise=0.0):
    """(class, details) of emitted `token` against primary `logits` and the
    logits of the same position in other evaluation orders (`others`: name ->
    logits, consulted only for a differing token outside the near-tie bar);
    `noise` is the largest deficit of a token the other orders pick along the
    sequence."""
    lf = logits.float()
    pick = greedy_bf16(lf)
    if token == pick:
        return "identical", {}
    d, m = deficit(lf, token), margin(lf, token)
    details = dict(oracle=pick, deficit=d, margin=m)
    if d < bar or m < bar / 2:
        return "near_tie", details
    top = int(torch.argmax(lf))
    gaps = {"primary": float(lf[top] - lf[token])}
    picks = {}
    for name, other in others.items():
        of = other.float()
        gaps[name] = float(of[top] - of[token])
        picks[name] = greedy_bf16(of)
    nearest = min(gaps.values())
    spread = max(gaps.values()) - nearest
    details.update(gaps=gaps, picks=picks, spread=spread, nearest=nearest,
                   sequence_noise=noise)
    if token in picks.values() or spread >= nearest or d <= noise:
        return "oracle_noise", details
    return "unexplained", details


def flip_deficit(logits, others):
    """The largest deficit, against the primary `logits`, of a token that an
    other evaluation order picks at the same position (0 if they all agree)."""
    pick = greedy_bf16(logits)
    worst = 0.0
    for other in others:
        p = greedy_bf16(other)
        if p != pick:
            worst = max(worst, deficit(logits, p))
    return worst


class TokenRecord:
    """Per-step comparison of emitted tokens with the oracle's teacher-forced logits.

    add() records a step against the primary logits; explain() supplies the
    other evaluation orders, which are computed only when some step needs
    them (a differing token outside the near-tie bar)."""

    def __init__(self, bar=NEAR_TIE):
        self.bar = bar
        self.steps = []
        self._logits = {}
        self.noise = None

    def add(self, step, logits, token):
        kind, details = classify(logits, int(token), {}, self.bar)
        # The primary logits are kept for the orders' noise estimate.
        self._logits[step] = logits.float().clone()
        if kind == "unexplained":
            kind = "pending"
        self.steps.append(dict(step=step, token=int(token), kind=kind, **details))

    def pending(self):
        return [s["step"] for s in self.steps if s["kind"] == "pending"]

    def explain(self, orders):
        """orders: name -> callable(step) -> logits of that step in that order.
        Invoked for every step when some step is pending (the orders' own
        flips along the sequence need them all), and not at all otherwise."""
        if not self.pending():
            return self
        self.noise = max(flip_deficit(self._logits[s["step"]],
                                      [fn(s["step"]) for fn in orders.values()])
                         for s in self.steps)
        for s in self.steps:
            if s["kind"] != "pending":
                continue
            others = {name: fn(s["step"]) for name, fn in orders.items()}
            kind, details = classify(self._logits[s["step"]], s["token"], others, self.bar,
                                     self.noise)
            s.update(kind=kind, **details)
        return self

    def summary(self):
        count = {k: sum(s["kind"] == k for s in self.steps)
                 for k in ("identical", "near_tie", "oracle_noise", "unexplained", "pending")}
        diff = [s for s in self.steps if s["kind"] != "identical"]
        return {
            "checked": len(self.steps),
            **count,
            # Steps no other evaluation order has looked at count as unexplained.
            "unexplained": count["unexplained"] + count["pending"],
            "bar": self.bar,
            "sequence_noise": self.noise,
            "max_deficit": max([s["deficit"] for s in diff], default=0.0),
            "max_margin": max([s["margin"] for s in diff], default=0.0),
            "differing_steps": [_rounded(s) for s in diff],
        }

    def line(self, name):
        s = self.summary()
        return (f"{name}: {s['identical']}/{s['checked']} ids identical to the oracle's, "
                f"{s['near_tie']} near-ties (< {self.bar:g}), {s['oracle_noise']} admitted "
                f"by the oracle's own evaluation orders, {s['unexplained']} unexplained; "
                f"max deficit {s['max_deficit']:.4g}, max bf16 margin {s['max_margin']:.4g}"
                + "".join(f"\n  step {d['step']}: {d}" for d in s["differing_steps"]))


def _rounded(value):
    if isinstance(value, float):
        return round(value, 6)
    if isinstance(value, dict):
        return {k: _rounded(v) for k, v in value.items()}
    return value


class Orders:
    """Lazily evaluated per-step logits of one emitted sequence in several
    orders: name -> maker() returning a [steps, V] tensor, made on first use."""

    def __init__(self, **makers):
        self._makers = makers
        self._made = {}

    def _get(self, name):
        if name not in self._made:
            self._made[name] = self._makers[name]()
        return self._made[name]

    def callables(self, offset=0):
        """name -> callable(step) for record steps numbered from `offset`."""
        return {name: (lambda step, n=name: self._get(n)[step - offset])
                for name in self._makers}


def sequence_orders(oracle, oracle64, prompt, tokens):
    """The other evaluation orders of a teacher-forced replay along `tokens`:
    the token-by-token decode (fp32) and the single causal pass in float64."""
    return Orders(stepwise=lambda: oracle.stepwise_logits(prompt, tokens),
                  float64=lambda: oracle64.teacher_forced_logits(prompt, tokens))


def teacher_forced(oracle, prompt, tokens, bar=NEAR_TIE, cache=None, timer=None):
    """Prefill `prompt` in one causal pass, then feed the emitted `tokens` one at
    a time; record how each emitted token compares with the oracle's logits.

    tokens[0] is the token emitted after the prompt, tokens[i] the one after
    tokens[i - 1]. `timer`, when a dict, receives "prefill_s" and "decode_s"
    (wall time of the prefill and of the len(tokens) - 1 decode steps).
    """
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
