"""Pins of oracle/parity.py, the greedy-token comparison of the parity records.

margin() searches only the perturbation that raises the emitted logit and
lowers all others; a brute force over a grid of arbitrary perturbations of
small logit vectors checks that this is the optimal one (bf16 rounding is
monotone), and hand-worked cases check ties and the halfway rounding.
"""
import itertools
import random

import pytest
import torch

from oracle import parity as OP

BF16 = torch.bfloat16


def brute_force_margin(logits, token, step=1e-4, limit=0.05, grid=9):
    """Smallest delta on a grid such that SOME perturbation p with |p_i| <= delta
    (each p_i on a grid of `grid` values in [-delta, delta]) makes `token` the
    lowest-id argmax of the bf16-rounded logits."""
    lf = torch.tensor(logits, dtype=torch.float32)
    n = lf.numel()
    delta = 0.0
    while delta <= limit:
        values = torch.linspace(-delta, delta, grid) if delta > 0 else torch.zeros(1)
        for p in itertools.product(values.tolist(), repeat=n):
            moved = (lf + torch.tensor(p)).to(BF16).float()
            if int(torch.argmax(moved)) == token:
                return delta
        delta += step
    return None


def test_margin_matches_brute_force_over_all_perturbations():
    rng = random.Random(7)
    for _ in range(8):
        # Three logits within a few bf16 ulps of each other near 2.0 (ulp 1/64).
        base = 2.0 + rng.randrange(0, 8) / 64
        logits = [base + rng.uniform(-0.03, 0.03) for _ in range(3)]
        oracle = OP.greedy_bf16(torch.tensor(logits))
        for token in range(3):
            fast = OP.margin(torch.tensor(logits), token)
            slow = brute_force_margin(logits, token)
            if token == oracle:
                assert fast == 0.0 and slow == 0.0
                continue
            assert slow is not None
            # The grid search steps delta by 1e-4; margin is exact to ~1e-12.
            assert slow - 1e-4 - 1e-9 <= fast <= slow + 1e-9, (logits, token, fast, slow)


def test_halfway_rounding_tie_and_lowest_id():
    # 2 + 2^-7 is halfway between bf16 2.0 and 2.015625 and rounds to even
    # (2.0): both logits round to 2.0, a tie that the lowest id wins.
    logits = torch.tensor([2.0, 2.0078125])
    assert OP.greedy_bf16(logits) == 0
    assert OP.deficit(logits, 0) == 0.0078125
    assert OP.margin(logits, 0) == 0.0
    # Any upward push of id 1 leaves the halfway point and rounds up.
    assert 0.0 < OP.margin(logits, 1) < 1e-6
    # Reversed ids: id 1 holds 2.0 and ties with id 0 (2.0078125 rounds to
    # 2.0); a tie goes to id 0, so id 1 must round up to 2.015625, which takes
    # a push just past the halfway gap of 2^-7 (pushing id 0 below 1.99609375
    # would take 0.0117).
    rev = torch.tensor([2.0078125, 2.0])
    assert OP.greedy_bf16(rev) == 0
    assert 0.0078125 < OP.margin(rev, 1) < 0.0078125 + 1e-6


def test_margin_is_half_a_pairwise_gap_where_bf16_is_fine():
    # Near zero the bf16 grid is far finer than the gap: the margin is d / 2.
    for d in (1e-3, 4e-3, 1e-2):
        logits = torch.tensor([0.0, -d, -1.0])
        m = OP.margin(logits, 1)
        assert abs(m - d / 2) < 1e-4, (d, m)
        assert OP.deficit(logits, 1) == torch.tensor(d).item() or \
            abs(OP.deficit(logits, 1) - d) < 1e-9


def test_record_classifies_near_ties_noise_and_unexplained():
    rec = OP.TokenRecord()                                # the 1e-3 near-tie bar
    rec.add(0, torch.tensor([0.0, -1.0, 0.5]), 2)        # identical
    rec.add(1, torch.tensor([0.0, -0.0005, -1.0]), 1)    # deficit 5e-4: near-tie
    rec.add(2, torch.tensor([0.0, -0.02, -1.0]), 1)      # needs other orders
    rec.add(3, torch.tensor([0.0, -0.02, -1.0]), 1)
    rec.add(4, torch.tensor([0.0, -0.025, -1.0]), 1)
    assert rec.pending() == [2, 3, 4]
    # Unexamined steps count as unexplained.
    assert rec.summary()["unexplained"] == 3
    other = {
        0: torch.tensor([0.0, -1.0, 0.5]),
        1: torch.tensor([0.0, -0.0005, -1.0]),
        2: torch.tensor([-0.001, 0.0, -1.0]),   # another order picks token 1
        3: torch.tensor([0.0, -0.008, -1.0]),   # gaps 0.02 / 0.008: spread 0.012 >= 0.008
        4: torch.tensor([0.0, -0.015, -1.0]),   # gaps 0.025 / 0.015: spread 0.01 < 0.015
    }
    calls = []

    def order(step):
        calls.append(step)
        return other[step]

    s = rec.explain({"other": order}).summary()
    # Every step is evaluated once a step is pending; the other order's only
    # own flip (step 2, to token 1) has a primary deficit of 0.02, which
    # admits no step with a larger deficit.
    assert sorted(set(calls)) == [0, 1, 2, 3, 4]
    assert abs(s["sequence_noise"] - 0.02) < 1e-6
    assert (s["checked"], s["identical"], s["near_tie"], s["oracle_noise"],
            s["unexplained"]) == (5, 1, 1, 2, 1)
    assert abs(s["max_deficit"] - 0.025) < 1e-6
    kinds = {d["step"]: d["kind"] for d in s["differing_steps"]}
    assert kinds == {1: "near_tie", 2: "oracle_noise", 3: "oracle_noise", 4: "unexplained"}
    # Nothing pending: no order is evaluated.
    quiet = OP.TokenRecord()
    quiet.add(0, torch.tensor([0.0, -1.0]), 0)
    quiet.explain({"other": lambda step: pytest.fail("evaluated without need")})


def test_sequence_noise_admits_a_step_the_local_spread_does_not():
    """A flip whose orders agree closely at its own position is oracle noise
    when one of those orders itself flips, elsewhere on the sequence, to a
    token at least as far below the primary's argmax."""
    rec = OP.TokenRecord()
    primary = [torch.tensor([0.0, -0.02, -1.0]), torch.tensor([0.0, -0.03, -1.0]),
               torch.tensor([0.0, -0.5, -1.0])]
    other = [torch.tensor([0.0, -0.021, -1.0]),   # local spread 0.001 < 0.02
             torch.tensor([-0.01, 0.0, -1.0]),    # the order picks token 1 (deficit 0.03)
             torch.tensor([0.0, -0.5, -1.0])]
    for i, (l, t) in enumerate(zip(primary, (1, 0, 0))):
        rec.add(i, l, t)
    s = rec.explain({"other": lambda step: other[step]}).summary()
    assert abs(s["sequence_noise"] - 0.03) < 1e-6
    assert (s["oracle_noise"], s["unexplained"]) == (1, 0)
    # The same flip alone (the order never flips) stays unexplained.
    alone = OP.TokenRecord()
    alone.add(0, primary[0], 1)
    assert alone.explain({"other": lambda step: other[0]}).summary()["unexplained"] == 1


def test_near_tie_counts_the_bf16_rounding_of_the_decision():
    # 2.0 and 2.0078125 round to the same bf16 value: id 0 wins the tie, and
    # id 1, the fp32 maximum, has deficit 0: a near-tie whatever its margin.
    kind, details = OP.classify(torch.tensor([2.0, 2.0078125]), 1, {})
    assert kind == "near_tie" and details["deficit"] == 0.0
    # A fp32 gap of 0.01 between logits in different bf16 buckets is no tie.
    kind, _ = OP.classify(torch.tensor([2.01, 2.0]), 1, {})
    assert kind == "unexplained"


def test_orders_are_made_once_and_only_when_asked():
    made = []

    def maker():
        made.append(1)
        return torch.arange(12.0).view(4, 3)

    orders = OP.Orders(x=maker).callables(offset=2)
    assert made == []
    assert orders["x"](3).tolist() == [3.0, 4.0, 5.0]
    assert orders["x"](2).tolist() == [0.0, 1.0, 2.0]
    assert made == [1]
