"""Pins of oracle/parity.py, the greedy-token comparison of the parity records.

margin() searches only the perturbation that raises the emitted logit and
lowers all others; a brute force over a grid of arbitrary perturbations of
small logit vectors checks that this is the optimal one (bf16 rounding is
monotone), and hand-worked cases check ties and the halfway rounding.
"""
import itertools
import random

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


def test_record_counts_and_bar():
    rec = OP.TokenRecord(2e-2)
    rec.add(0, torch.tensor([0.0, -1.0, 0.5]), 2)        # identical
    rec.add(1, torch.tensor([0.0, -0.015, -1.0]), 1)     # deficit 0.015 < bar
    rec.add(2, torch.tensor([0.0, -0.05, -1.0]), 1)      # deficit 0.05, margin 0.025
    s = rec.summary()
    assert (s["checked"], s["identical"], s["over_bar"]) == (3, 1, 1)
    assert abs(s["max_deficit"] - 0.05) < 1e-6
    assert s["deficit_over_1e-3"] == 2
