"""Prompt lookup and acceptance: the reference's literal known answers
(dryft/tests/test_speculate.py:10-63), run against hackthenorth_amd.speculate."""
import random

import pytest

from hackthenorth_amd.speculate import (BackoffPromptLookup, PromptLookup, draft_width,
                                        verified_tokens)


def test_lookup_only_proposes_previously_seen_continuations():
    lookup = PromptLookup([1, 2, 3, 4, 5, 6, 7, 8, 1, 2, 3, 4], draft_length=3)
    assert lookup.propose() == [5, 6, 7]
    lookup.append(99)
    assert lookup.propose() is None


def test_lookup_learns_verified_output_without_self_matching():
    lookup = PromptLookup([1, 2], draft_length=3)
    assert lookup.propose() is None
    for token in [3, 4, 5, 6, 7, 1, 2, 3, 4]:
        lookup.append(token)
    assert lookup.propose() == [5, 6, 7]


def test_acceptance_emits_only_correct_prefix_and_one_target_token():
    proposal = [10, 11, 12]
    for accepted in range(4):
        predictions = proposal[:accepted] + [99] + [88] * (3 - accepted)
        assert verified_tokens(proposal, predictions) == proposal[:accepted] + [99]


def test_verification_requires_bonus_prediction():
    with pytest.raises(ValueError):
        verified_tokens([1, 2, 3], [1, 2, 3])


def test_backoff_prefers_longer_match_over_more_recent_short_match():
    history = [1, 2, 3, 4, 10, 11, 12, 9, 3, 4, 20, 21, 22, 1, 2, 3, 4]
    assert BackoffPromptLookup(history, draft_length=3).propose() == [10, 11, 12]


def test_backoff_uses_short_match_and_resets_for_new_prompt():
    first = BackoffPromptLookup([8, 9, 10, 11, 12, 1, 8, 9], draft_length=3)
    assert first.propose() == [10, 11, 12]
    assert BackoffPromptLookup([1, 8, 9]).propose() is None


@pytest.mark.parametrize("width", [3, 7])
def test_backoff_matches_naive_history_search_after_every_append(width):
    rng = random.Random(1701)
    history = [rng.randrange(5) for _ in range(24)]
    lookup = BackoffPromptLookup(history, draft_length=width)
    for _ in range(200):
        expected = None
        for ngram in (4, 3, 2):
            if len(history) < ngram:
                continue
            matches = [i for i in range(len(history) - ngram - width + 1)
                       if history[i:i + ngram] == history[-ngram:]]
            if matches:
                start = matches[-1] + ngram
                expected = history[start:start + width]
                break
        assert lookup.propose() == expected
        token = rng.randrange(5)
        history.append(token)
        lookup.append(token)


def test_draft_width_caps_short_requests():
    assert [draft_width(n) for n in (1, 2, 3, 5, 9, 100)] == [0, 0, 1, 3, 7, 7]
