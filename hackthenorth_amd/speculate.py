"""Prompt-lookup drafts and exact greedy verification (dryft/engine/speculate.py).

The acceptance rule is part of the output contract: a draft token is kept
only while it equals the target's greedy prediction, and exactly one target
token (the correction, or the bonus after a full match) follows the accepted
prefix (speculate.py:55-69).
"""

#: Draft width of the reference's verifier (speculate.py:3).
DRAFT_TOKENS = 7


def draft_width(output_length):
    """Verifier width for a request of output_length tokens (speculate.py:6-8)."""
    return max(0, min(DRAFT_TOKENS, output_length - 2))


class PromptLookup:
    """Propose the continuation of the most recent earlier occurrence of the
    last `ngram` tokens (speculate.py:11-33).

    The index maps each n-gram to the position right after its latest
    occurrence whose continuation of `draft_length` tokens is fully known;
    it is extended incrementally as tokens are appended.
    """

    def __init__(self, prompt, draft_length=DRAFT_TOKENS, ngram=4):
        self.tokens = list(prompt)
        self.draft_length = draft_length
        self.ngram = ngram
        self._indexed = 0          # occurrences starting before this are indexed
        self._after = {}

    def append(self, token):
        self.tokens.append(token)

    def propose(self):
        n, width = self.ngram, self.draft_length
        limit = len(self.tokens) - n - width + 1
        for start in range(self._indexed, limit):
            self._after[tuple(self.tokens[start:start + n])] = start + n
        self._indexed = max(self._indexed, limit)
        if len(self.tokens) < n:
            return None
        follow = self._after.get(tuple(self.tokens[-n:]))
        if follow is None:
            return None
        return self.tokens[follow:follow + width]


class BackoffPromptLookup:
    """Longest match first: 4-, then 3-, then 2-gram lookups (speculate.py:36-52)."""

    def __init__(self, prompt, draft_length=DRAFT_TOKENS):
        self.matchers = [PromptLookup(prompt, draft_length, n) for n in (4, 3, 2)]

    def append(self, token):
        for m in self.matchers:
            m.append(token)

    def propose(self):
        for m in self.matchers:
            proposal = m.propose()
            if proposal is not None:
                return proposal
        return None


def verified_tokens(proposal, predictions):
    """Accepted draft prefix plus one target token (speculate.py:55-69).

    predictions[i] is the target's greedy token after current + proposal[:i].
    """
    if len(predictions) != len(proposal) + 1:
        raise ValueError("verification needs one prediction per draft token plus a bonus")
    accepted = 0
    while accepted < len(proposal) and proposal[accepted] == predictions[accepted]:
        accepted += 1
    return list(predictions[:accepted + 1])
