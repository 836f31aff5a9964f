"""Prompt-lookup drafts and exact greedy verification (dryft/engine/speculate.py).

The behaviour is the reference's contract, the one its tests pin
(dryft/tests/test_speculate.py:10-63): a lookup proposes the continuation
that followed the latest earlier occurrence of the current n-gram, counting
only occurrences whose whole continuation is already known, and a draft token
is kept only while it equals the target's greedy prediction, with exactly one
target token (correction or bonus) after the accepted prefix
(speculate.py:55-69).

The index here is maintained as tokens arrive: appending a token makes one
more occurrence old enough to have a full continuation, and that occurrence
(the newest of its n-gram) overwrites the n-gram's entry, so a proposal is one
dictionary lookup.
"""

#: Draft width of the reference's verifier (speculate.py:3).
DRAFT_TOKENS = 7


def draft_width(output_length):
    """Verifier width for a request of output_length tokens (speculate.py:6-8)."""
    return max(0, min(DRAFT_TOKENS, output_length - 2))


class PromptLookup:
    """n-gram prompt lookup over a growing token history (speculate.py:11-33).

    `_next[gram]` is the index right after the newest occurrence of `gram`
    that starts at least `ngram + draft_length` tokens before the end of the
    history, so its `draft_length` continuation tokens all exist.
    """

    def __init__(self, prompt, draft_length=DRAFT_TOKENS, ngram=4):
        self.ngram = ngram
        self.draft_length = draft_length
        self.tokens = []
        self._next = {}
        for token in prompt:
            self.append(token)

    def append(self, token):
        self.tokens.append(token)
        # The occurrence starting here has just become complete (n-gram plus
        # draft_length continuation tokens); a later one of the same n-gram
        # replaces it when it completes.
        start = len(self.tokens) - self.ngram - self.draft_length
        if start >= 0:
            gram = tuple(self.tokens[start:start + self.ngram])
            self._next[gram] = start + self.ngram

    def propose(self):
        """The draft (draft_length tokens) or None when the current n-gram has
        no complete earlier occurrence."""
        if len(self.tokens) < self.ngram:
            return None
        follow = self._next.get(tuple(self.tokens[-self.ngram:]))
        if follow is None:
            return None
        return self.tokens[follow:follow + self.draft_length]


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

    predictions[i] is the target's greedy token after current + proposal[:i];
    the first draft that differs from its prediction ends the accepted prefix,
    and that prediction is the correction (after a full match, the last
    prediction is the bonus). Predictions past a rejected draft were computed
    on tokens that will not be emitted and are dropped.
    """
    if len(predictions) != len(proposal) + 1:
        raise ValueError(f"{len(proposal)} draft tokens need {len(proposal) + 1} target "
                         f"predictions, got {len(predictions)}")
    for i, draft in enumerate(proposal):
        if predictions[i] != draft:
            return list(predictions[:i + 1])
    return list(predictions)
