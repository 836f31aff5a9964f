"""Speculative decoding with a small draft model (batch one, greedy).

The reference speculates with prompt lookup only (dryft/engine/speculate.py);
this adds a draft model of the same vocabulary. One cycle:

  1. the draft's captured k-step graph decodes d1..dk greedily from the
     current token c at position p (each step feeds its own output back);
  2. the target's captured verify graph scores [c, d1..dk] at positions
     p .. p+k in one multi-row pass (k + 1 greedy predictions);
  3. verified_tokens (dryft/engine/speculate.py:55-69) keeps the matching
     prefix plus the target's correction or bonus token.

Greedy verification emits exactly the target's greedy tokens: a draft only
changes how many arrive per target pass. KV entries past the accepted prefix
are left in both caches; position-causal attention masks them and later
steps overwrite them. When all k drafts are accepted, the draft has not yet
consumed dk, so the next cycle first steps it on dk.
"""
import torch

from .decode import DecodeState
from .kernels.attention import check_xcd_merge
from .prefill import prefill
from .speculate import verified_tokens


class DraftSpeculator:
    def __init__(self, target, draft, prompt_length, output_length, draft_tokens=4):
        if target.config.vocab_size != draft.config.vocab_size:
            raise ValueError("draft and target models must share the vocabulary")
        if draft_tokens < 1:
            raise ValueError("draft_tokens must be at least 1")
        self.k = int(draft_tokens)
        self.target, self.draft = target, draft
        self.shape = (1, prompt_length, output_length)
        self.target_state = DecodeState(target, 1, prompt_length, output_length,
                                        speculative=True, draft_tokens=self.k)
        # The draft may run k + 1 slots past the last emitted position.
        self.draft_state = DecodeState(draft, 1, prompt_length, output_length + self.k + 1)
        self._capture_drafter()
        self.reset_stats()

    def _capture_drafter(self):
        ds = self.draft_state
        device = self.draft.device
        self.proposal = torch.zeros((self.k,), dtype=torch.int64, device=device)
        stream = torch.cuda.Stream(device=device)
        stream.wait_stream(torch.cuda.current_stream(device))
        # In inference mode, as DecodeState.capture (torch's shared graph RNG state).
        with torch.inference_mode(), torch.cuda.stream(stream):
            ds.position.fill_(self.shape[1])
            for i in range(self.k):
                ds.step(self.draft)
                self.proposal[i:i + 1].copy_(ds.token[0])
        torch.cuda.current_stream(device).wait_stream(stream)
        self.draft_graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(self.draft_graph, stream=stream):
            for i in range(self.k):
                ds.step(self.draft)
                self.proposal[i:i + 1].copy_(ds.token[0])

    def reset_stats(self):
        self.cycles = 0
        self.drafted = 0
        self.accepted = 0

    @property
    def acceptance(self):
        return self.accepted / self.drafted if self.drafted else 0.0

    def prefill(self, prompt):
        """Both models consume the prompt; returns the target's first token."""
        ids = torch.as_tensor(prompt, dtype=torch.int64, device=self.target.device).view(1, -1)
        first = int(prefill(self.target, self.target_state, ids)[0, 0])
        prefill(self.draft, self.draft_state, ids.to(self.draft.device))
        return first

    def cycle(self, current, position, catch_up=None):
        """One draft + verify cycle from token `current` at `position`.

        catch_up, when set, is the last accepted draft token the draft model
        has not consumed yet (it sits at position - 1). Returns the emitted
        tokens (1 .. k + 1).
        """
        ds, ts = self.draft_state, self.target_state
        if catch_up is not None:
            ds.token.fill_(catch_up)
            ds.position.fill_(position - 1)
            ds.graph.replay()
        ds.token.fill_(current)
        ds.position.fill_(position)
        self.draft_graph.replay()
        ts.verify_input[:, :1].fill_(current)
        ts.verify_input[0, 1:].copy_(self.proposal)
        ts.position.fill_(position)
        ts.verify_graph.replay()
        both = torch.cat((self.proposal, ts.verify_output[0])).tolist()
        proposal, predictions = both[:self.k], both[self.k:]
        emitted = verified_tokens(proposal, predictions)
        self.cycles += 1
        self.drafted += self.k
        self.accepted += len(emitted) - 1
        return emitted, proposal

    def generate(self, prompt, max_new_tokens):
        """Yield exactly max_new_tokens single-token lists (the target's greedy tokens)."""
        if max_new_tokens <= 0:
            return
        with torch.inference_mode():
            current = self.prefill(prompt)
            yield [current]
            yield from self.continue_from(current, len(prompt), max_new_tokens - 1)

    def _check_merge(self):
        check_xcd_merge(self.target.device)
        if self.draft.device != self.target.device:
            check_xcd_merge(self.draft.device)

    def continue_from(self, current, position, count):
        """Yield `count` more tokens after `current`, which sits at `position`
        (both caches hold every earlier position). The in-kernel attention
        merge's mismatch count is read after the first cycle and before the
        last tokens are yielded (kernels.attention.check_xcd_merge)."""
        with torch.inference_mode():
            emitted_count = 0
            catch_up = None
            cycles = 0
            while emitted_count < count:
                emitted, proposal = self.cycle(current, position, catch_up)
                cycles += 1
                if cycles == 1 or emitted_count + len(emitted) >= count:
                    self._check_merge()
                all_accepted = len(emitted) == self.k + 1
                catch_up = proposal[-1] if all_accepted else None
                position += len(emitted)
                for token in emitted[:count - emitted_count]:
                    emitted_count += 1
                    yield [token]
                current = emitted[-1]
