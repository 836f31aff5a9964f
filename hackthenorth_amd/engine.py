"""Engine(model_path).generate(input_ids, max_new_tokens) (dryft/engine/engine.py:175-249).

Contract (QWEN_ENGINE_CONTRACT.md:24-36 in the reference): generate yields
one list with one token id per sequence for every output step, exactly
max_new_tokens times, greedy, never stopping at end-of-sequence ids.
"""
import torch

from .decode import DecodeState, stream_decode
from .draft import DraftSpeculator
from .kernels.attention import XcdMergeError, check_xcd_merge
from .model import Qwen3Model
from .prefill import prefill
from .speculate import BackoffPromptLookup


class Engine:
    def __init__(self, model_path: str, speculative: bool = True, device="cuda",
                 draft_model_path: str = None, draft_tokens: int = 4) -> None:
        """Load config.json (+ safetensors, or the seeded random init) onto the GPU.

        speculative=False disables the batch-one prompt-lookup verifier, giving
        one decode step per output token. draft_model_path (same vocabulary)
        switches batch-one speculation from prompt lookup to a draft model
        proposing draft_tokens tokens per target verify pass.
        """
        if not torch.cuda.is_available():
            raise RuntimeError("Engine needs a HIP GPU")
        self.model = Qwen3Model.from_pretrained(model_path, device)
        self.draft = (Qwen3Model.from_pretrained(draft_model_path, device)
                      if draft_model_path else None)
        self.draft_tokens = draft_tokens
        self.speculative = speculative
        self.state = None
        self.speculator = None
        self.reset_stats()

    def reset_stats(self):
        """Counters of the batch-one prompt-lookup loop: verify passes, draft
        tokens proposed and accepted, and plain decode steps."""
        self.stats = {"verify_passes": 0, "proposed": 0, "accepted": 0, "decode_steps": 0}

    def generate(self, input_ids: list, max_new_tokens: int):
        """Yield max_new_tokens lists of one greedy token per sequence.

        The in-kernel attention merge assumes round-robin workgroup dispatch
        (checked when the library first runs on a device); every request
        also reads the merges' mismatch count after its second output and
        before its last (check_xcd_merge), and raises XcdMergeError, with the
        captured states dropped and the merge launch switched on, if a merge
        saw a split from another XCD.
        """
        if max_new_tokens <= 0:
            return
        device = self.model.device
        try:
            for i, tokens in enumerate(self._generate(input_ids, max_new_tokens)):
                if i == 1 or i == max_new_tokens - 1:
                    check_xcd_merge(device)
                yield tokens
        except XcdMergeError:
            self.state = None
            self.speculator = None
            raise

    def _generate(self, input_ids, max_new_tokens):
        if self.draft is not None and self.speculative and len(input_ids) == 1:
            shape = (1, len(input_ids[0]), max_new_tokens)
            if self.speculator is None or self.speculator.shape != shape:
                self.speculator = None
                self.speculator = DraftSpeculator(self.model, self.draft, shape[1], shape[2],
                                                  self.draft_tokens)
            yield from self.speculator.generate(input_ids[0], max_new_tokens)
            return
        with torch.inference_mode():
            shape = (len(input_ids), len(input_ids[0]), max_new_tokens)
            if self.state is None or self.state.shape != shape:
                self.state = None
                self.state = DecodeState(self.model, *shape, speculative=self.speculative)
            state = self.state
            prompt = torch.tensor(input_ids, dtype=torch.int64, device=self.model.device)
            current = prefill(self.model, state, prompt)
            tokens = current[:, 0].tolist()
            if state.draft_tokens == 0:
                self.stats["decode_steps"] += max_new_tokens - 1
                yield from stream_decode(state, tokens, max_new_tokens)
                return
            yield tokens
            lookup = BackoffPromptLookup(input_ids[0], draft_length=state.draft_tokens)
            lookup.append(tokens[0])
            emitted = 1
            while emitted < max_new_tokens:
                proposal = lookup.propose()
                if proposal:
                    verified = state.verify(tokens[0], proposal, shape[1] + emitted - 1)
                    self.stats["verify_passes"] += 1
                    self.stats["proposed"] += len(proposal)
                    self.stats["accepted"] += len(verified) - 1
                    # Scratch slots let a verify run at any position; emit only
                    # what the request still owes.
                    for token in verified[:max_new_tokens - emitted]:
                        tokens = [token]
                        lookup.append(token)
                        emitted += 1
                        yield tokens
                else:
                    state.graph.replay()
                    self.stats["decode_steps"] += 1
                    tokens = state.token[:, 0].tolist()
                    lookup.append(tokens[0])
                    emitted += 1
                    yield tokens
