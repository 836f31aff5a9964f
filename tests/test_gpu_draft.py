"""Draft-model speculation emits exactly the target's greedy tokens.

The target's plain captured decode is the reference sequence here, and
speculative runs must reproduce it id for id: on the tiny shape the verify
rows' multi-row kernels and the one-token kernels agree on every greedy pick.
(The comparison with the oracle's own greedy ids, with its near-tie bar, is
test_gpu_configs.test_draft_speculation_emits_oracle_greedy_ids.) Two drafts
cover both acceptance extremes: the target itself (nearly every draft
accepted, so the all-accepted catch-up path runs) and an unrelated model
(nearly none).
"""
import pytest
import torch

from hackthenorth_amd import decode as D
from hackthenorth_amd.draft import DraftSpeculator
from hackthenorth_amd.engine import Engine
from hackthenorth_amd.model import Qwen3Model, shape_config, write_random_model_dir
from oracle import qwen3 as Q

pytestmark = pytest.mark.gpu


def plain_tokens(model, prompt, steps):
    with torch.inference_mode():
        state = D.DecodeState(model, 1, len(prompt), steps)
        first = state.prefill(model, torch.tensor([prompt], device="cuda"))
        return [t[0] for t in D.stream_decode(state, first[:, 0].tolist(), steps)]


def first_divergence(actual, expected):
    """Index of the first differing id, or None when the lists are equal."""
    for i, (a, e) in enumerate(zip(actual, expected)):
        if a != e:
            return i
    assert len(actual) == len(expected)
    return None


@pytest.mark.parametrize("k", [1, 4])
def test_self_draft_accepts_and_matches_plain_decode(k):
    model = Qwen3Model.random(shape_config("tiny", seed=0), seed=0)
    prompt = Q.prompt_ids(11, 97, seed=1)
    steps = 40
    expected = plain_tokens(model, prompt, steps)
    spec = DraftSpeculator(model, model, len(prompt), steps, draft_tokens=k)
    got = [t[0] for t in spec.generate(prompt, steps)]
    assert len(got) == steps
    div = first_divergence(got, expected)
    assert div is None, (div, got, expected)
    assert spec.acceptance > 0.9, spec.acceptance
    # A second request on the same speculator resets nothing it should not.
    assert [t[0] for t in spec.generate(prompt, steps)] == got


def test_unrelated_draft_still_emits_target_tokens():
    target = Qwen3Model.random(shape_config("tiny", seed=0), seed=0)
    draft = Qwen3Model.random(shape_config("tiny", seed=5), seed=5)
    prompt = Q.prompt_ids(13, 97, seed=2)
    steps = 33
    expected = plain_tokens(target, prompt, steps)
    spec = DraftSpeculator(target, draft, len(prompt), steps, draft_tokens=4)
    got = [t[0] for t in spec.generate(prompt, steps)]
    assert got == expected
    assert spec.cycles > 0 and spec.drafted == 4 * spec.cycles


def test_engine_with_draft_model(tmp_path):
    target_dir = write_random_model_dir(str(tmp_path / "t"), "tiny", seed=0)
    draft_dir = write_random_model_dir(str(tmp_path / "d"), "tiny", seed=0)
    prompt = Q.prompt_ids(9, 97, seed=3)
    plain = [t[0] for t in Engine(target_dir, speculative=False).generate([prompt], 20)]
    eng = Engine(target_dir, draft_model_path=draft_dir, draft_tokens=4)
    out = [t[0] for t in eng.generate([prompt], 20)]
    assert out == plain
    for n in (1, 2, 6):
        assert len(list(eng.generate([prompt], n))) == n
