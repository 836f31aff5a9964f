"""State reset, rollback and generator boundaries, after the reference's own
tests (dryft/tests/test_prefill.py:27-61, dryft/tests/test_decode.py:117-203),
with the CPU oracle in place of native transformers:

  * a graphed prefill after the token, the position and every cache slot
    were corrupted (+-1000) equals the eager prefill bit for bit, restores the
    position and the decode stream, for (batch, prompt, output) = (2, 7, 6),
    (1, 1, 1) and (1, 12, 9);
  * a prompt of more than 2048 elements is prefilled eagerly (no graph);
  * the captured verify pass at every acceptance count 0..3 (a planted wrong
    draft token), the rollback, and the next step's token;
  * Engine.generate with prompt-lookup speculation at output lengths 1, 4, 5
    and 9 on repeated-token prompts, every token checked against the oracle;
  * a Qwen3-0.6B-shape self-draft at context 4096 (acceptance > 0, the
    all-accepted catch-up path at a real shape).

Token checks are teacher-forced records (oracle/parity.py): each id equal to
the oracle's pick, a near-tie within 1e-3, or explained by the oracle's own
evaluation orders.
"""
import pytest
import torch

from oracle import parity as OP
from oracle import qwen3 as Q
from oracle import rng as ORNG
from parity_helpers import check_record, record_sequence
from hackthenorth_amd import decode as D
from hackthenorth_amd.draft import DraftSpeculator
from hackthenorth_amd.engine import Engine
from hackthenorth_amd.model import Qwen3Model, shape_config, write_random_model_dir
from hackthenorth_amd.prefill import prefill
from hackthenorth_amd.speculate import verified_tokens

pytestmark = pytest.mark.gpu
TINY = Q.SHAPES["tiny"]


def tiny_model():
    return Qwen3Model.random(shape_config("tiny", seed=0), seed=0)


def random_ids(seed, shape):
    count = shape[0] * shape[1]
    return torch.tensor([int(v) for v in ORNG.randint(seed, 7, count, TINY.vocab)],
                        dtype=torch.int64).view(shape)


def check_greedy(oracle, prefixes, tokens, label):
    """Each token against the oracle's full-prefix greedy pick of its prefix."""
    record = OP.TokenRecord()
    logits = []
    for i, (prefix, token) in enumerate(zip(prefixes, tokens)):
        ids = torch.tensor([prefix])
        lf = oracle.forward(ids, Q.new_cache(TINY, len(prefix)), torch.arange(len(prefix)))[1]
        logits.append(lf[0, 0])
        record.add(i, lf[0, 0], token)
    o64 = Q.Oracle(TINY, oracle.weights, oracle.capacity, acc=torch.float64)

    def float64(step):
        prefix = prefixes[step]
        return o64.forward(torch.tensor([prefix]), Q.new_cache(TINY, len(prefix)),
                           torch.arange(len(prefix)))[1][0, 0]

    check_record(record, label, {"float64": float64})


@pytest.mark.parametrize("batch,length,output", [(2, 7, 6), (1, 1, 1), (1, 12, 9)])
def test_graphed_prefill_restores_corrupted_state(batch, length, output):
    model = tiny_model()
    with torch.inference_mode():
        eager = D.DecodeState(model, batch, length, output)
        graphed = D.DecodeState(model, batch, length, output)
        for repeat in range(3):
            ids = random_ids(40 + repeat, (batch, length)).cuda()
            for state in (eager, graphed):
                state.token.fill_(96)
                state.position.fill_(length + output + 7)
                for tensor in state.cache.keys + state.cache.values:
                    tensor.fill_(1000 if repeat % 2 else -1000)
            expected = eager.prefill(model, ids).clone()
            actual = prefill(model, graphed, ids)
            assert torch.equal(actual, expected)
            assert int(graphed.position) == length
            assert not graphed.cache.prefill
            assert hasattr(graphed, "prefill_graph")
            assert torch.equal(eager.cache.storage, graphed.cache.storage)
            for _ in range(output - 1):
                eager.graph.replay()
                graphed.graph.replay()
                assert torch.equal(graphed.token, eager.token)
                assert torch.equal(graphed.position, eager.position)


def test_prompt_over_2048_elements_is_prefilled_eagerly():
    model = tiny_model()
    with torch.inference_mode():
        ids = random_ids(50, (2, 1025)).cuda()
        state = D.DecodeState(model, 2, 1025, 1)
        expected = state.prefill(model, ids).clone()
        actual = prefill(model, state, ids)
        assert torch.equal(actual, expected)
        assert not hasattr(state, "prefill_graph")
    oracle = Q.Oracle(TINY, Q.generate_weights(TINY, seed=0), 1025)
    check_greedy(oracle, ids.cpu().tolist(), actual[:, 0].tolist(), "prefill of 2 x 1025")


def test_verify_at_every_acceptance_count_then_rollback():
    """dryft/tests/test_decode.py:117-167 on the captured verify graph: the
    proposal is the oracle's own greedy continuation with token `accept`
    replaced, so exactly `accept` drafts are accepted; the emitted tokens and
    the next step after the rollback are the oracle's greedy picks."""
    model = tiny_model()
    oracle = Q.Oracle(TINY, Q.generate_weights(TINY, seed=0), 20)
    prompt_len, k = 7, 3
    with torch.inference_mode():
        state = D.DecodeState(model, 1, prompt_len, 8, speculative=True, draft_tokens=k)
        assert state.verify_graph is not None
        for accept in range(k + 1):
            prompt = random_ids(60 + accept, (1, prompt_len))
            current = int(prefill(model, state, prompt.cuda())[0, 0])
            prefix = prompt[0].tolist() + [current]
            proposal, draft = [], list(prefix)
            for _ in range(k):
                ids = torch.tensor([draft])
                tok = int(oracle.forward(ids, Q.new_cache(TINY, len(draft)),
                                         torch.arange(len(draft)))[0])
                proposal.append(tok)
                draft.append(tok)
            if accept < k:
                proposal[accept] = (proposal[accept] + 1) % TINY.vocab
            # The eager multi-row pass and the captured verify graph agree.
            positions = torch.arange(prompt_len, prompt_len + k + 1, device="cuda")
            eager = D.forward(model, torch.tensor([[current, *proposal]], device="cuda"),
                              state.cache, positions, last_only=False,
                              rotary=state.rotary)[0].tolist()
            emitted = state.verify(current, proposal, prompt_len)
            assert emitted == verified_tokens(proposal, eager)
            assert len(emitted) == accept + 1, (accept, emitted, proposal, eager)
            assert int(state.position) == prompt_len + len(emitted)
            assert int(state.token[0, 0]) == emitted[-1]
            prefixes, tokens = [], []
            for token in emitted:
                prefixes.append(list(prefix))
                tokens.append(token)
                prefix.append(token)
            # Rollback: the next step overwrites the rejected slots' K/V.
            state.graph.replay()
            prefixes.append(list(prefix))
            tokens.append(int(state.token[0, 0]))
            check_greedy(oracle, prefixes, tokens, f"verify accepting {accept} of {k}")


@pytest.mark.parametrize("length", [1, 4, 5, 9])
def test_speculative_generator_lengths_on_repeated_prompts(tmp_path, length):
    """dryft/tests/test_decode.py:186-203: prompt lookup proposes from a
    repeated-token prompt, and every yielded token is the oracle's."""
    path = write_random_model_dir(str(tmp_path / "tiny"), "tiny", seed=0)
    engine = Engine(path, speculative=True)
    oracle = Q.Oracle(TINY, Q.generate_weights(TINY, seed=0), 12 + length)
    for token in (7, 11):
        prompt = [token] * 12
        outputs = list(engine.generate([prompt], length))
        assert len(outputs) == length and all(len(o) == 1 for o in outputs)
        # The reference's verifier width (speculate.py:6-8): none for <= 2 tokens.
        assert engine.state.draft_tokens == max(0, min(7, length - 2))
        record_sequence(oracle, prompt, [o[0] for o in outputs],
                        f"prompt lookup, [{token}] * 12, {length} tokens")


def test_0p6b_self_draft_at_context_4096():
    """A draft equal to the target accepts (nearly) every proposal, so the
    catch-up path (all k drafts accepted, the draft stepped on its last one)
    runs at a real shape, over a 4096-token prompt prefilled eagerly."""
    shape = Q.SHAPES["0.6b"]
    prompt_len, steps, k = 4096, 24, 4
    prompt = Q.prompt_ids(prompt_len, shape.vocab, seed=11)
    model = Qwen3Model.random(shape_config("qwen3-0.6b"))
    spec = DraftSpeculator(model, model, prompt_len, steps, draft_tokens=k)
    got = [t[0] for t in spec.generate(prompt, steps)]
    assert len(got) == steps
    print(f"0.6b self-draft at 4096: acceptance {spec.acceptance:.3f} over {spec.cycles} "
          f"cycles", flush=True)
    assert spec.acceptance > 0.5
    assert spec.cycles < steps - 1
    oracle = Q.Oracle(shape, Q.generate_weights(shape, seed=0), prompt_len + steps)
    record_sequence(oracle, prompt, got, "0.6b self-draft, context 4096")
