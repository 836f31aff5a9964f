"""Host logic of the in-kernel attention merge's XCD guard, on the CPU with a
stubbed mismatch counter: check_xcd_merge switches the device to the merge
launch and raises; Engine.generate checks after its second output and before
its last, and drops its captured states on the error."""
import types

import pytest

from hackthenorth_amd import engine as E
from hackthenorth_amd.kernels import attention as A


def test_check_xcd_merge_disables_the_in_kernel_merge_then_raises(monkeypatch):
    calls = []
    monkeypatch.setattr(A, "xcd_merge_mismatches", lambda device=None, reset=False: 3)
    monkeypatch.setattr(A._lib, "call", lambda name, *args: calls.append(name))

    class _Device:
        def __init__(self, index):
            calls.append(("device", index))

        def __enter__(self):
            return self

        def __exit__(self, *exc):
            return False

    monkeypatch.setattr(A.torch.cuda, "device", _Device)
    with pytest.raises(A.XcdMergeError, match="3 in-kernel attention merges"):
        A.check_xcd_merge("cuda:0")
    assert calls == [("device", 0), "htn_attention_disable_in_kernel_merge"]


def test_check_xcd_merge_is_silent_at_zero(monkeypatch):
    monkeypatch.setattr(A, "xcd_merge_mismatches", lambda device=None, reset=False: 0)
    monkeypatch.setattr(A._lib, "call", lambda *a: pytest.fail("must not disable"))
    A.check_xcd_merge("cuda:0")


def _engine(outputs):
    engine = E.Engine.__new__(E.Engine)
    engine.model = types.SimpleNamespace(device="cuda:0")
    engine.state, engine.speculator = "captured", "captured"
    engine._generate = lambda ids, n: iter(outputs[:n])
    return engine


@pytest.mark.parametrize("n", [1, 2, 5])
def test_generate_checks_after_second_output_and_before_last(monkeypatch, n):
    seen = []
    engine = _engine([[i] for i in range(5)])
    emitted = []
    monkeypatch.setattr(E, "check_xcd_merge", lambda device: seen.append(len(emitted)))
    for tokens in engine.generate([[1, 2]], n):
        emitted.append(tokens)
    assert emitted == [[i] for i in range(n)]
    assert seen == sorted({1, n - 1} & set(range(n)))
    assert engine.state == "captured"


def test_generate_drops_captured_states_on_a_mismatch(monkeypatch):
    engine = _engine([[i] for i in range(5)])

    def mismatch(device):
        raise A.XcdMergeError("stub")

    monkeypatch.setattr(E, "check_xcd_merge", mismatch)
    gen = engine.generate([[1, 2]], 5)
    assert next(gen) == [0]
    with pytest.raises(A.XcdMergeError):
        next(gen)
    assert engine.state is None and engine.speculator is None
