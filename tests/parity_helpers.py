"""Shared parity checks of the GPU tests: per-element hidden-state bars in bf16
ulps, and teacher-forced token records explained against the oracle's own
evaluation orders (oracle/parity.py)."""
import torch

from oracle import parity as OP
from oracle import qwen3 as Q

# Per-element bar of a decoder layer's bf16 output against the oracle's on
# identical inputs, in bf16 ulps of max(|expected|, rms of the layer): one
# layer rounds to bf16 at seven boundaries, and a one-ulp flip at an early one
# (fp32 summation order decides it) moves the output by a few ulps of the
# terms it passes through; elements that cancel to below the layer's rms
# carry the ulps of the terms that cancelled. Measured on MI355X: at most 4
# ulps over the 8.4M outputs of a 2048-row 8B prefill layer, 3 elsewhere.
HIDDEN_ULPS = 6


def bf16_ulp(x):
    """One bf16 ulp at |x| (8 significant bits), for normal magnitudes."""
    mag = x.abs().clamp_min(2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(mag)) - 7)


def check_hidden(label, actual, expected, ulps=HIDDEN_ULPS):
    """|a - e| <= ulps bf16 ulps of max(|e|, rms(e)) for every element, and
    cosine >= 0.9999 (float64); prints the largest error and its 99.9th
    percentile in those units."""
    act = actual.detach().cpu().double().reshape(-1)
    exp = expected.detach().cpu().double().reshape(-1)
    rms = float(exp.square().mean().sqrt())
    unit = bf16_ulp(torch.maximum(exp.abs(), torch.full_like(exp, max(rms, 1e-30))))
    err = (act - exp).abs() / unit
    cos = float(torch.nn.functional.cosine_similarity(act, exp, dim=0))
    worst = int(err.argmax())
    print(f"{label}: max {float(err.max()):.3g} ulps (expected {float(exp[worst]):.5g}, got "
          f"{float(act[worst]):.5g}), 99.9th percentile {float(err.quantile(0.999)):.3g} ulps, "
          f"{int((err > 1).sum())} of {err.numel()} beyond 1 ulp, rms {rms:.4g}, "
          f"cos {cos:.7f}", flush=True)
    assert float(err.max()) <= ulps, label
    assert cos >= 0.9999, label


def check_record(record, label, orders=None):
    """Explain the record's differing steps with `orders` (name -> callable(step)
    -> logits) when it has any, print it, and require no unexplained step."""
    if orders is not None and record.pending():
        record.explain(orders)
    print(record.line(label), flush=True)
    summary = record.summary()
    assert summary["unexplained"] == 0, summary
    return summary


def record_sequence(oracle, prompt, tokens, label, logits=None, oracle64=None):
    """Teacher-forced record of one emitted sequence: the primary order is the
    oracle's single causal pass along prompt + tokens; differing steps are
    explained against its token-by-token decode and its float64 evaluation."""
    if logits is None:
        logits = oracle.teacher_forced_logits(prompt, tokens)
    record = OP.TokenRecord()
    for i, t in enumerate(tokens):
        record.add(i, logits[i], t)
    if oracle64 is None:
        oracle64 = Q.Oracle(oracle.shape, oracle.weights, oracle.capacity, acc=torch.float64)
    return check_record(record, label,
                        OP.sequence_orders(oracle, oracle64, prompt, tokens).callables())
