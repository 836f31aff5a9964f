"""Weight-only int8 / fp8-e4m3fn GEMVs and decode against the CPU oracle.

Bars: the device generator is bit-exact with numpy; a one-hot activation
reads back every 8-bit code exactly (the hardware fp8 decode is the OCP
e4m3fn one); projection outputs lie within one bf16 ulp of the oracle's
(both round the same fp32 dot product, summed in different orders) and
within the bf16 activation bar (max-abs 2e-2 + 2e-2 relative); argmax ids are
exact unless the oracle's top-2 gap is below 1e-3; the decode layers keep
the per-layer bar (cosine >= 0.9999) and teacher-forced greedy ids match.
"""
import numpy as np
import pytest
import torch

from oracle import qwen3 as Q
from oracle import rng as R
from hackthenorth_amd import decode as D
from hackthenorth_amd.kernels import greedy as G
from hackthenorth_amd.kernels import projection as P
from hackthenorth_amd.kernels.down import down_residual
from hackthenorth_amd.kernels.embed import embed_gather
from hackthenorth_amd.model import Qwen3Model, shape_config
from hackthenorth_amd.quant import QuantizedWeight

pytestmark = pytest.mark.gpu
FORMATS = ["int8", "fp8_e4m3"]


def nrm(stream, shape, std=1.0, seed=11):
    return Q.normal_bf16(seed, stream, shape, std)


def qweight(fmt, n, k, stream=40, seed=3):
    """(device QuantizedWeight, oracle float32 values, oracle scales) from the generator."""
    w = QuantizedWeight.empty(n, k, fmt, "cuda").randomize_(seed, stream, stream + 8)
    codes = R.w8_codes(seed, stream, n * k, fmt)
    assert np.array_equal(w.data.cpu().numpy().reshape(-1), codes)
    scale = R.uniform_f32(seed, stream + 8, n, 0.001, 0.01)
    assert np.array_equal(w.scale.cpu().numpy(), scale)
    return w, torch.from_numpy(R.w8_values(codes, fmt)).reshape(n, k), torch.from_numpy(scale)


def within_one_ulp(actual, expected):
    a = actual.detach().cpu().float().reshape(-1)
    e = expected.float().reshape(-1)
    ulp = torch.pow(2.0, torch.floor(torch.log2(e.abs().clamp_min(1e-30))) - 7)
    bad = (a - e).abs() > ulp
    assert not bool(bad.any()), (a[bad][:5], e[bad][:5])
    torch.testing.assert_close(a, e, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("fmt", FORMATS)
def test_device_w8_generator_matches_numpy(fmt):
    for count, stream in ((100_003, 5), (16, 6), (4097, 7)):
        t = QuantizedWeight.empty(1, count, fmt, "cuda").randomize_(9, stream, stream + 8)
        assert np.array_equal(t.data.cpu().numpy().reshape(-1), R.w8_codes(9, stream, count, fmt))
        assert np.array_equal(t.scale.cpu().numpy(), R.uniform_f32(9, stream + 8, 1, 0.001, 0.01))


@pytest.mark.parametrize("fmt", FORMATS)
def test_one_hot_activation_reads_every_code_exactly(fmt):
    k = 32
    codes = torch.arange(256, dtype=torch.uint8)
    data = codes[:, None].repeat(1, k).contiguous()
    w = QuantizedWeight(data.cuda(), torch.ones(256, device="cuda"), fmt)
    values = torch.from_numpy(R.w8_values(codes.numpy(), fmt))
    for j in (0, 5, 17, 31):
        x = torch.zeros(1, 1, k, dtype=torch.bfloat16)
        x[..., j] = 1
        y = P.projection(x.cuda(), w).cpu().float().reshape(-1)
        nan = torch.isnan(values)
        assert torch.equal(torch.isnan(y), nan)
        assert torch.equal(y[~nan], values[~nan])      # exact: every code is a bf16 value


W8_SHAPES = [(4096, 1024), (257, 2560), (40, 4096), (33, 12288), (1536, 4096), (31, 112),
             (100, 16)]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("n,k", W8_SHAPES)
def test_w8_gemv_family_matches_oracle(fmt, n, k):
    w, values, scale = qweight(fmt, 2 * n, k)
    top = QuantizedWeight(w.data[:n].contiguous(), w.scale[:n].contiguous(), fmt)
    x, g, res = nrm(11, (1, 1, k)), nrm(12, (k,)), nrm(13, (1, 1, n), std=30.0)
    xd, gd, rd = x.cuda(), g.cuda(), res.cuda()
    within_one_ulp(P.projection(xd, top), Q.linear_w8(x, values[:n], scale[:n]))
    normed = Q.rms_norm(x, g, 1e-6)
    gu = Q.linear_w8(normed, values, scale)
    within_one_ulp(P.norm_projection(xd, gd, w, 1e-6), gu)
    torch.testing.assert_close(P.norm_projection(xd, gd, w, 1e-6, swiglu=True).cpu().float(),
                               Q.silu_mul(gu[..., :n], gu[..., n:]).float(), atol=2e-2, rtol=2e-2)
    expected = (Q.linear_w8(x, values[:n], scale[:n]).float() + res.float()).to(torch.bfloat16)
    for out in (P.output_projection_residual(xd, top, rd), down_residual(xd, top, rd)):
        torch.testing.assert_close(out.cpu().float(), expected.float(), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("fmt", FORMATS)
def test_w8_greedy_head_matches_oracle_argmax(fmt):
    v, k = 151936, 1024
    w, values, scale = qweight(fmt, v, k, stream=60)
    gain = nrm(15, (k,))
    for i, std in enumerate((1.0, 3.0)):
        x = nrm(16 + i, (1, 1, k), std=std)
        xn = Q.rms_norm(x, gain, 1e-6)
        logits = (xn.float().reshape(-1) @ values.T) * scale
        out = torch.zeros(1, 1, dtype=torch.int64, device="cuda")
        position = torch.tensor([7], dtype=torch.int64, device="cuda")
        G.greedy_head(x.cuda(), gain.cuda(), 1e-6, w, out, position)
        expected = int(Q.greedy(logits.to(torch.bfloat16)))
        got = int(out)
        if got != expected:
            assert float(logits[expected] - logits[got]) < 1e-3
        assert int(position) == 8


def test_w8_rejects_unaligned_rows():
    w = QuantizedWeight(torch.zeros(4, 24, dtype=torch.uint8, device="cuda"),
                        torch.ones(4, device="cuda"), "int8")
    with pytest.raises(ValueError):
        P.projection(torch.zeros(1, 1, 24, dtype=torch.bfloat16, device="cuda"), w)


def _tiny(fmt, capacity):
    cfg = shape_config("tiny", seed=0, weight_format=fmt)
    model = Qwen3Model.random(cfg, seed=0)
    shape = Q.SHAPES["tiny"]
    oracle = Q.Oracle(shape, Q.generate_weights(shape, seed=0, weight_format=fmt), capacity)
    return model, oracle, shape


@pytest.mark.parametrize("fmt", FORMATS)
def test_w8_model_weights_equal_oracle_weights(fmt):
    model, oracle, _ = _tiny(fmt, 8)
    w = oracle.weights
    pairs = [(model.lm_head_weight, "lm_head")]
    for i, layer in enumerate(model.layers):
        pairs += [(t, f"{i}.{kind}") for kind, t in layer.tensors().items()]
    for q, name in pairs:
        assert torch.equal(torch.from_numpy(R.w8_values(q.data.cpu().numpy(), fmt)), w[name])
        assert torch.equal(q.scale.cpu(), w[name + ".scale"])
    assert torch.equal(model.embed_weight.cpu().view(torch.int16), w["embed"].view(torch.int16))


@pytest.mark.parametrize("fmt", FORMATS)
def test_w8_layers_and_teacher_forced_ids_match_oracle(fmt):
    prompt = Q.prompt_ids(12, 97, seed=1)
    steps = 20
    capacity = len(prompt) + steps
    model, oracle, shape = _tiny(fmt, capacity)
    tokens, _, _ = oracle.greedy_decode(prompt, steps)
    logits = oracle.teacher_forced_logits(prompt, tokens)
    with torch.inference_mode():
        # Per-layer bar on identical inputs at the last prompt token.
        cache = D.KVCache(model, 1, capacity)
        rotary = D.RotaryTable(model, capacity)
        for i, t in enumerate(prompt[:-1]):
            D.forward(model, torch.tensor([[t]], device="cuda"), cache,
                      torch.tensor([i], device="cuda"), rotary=rotary)
        ocache = Q.Cache(cache.storage[:, 0].cpu(), cache.storage[:, 1].cpu())
        last = len(prompt) - 1
        pos = torch.tensor([last], dtype=torch.int64, device="cuda")
        h = embed_gather(torch.tensor([prompt[-1]], device="cuda"), model.embed_weight)
        for layer in range(shape.layers):
            mine = D.decode_layer(model, layer, h, cache, pos, rotary)
            exp = oracle.layer(layer, h.cpu().view(1, 1, -1), ocache, torch.tensor([last]))
            a, e = mine.cpu().float().reshape(-1), exp.float().reshape(-1)
            cos = float(torch.nn.functional.cosine_similarity(a.double(), e.double(), dim=0))
            print(f"{fmt} layer {layer}: max|err|={float((a - e).abs().max()):.4g} "
                  f"max|h|={float(e.abs().max()):.4g} cos={cos:.7f}", flush=True)
            torch.testing.assert_close(a, e, atol=2e-2, rtol=2e-2)
            assert cos >= 0.9999
            h = mine
        # Teacher-forced ids through the captured decode graph.
        state = D.DecodeState(model, 1, len(prompt), steps)
        preds = [int(state.prefill(model, torch.tensor([prompt], device="cuda")))]
        forced = torch.tensor(tokens, dtype=torch.int64, device="cuda")
        for i in range(1, steps):
            state.token.copy_(forced[i - 1:i].view(1, 1))
            state.graph.replay()
            preds.append(int(state.token))
    for i, p in enumerate(preds):
        o = int(logits[i].to(torch.bfloat16).float().argmax())
        if p != o:
            assert float(logits[i].max() - logits[i][p]) < 2e-2, (i, p, o)
