"""Pins for the oracle's 8-bit weight-only restatement (no GPU).

The fp8 codec is checked against torch.float8_e4m3fn (a library routine), the
8-bit linear against the already-pinned bf16 linear and against exact
power-of-two scaling, and the generator's codes against the integer draws.
"""
import numpy as np
import pytest
import torch

from oracle import qwen3, rng


def test_e4m3_decode_matches_torch_for_every_code():
    codes = np.arange(256, dtype=np.uint8)
    ours = rng.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    assert np.isnan(ours).sum() == 2                       # 0x7f and 0xff only
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    assert ours[0x7e] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6


def test_e4m3_encode_matches_torch_rounding():
    ints = np.arange(-127, 128).astype(np.float32)
    x = np.concatenate([ints, np.random.default_rng(0).standard_normal(200_000)
                        .astype(np.float32) * 40,
                        # exact halfway points between grid neighbours (ties to even)
                        np.array([17.0, 19.0, 21.0, 35.0, 37.0, 0.0107421875], np.float32)])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    ours = rng.e4m3_encode(x)
    nz = rng.e4m3_decode(ref) != 0            # torch keeps the sign of zero; values agree
    assert np.array_equal(ours[nz], ref[nz])
    assert np.all(rng.e4m3_decode(ours[~nz]) == 0)


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3"])
def test_w8_codes_decode_to_the_integer_draws(fmt):
    draws = rng.int8_uniform(0, 123, 50_000)
    assert draws.min() == -127 and draws.max() == 127
    values = rng.w8_values(rng.w8_codes(0, 123, 50_000, fmt), fmt)
    if fmt == "int8":
        assert np.array_equal(values, draws.astype(np.float32))
    else:
        ref = torch.from_numpy(draws.astype(np.float32)).to(torch.float8_e4m3fn).float().numpy()
        assert np.array_equal(values, ref)
        # e4m3 keeps 4 significant bits: 0..16 exact, 127 rounds to 128.
        assert np.array_equal(values[np.abs(draws) <= 16], draws[np.abs(draws) <= 16])


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3"])
def test_w8_linear_unit_scale_is_the_bf16_linear(fmt):
    n, k = 48, 256
    values = torch.from_numpy(rng.w8_values(rng.w8_codes(3, 9, n * k, fmt), fmt)).reshape(n, k)
    bf = values.to(torch.bfloat16)
    assert torch.equal(bf.float(), values)   # every 8-bit value is exact in bf16
    x = qwen3.normal_bf16(1, 2, (3, k), 1.0)
    got = qwen3.linear_w8(x, values, torch.ones(n))
    assert torch.equal(got, qwen3.linear(x, bf))


def test_w8_linear_power_of_two_scales_commute_with_rounding():
    n, k = 64, 512
    values = torch.from_numpy(rng.w8_values(rng.w8_codes(5, 11, n * k, "int8"), "int8"))
    values = values.reshape(n, k)
    x = qwen3.normal_bf16(1, 4, (2, k), 1.0)
    exps = torch.arange(n) % 7 - 3
    scale = torch.pow(2.0, exps.float())
    got = qwen3.linear_w8(x, values, scale)
    base = qwen3.linear(x, values.to(torch.bfloat16)).float()
    assert torch.equal(got.float(), base * scale)            # per-row, not per-column
    # A plausible mistake -- scales applied along K -- fails.
    col_scale = scale.repeat(k // n)[None, :]
    wrong = qwen3.linear(x, (values * col_scale).to(torch.bfloat16))
    assert not torch.equal(got, wrong)


def test_w8_linear_matches_float64_within_half_ulp():
    n, k = 96, 1024
    values = torch.from_numpy(rng.w8_values(rng.w8_codes(2, 13, n * k, "fp8_e4m3"),
                                            "fp8_e4m3")).reshape(n, k)
    scale = torch.from_numpy(rng.uniform_f32(2, 14, n, 0.001, 0.01))
    x = qwen3.normal_bf16(1, 5, (1, k), 1.0)
    got = qwen3.linear_w8(x, values, scale).double()
    exact = (x.double() @ values.double().T) * scale.double()
    ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs())) - 7)
    assert torch.all((got - exact).abs() <= 0.5 * ulp * 1.001 + 1e-30)


def test_generate_weights_w8_layout():
    s = qwen3.SHAPES["tiny"]
    w = qwen3.generate_weights(s, weight_format="int8")
    assert w["0.qkv"].shape == (s.qkv_rows, s.hidden) and w["0.qkv.scale"].shape == (s.qkv_rows,)
    assert w["lm_head.scale"].shape == (s.vocab,)
    assert w["embed"].dtype == torch.bfloat16
    sc = w["1.down.scale"]
    assert float(sc.min()) >= 0.001 and float(sc.max()) < 0.01
    # Row scales come from their own stream, not the weight stream.
    assert not torch.equal(w["0.o.scale"][:8], w["0.qkv.scale"][:8])
