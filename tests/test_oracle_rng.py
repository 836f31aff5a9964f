"""Pin the counter RNG the oracle and the HIP generator share."""
import numpy as np

from oracle import rng as R


def splitmix64_reference(z):
    """Textbook splitmix64 finaliser on Python ints (Steele, Lea, Flood 2014)."""
    m = (1 << 64) - 1
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def test_mix64_matches_the_textbook_finaliser():
    zs = [0, 1, 2, 0x9E3779B97F4A7C15, (1 << 64) - 1, 12345678901234567]
    got = R.mix64(np.array(zs, dtype=np.uint64))
    assert [int(g) for g in got] == [splitmix64_reference(z) for z in zs]
    # splitmix64 with state 0: first output is mix(golden) = 0xE220A8397B1DCDAF.
    assert int(R.mix64(np.array([0x9E3779B97F4A7C15], dtype=np.uint64))[0]) == 0xE220A8397B1DCDAF


def test_hash_counter_layout():
    key = R.stream_key(5, 9)
    assert int(key) == splitmix64_reference(5 ^ ((9 * 0xD1B54A32D192ED03) & ((1 << 64) - 1)))
    h = R.hashes(5, 9, 10, 3)
    for i in range(3):
        expect = splitmix64_reference((int(key) + (11 + i) * 0x9E3779B97F4A7C15) & ((1 << 64) - 1))
        assert int(h[i]) == expect


def test_normal_moments_and_range():
    v = R.normal_f32(0, 3, 1 << 20, std=0.02)
    assert abs(v.mean()) < 1e-4
    assert abs(v.std() - 0.02) < 2e-4
    assert np.abs(v).max() <= 0.02 * R.IH_MEAN / R.IH_STD + 1e-6
    # Fourth moment of Irwin-Hall(4): kurtosis 3 - 1.2/4 = 2.7.
    z = v / v.std()
    assert abs(float((z ** 4).mean()) - 2.7) < 0.02


def test_bf16_rounding_is_round_to_nearest_even():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0, -0.0, np.inf, 3.0e38],
                 dtype=np.float32)
    got = R.f32_to_bf16_bits(x)
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7 -> even (1.0); 1 + 3*2^-8 -> 1 + 2^-6.
    assert list(got) == [0x3F80, 0x3F80, 0x3F82, 0xC020, 0x0000, 0x8000, 0x7F80, 0x7F62]
    nan = R.f32_to_bf16_bits(np.array([np.nan], dtype=np.float32))
    assert (int(nan[0]) & 0x7F80) == 0x7F80 and (int(nan[0]) & 0x7F) != 0


def test_randint_and_int8_ranges():
    r = R.randint(1, 7, 100000, 151936)
    assert r.min() >= 0 and r.max() < 151936
    assert abs(r.mean() - 151935 / 2) < 151936 * 0.01
    q = R.int8_uniform(2, 3, 100000)
    assert q.min() == -127 and q.max() == 127
