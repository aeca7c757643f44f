"""The C restatement of .NET's seeded System.Random (oracle/vxs_oracle_random.c) pinned, and the
product's host generator (voxwerk_amd.sampler.DotNetRandom) checked against it bit for bit.

Pins: the published first values of new Random(0), new Random(1) and new Random(42) (recalled, not
produced by a .NET run: none is available here, so agreement with .NET itself stays "parity
unpinned"); the lagged-Fibonacci recurrence of Knuth's subtractive generator that every output after
the 55th obeys; seeds whose seeding wraps 32-bit arithmetic, and int.MinValue.
"""
import numpy as np
import pytest

from oracle import ref
from voxwerk_amd.sampler import DotNetRandom, _i32

MBIG = 2**31 - 1

# seeds around every special case: 0, negatives (|seed| is used), int.MinValue (Math.Abs would
# overflow: .NET uses int.MaxValue), MSEED and above (the seeding wraps), the largest seeds
WRAP_SEEDS = [0, 1, 42, -1, -42, 161803397, 161803398, 161803399, 10**9, 2 * 10**9, 2**31 - 1, -(2**31),
              -(2**31) + 1, 123456789, -987654321]


def test_published_first_values():
    assert ref.random_stream(0, 3)[0].tolist() == [1559595546, 1755192844, 1649316166]
    assert ref.random_stream(1, 1)[0][0] == 534011718
    assert ref.random_stream(42, 1)[0][0] == 1434747710


@pytest.mark.parametrize("seed", WRAP_SEEDS)
def test_lagged_recurrence(seed):
    """r[n] = (r[n-55] - r[n-34]) mod (2^31 - 1) for n >= 55: the table slot a draw overwrites was
    written 55 draws before, the slot 21 ahead of it 34 draws before. A wrong lag, cursor start or
    modulus breaks it."""
    s, d = ref.random_stream(seed, 20000)
    r = s.astype(np.int64)
    n = np.arange(55, r.size)
    assert np.array_equal(r[n], np.mod(r[n - 55] - r[n - 34], MBIG))
    assert s.min() >= 0 and s.max() < MBIG
    assert np.array_equal(d, s.astype(np.float64) * (1.0 / MBIG))


def test_negative_seed_uses_magnitude():
    assert np.array_equal(ref.random_stream(-5, 100)[0], ref.random_stream(5, 100)[0])
    assert np.array_equal(ref.random_stream(-(2**31), 100)[0], ref.random_stream(2**31 - 1, 100)[0])


@pytest.mark.parametrize("seed", WRAP_SEEDS)
def test_host_generator_matches_oracle(seed):
    """DotNetRandom (the product's host generator) against the C restatement, NextDouble bit for
    bit, for new Random(seed) and the code predictor's new Random(seed + 1) with C#'s wrap."""
    for sd in (seed, _i32(seed + 1)):
        g = DotNetRandom(sd)
        got = np.array([g.NextDouble() for _ in range(5000)])
        want = ref.random_stream(sd, 5000)[1]
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64)), sd


def test_long_stream_matches_oracle():
    rng = np.random.default_rng(2024)
    for sd in rng.integers(-2**31, 2**31, 3).tolist():
        g = DotNetRandom(int(sd))
        got = np.array([g.Next() for _ in range(100000)], np.int32)
        assert np.array_equal(got, ref.random_stream(int(sd), 100000)[0]), sd
