"""GPU: a seeded randomised parity sweep (tests/sweep.py) over every path of the sampler against the
oracle: ids identical except counted boundary draws and cuts, probabilities within 1e-5 relative;
random logit-head calls within the fp32 bound of the exact product; and random sequences of batched
stages over a resident history store (ids, histories and device generators against the host's copy);
random batches through the one-wave kernel's statistics build (per-entry probabilities); and random
penalty and argmax host calls."""
import pytest

from sweep import batch_sweep, head_sweep, misc_sweep, stats_sweep, sweep

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", [101, 102, 103])
def test_random_sweep(ctx, seed):
    tot, bad = sweep(ctx, seed, batches=120, threads=8, log=lambda s: print(s, flush=True))
    print(f"seed {seed}: {tot}", flush=True)
    assert bad is None, f"seed {seed}: {bad} rows {bad.unexplained[:10]}"


def test_random_head_sweep(ctx):
    bad = head_sweep(ctx, 201, 80, log=lambda s: print(s, flush=True))
    assert not bad, bad[:3]


def test_random_batch_sequences(ctx):
    bad = batch_sweep(ctx, 301, 6, log=lambda s: print(s, flush=True))
    assert not bad, bad[:3]


def test_random_stats_batches(ctx):
    bad = stats_sweep(ctx, 401, 30, log=lambda s: print(s, flush=True))
    assert not bad, bad[:3]


def test_random_penalty_and_argmax_calls(ctx):
    bad = misc_sweep(ctx, 501, 40, log=lambda s: print(s, flush=True))
    assert not bad, bad[:3]
