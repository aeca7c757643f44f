"""GPU: a seeded randomised parity sweep (tests/sweep.py) over every path of the sampler against the
oracle: ids identical except counted boundary draws and cuts, probabilities within 1e-5 relative."""
import pytest

from sweep import sweep

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", [101, 102, 103])
def test_random_sweep(ctx, seed):
    tot, bad = sweep(ctx, seed, batches=120, threads=8, log=lambda s: print(s, flush=True))
    print(f"seed {seed}: {tot}", flush=True)
    assert bad is None, f"seed {seed}: {bad} rows {bad.unexplained[:10]}"
