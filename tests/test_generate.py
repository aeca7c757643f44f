"""Host logic of the generation loops (voxwerk_amd/generate.py), run on the CPU oracle.

The invariant is the reference's batched-generation parity test (tests/Voxwerk.Tests/
TalkerParityTests.cs:125-147): every job of GenerateBatch yields the frames that Generate yields for
it alone, whatever the batch size, because each job keeps its own samplers and history."""
import numpy as np
import pytest

from talker_model import OracleContext, SyntheticTalker
from voxwerk_amd.generate import BatchJob, generate, generate_batch
from voxwerk_amd.sampler import CODEC_EOS_ID, GenerationOptions, SamplingOptions


def _jobs():
    s = SamplingOptions
    return [
        BatchJob("a", GenerationOptions(MaxNewTokens=12, Seed=7)),
        BatchJob("b", GenerationOptions(MaxNewTokens=9, Seed=11, Talker=s(TopK=20, TopP=0.8, Temperature=1.2))),
        BatchJob("c", GenerationOptions(MaxNewTokens=10, Talker=s.Greedy(), SubTalker=s.Greedy())),
        BatchJob("d", GenerationOptions(MaxNewTokens=14, Seed=3, RepetitionPenalty=1.3,
                                        SubTalker=s(TopK=0, TopP=0.5, Temperature=0.7))),
        BatchJob("e", GenerationOptions(MaxNewTokens=6, Seed=99, Talker=s(TopK=3, TopP=1.0, Temperature=0.9))),
    ]


def _run_batch(ctx, jobs, max_batch, model):
    done = {}

    def on_done(job, frames):
        assert job not in done, f"job {job} reported twice"
        done[job] = [f.copy() for f in frames]

    generate_batch(jobs, max_batch, on_done, model, context=ctx)
    return done


@pytest.mark.parametrize("max_batch", [1, 2, 5, 8])
def test_generate_batch_equals_generate_on_the_oracle(max_batch):
    jobs = _jobs()
    ctx = OracleContext()
    model = SyntheticTalker(seed=5)
    done = _run_batch(ctx, jobs, max_batch, model)
    assert sorted(done) == list(range(len(jobs)))
    for j, job in enumerate(jobs):
        alone = generate(j, job.Options, model, context=ctx)
        assert len(done[j]) == len(alone), f"job {j}: {len(done[j])} frames batched, {len(alone)} alone"
        for t, (a, b) in enumerate(zip(done[j], alone)):
            assert np.array_equal(a, b), f"job {j} frame {t}: {a} vs {b}"
        assert len(alone) <= job.Options.MaxNewTokens - 1
        assert all(f.shape == (16,) and f[0] != CODEC_EOS_ID and f[0] < 2048 for f in alone)


def test_generate_batch_lengths_and_slots():
    jobs = _jobs()
    ctx = OracleContext()
    model = SyntheticTalker(seed=1)
    done = _run_batch(ctx, jobs, 2, model)
    lengths = [len(done[j]) for j in range(len(jobs))]
    assert any(n < jobs[j].Options.MaxNewTokens - 1 for j, n in enumerate(lengths)), "no job ended on EOS"
    assert any(n == jobs[j].Options.MaxNewTokens - 1 for j, n in enumerate(lengths)), "no job hit MaxNewTokens"
    assert model.calls["prefill"] == len(jobs)


def test_generate_batch_rejects_bad_batch():
    with pytest.raises(ValueError):
        generate_batch(_jobs(), 0, lambda j, f: None, SyntheticTalker(), context=OracleContext())
    generate_batch([], 4, lambda j, f: None, SyntheticTalker(), context=OracleContext())
