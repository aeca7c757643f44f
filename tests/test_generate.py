"""Host logic of the generation loops (voxwerk_amd/generate.py), run on the CPU oracle.

The invariant is the reference's batched-generation parity test (tests/Voxwerk.Tests/
TalkerParityTests.cs:125-147): every job of GenerateBatch yields the frames that Generate yields for
it alone, whatever the batch size, because each job keeps its own samplers and history."""
import numpy as np
import pytest

from talker_model import OracleContext, SyntheticTalker
from voxwerk_amd.generate import BatchJob, CancellationToken, OperationCanceledError, generate, generate_batch
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


def test_generate_on_frame_counts_frames():
    """onFrame(frames.Count) after every frame (TalkerGenerator.cs:277)."""
    ctx, model = OracleContext(), SyntheticTalker(seed=5)
    seen = []
    frames = generate(0, _jobs()[0].Options, model, context=ctx, on_frame=seen.append)
    assert seen == list(range(1, len(frames) + 1))


def test_generate_cancellation_stops_at_the_next_step():
    """ct.ThrowIfCancellationRequested() at the top of each step (TalkerGenerator.cs:243): cancelling from
    the frame callback ends the loop before the next talker Select."""
    ctx, model = OracleContext(), SyntheticTalker(seed=5)
    opts = _jobs()[0].Options
    full = generate(0, opts, model, context=ctx)
    assert len(full) >= 3
    ct = CancellationToken()
    seen = []

    def on_frame(n):
        seen.append(n)
        if n == 2:
            ct.cancel()

    with pytest.raises(OperationCanceledError):
        generate(0, opts, SyntheticTalker(seed=5), context=ctx, ct=ct, on_frame=on_frame)
    assert seen == [1, 2]
    with pytest.raises(OperationCanceledError):  # already cancelled: no step runs
        generate(0, opts, model, context=ctx, ct=ct)


def test_generate_batch_cancellation():
    """GenerateBatch checks the token once per step (TalkerGenerator.cs:332): jobs reported before the
    cancel keep their frames, the rest are never reported."""
    ctx, model = OracleContext(), SyntheticTalker(seed=1)
    jobs = _jobs()
    full = _run_batch(ctx, jobs, 2, model)
    ct = CancellationToken()
    done = {}

    def on_done(job, frames):
        done[job] = [f.copy() for f in frames]
        ct.cancel()

    with pytest.raises(OperationCanceledError):
        generate_batch(jobs, 2, on_done, SyntheticTalker(seed=1), context=ctx, ct=ct)
    assert len(done) >= 1 and len(done) < len(jobs)
    for j, frames in done.items():
        assert all(np.array_equal(a, b) for a, b in zip(frames, full[j])) and len(frames) == len(full[j])
