"""GPU: batched sampling with device-resident histories (vxs_sample_batch / vxs_history_*), through the
C ABI, against the CSR-history call on the same inputs, the CPU oracle, and the unbatched loop.

Bar: resident-history ids identical to the CSR-history ids (same kernels, same arithmetic) and the
store identical to the host copy of every history; against the oracle, ids identical except counted
draw / top-p boundaries within 1e-6; batched generation frame-for-frame equal to unbatched generation
(tests/Voxwerk.Tests/TalkerParityTests.cs:125-147)."""
import numpy as np
import pytest

from oracle import ref
from talker_model import RecordingContext, SyntheticTalker
from voxwerk_amd._lib import PARAMS_DTYPE, VXS_ERR_HISTORY_FULL, VXS_ERR_INVALID_ARG
from voxwerk_amd.generate import BatchJob, generate, generate_batch
from voxwerk_amd.sampler import GenerationOptions, HistoryFull, SamplerError, SamplingOptions

pytestmark = pytest.mark.gpu


def _talker_rows(rows, vocab, rng):
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = rng.random(rows) < 0.8
    p["top_k"] = rng.choice([0, 1, 20, 50, 256, 300], size=rows)
    p["top_p"] = rng.choice([1.0, 0.95, 0.8, 0.3], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.7, 0.9, 1.0, 1.3], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.05, 1.3, 0.9, 1.0], size=rows).astype(np.float32)
    p["supp_begin"] = max(vocab - 1024, 0)
    p["supp_end"] = vocab
    p["keep_id"] = min(2150, vocab - 1)
    p["ban_id"] = -1
    return p


def _csr(lists):
    off = np.zeros(len(lists) + 1, np.int32)
    np.cumsum([len(h) for h in lists], out=off[1:])
    return off, np.array([i for h in lists for i in h], np.int32)


@pytest.mark.parametrize("vocab,rows,path", [(3072, 24, "auto"), (3072, 24, "wave"), (2048, 16, "block"),
                                             (8192, 8, "auto"), (151936, 4, "auto")])
def test_resident_history_matches_csr(ctx, vocab, rows, path):
    rng = np.random.default_rng(vocab + rows)
    steps = 10
    slots = rng.permutation(rows + 3)[:rows].astype(np.int32)  # not the identity, some slots unused
    params = _talker_rows(rows, vocab, rng)
    hist = [list(rng.integers(0, min(vocab, 2048), size=int(rng.integers(0, 40)))) for _ in range(rows)]
    print(f"vocab={vocab} rows={rows} path={path}", flush=True)
    with ctx.history(rows + 3, 64) as store:
        for r, s in enumerate(slots):
            store.set(int(s), hist[r])
        for t in range(steps):
            x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
            x[:, :64] += 4.0  # ids the histories hold get large logits, so the penalty decides draws
            u = rng.random(rows)
            off, ids = _csr(hist)
            want = ctx.sample(x, params, u, off, ids, path=path)
            got = ctx.sample_batch(store, x, slots, params, u, append=True, path=path)
            assert np.array_equal(got, want), f"step {t}: resident {got} vs CSR {want}"
            c = ref.classify(got, ref.sample(x, params, u, off, ids))
            assert c["unexplained"] == 0, f"step {t}: {c}"
            for r in range(rows):
                hist[r].append(int(got[r]))
        for r, s in enumerate(slots):
            assert store.get(int(s)).tolist() == hist[r], f"slot {s}"


def test_resident_history_without_append_and_empty_slots(ctx):
    rng = np.random.default_rng(3)
    rows, vocab = 6, 2048
    params = np.zeros(rows, dtype=PARAMS_DTYPE)
    params["do_sample"] = 1
    params["top_k"] = 50
    params["top_p"] = np.float32(0.9)
    params["temperature"] = np.float32(0.9)
    params["rep_penalty"] = np.float32(1.0)  # the code-predictor stage: no penalty, no history growth
    params["keep_id"] = params["ban_id"] = -1
    with ctx.history(rows, 8) as store:
        x = rng.standard_normal((rows, vocab)).astype(np.float32)
        u = rng.random(rows)
        got = ctx.sample_batch(store, x, np.arange(rows), params, u, append=False)
        assert np.array_equal(got, ctx.sample(x, params, u))
        assert all(store.get(s).size == 0 for s in range(rows))


def test_history_full_and_bad_slots(ctx):
    rows, vocab = 3, 1024
    x = np.zeros((rows, vocab), np.float32)
    x[:, 5] = 1.0
    greedy = np.zeros((), dtype=PARAMS_DTYPE)
    greedy["rep_penalty"] = np.float32(1.0)
    greedy["keep_id"] = greedy["ban_id"] = -1
    with ctx.history(4, 2) as store:
        store.set(1, [7, 8])  # full
        ids = ctx.sample_batch(store, x, [0, 1, 2], greedy, raise_on_error=False)
        assert ids.tolist() == [5, VXS_ERR_HISTORY_FULL, 5]
        assert store.get(1).tolist() == [7, 8] and store.get(0).tolist() == [5]
        with pytest.raises(HistoryFull):
            ctx.sample_batch(store, x, [0, 1, 2], greedy)
        with pytest.raises(SamplerError):
            ctx.sample_batch(store, x, [0, 0, 2], greedy)  # a slot twice
        with pytest.raises(SamplerError):
            ctx.sample_batch(store, x, [0, 4, 2], greedy)  # outside the store
        with pytest.raises(SamplerError):
            store.set(0, [1, 2, 3])  # longer than cap
        with pytest.raises(SamplerError):
            store.set(4, [])


def test_sample_batch_device_matches_host(ctx):
    from voxwerk_amd.hip import DeviceArray

    rng = np.random.default_rng(11)
    rows, vocab = 20, 3072
    params = _talker_rows(rows, vocab, rng)
    x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    u = rng.random(rows)
    slots = np.array(list(range(rows - 1)) + [rows + 5], np.int32)  # the last row names a bad slot
    hist = [list(rng.integers(0, 64, size=5)) for _ in range(rows)]
    with ctx.history(rows, 16) as hs, ctx.history(rows, 16) as dev_store:
        for r in range(rows - 1):
            hs.set(r, hist[r])
            dev_store.set(r, hist[r])
        host = ctx.sample_batch(hs, x[:-1], slots[:-1], params[:-1], u[:-1])
        dx, dp, du, ds = (DeviceArray.from_numpy(a) for a in (x, params, u, slots))
        dout = DeviceArray((rows,), np.int32)
        ctx.sample_batch_device(dev_store, rows, vocab, dx.ptr, vocab, ds.ptr, dp.ptr, 1, du.ptr, dout.ptr)
        ctx.synchronize()
        got = dout.numpy()
        assert np.array_equal(got[:-1], host)
        assert got[-1] == VXS_ERR_INVALID_ARG
        for r in range(rows - 1):
            assert np.array_equal(dev_store.get(r), hs.get(r))


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


@pytest.mark.parametrize("max_batch", [2, 5])
def test_generate_batch_equals_generate(ctx, max_batch):
    jobs = _jobs()
    model = SyntheticTalker(seed=5)
    rec = RecordingContext(ctx)
    done = {}
    generate_batch(jobs, max_batch, lambda j, f: done.__setitem__(j, f), model, context=rec)
    assert sorted(done) == list(range(len(jobs)))
    for j, job in enumerate(jobs):
        alone = generate(j, job.Options, model, context=ctx)
        assert len(done[j]) == len(alone), f"job {j}"
        for t, (a, b) in enumerate(zip(done[j], alone)):
            assert np.array_equal(a, b), f"job {j} frame {t}: batched {a} vs alone {b}"
    calls, rows, boundary = rec.check_against_oracle()
    print(f"max_batch={max_batch}: {calls} batched calls, {rows} rows vs oracle, {boundary} boundary rows", flush=True)


def _i32(x):
    return ((x + 0x80000000) & 0xFFFFFFFF) - 0x80000000


def test_device_generators_match_dotnet_random(ctx):
    """The slot generators drawn on the device reproduce the oracle's C restatement of .NET's seeded
    System.Random and the host DotNetRandom bit for bit, for new Random(seed) and new Random(seed + 1),
    over 20000 draws per generator taken in uneven pieces, wrapping seeds included."""
    from oracle import ref
    from voxwerk_amd.sampler import DotNetRandom

    seeds = [0, 1, 42, 161803397, 161803398, 161803399, 10**9, 2**31 - 1, -(2**31), -(2**31) + 1, -7,
             2_000_000_000, 123456789, -987654321]
    n = 20000
    with ctx.history(len(seeds), 4) as store:
        for s, seed in enumerate(seeds):
            store.seed(s, seed)
        for s, seed in enumerate(seeds):
            for stream, sd in (("talker", seed), ("sub", _i32(seed + 1))):
                want = ref.random_stream(sd, n)[1]
                got = np.concatenate([store.draw(s, stream, k) for k in (1, 199, 500, 4300, n - 5000)])
                assert np.array_equal(got.view(np.uint64), want.view(np.uint64)), (seed, stream)
                host = DotNetRandom(sd)
                first = np.array([host.NextDouble() for _ in range(700)])
                assert np.array_equal(first.view(np.uint64), want[:700].view(np.uint64)), (seed, stream)


def test_batch_draws_uniforms_on_device(ctx):
    from voxwerk_amd.sampler import DotNetRandom

    rng = np.random.default_rng(5)
    rows, vocab = 16, 3072
    params = _talker_rows(rows, vocab, rng)
    seeds = rng.integers(-2**31, 2**31, rows).tolist()
    slots = np.arange(rows, dtype=np.int32)[::-1].copy()
    host = [DotNetRandom(int(sd)) for sd in seeds]
    with ctx.history(rows, 16) as a, ctx.history(rows, 16) as b:
        for r in range(rows):
            b.seed(int(slots[r]), int(seeds[r]))
        with pytest.raises(SamplerError):
            ctx.sample_batch(a, np.zeros((rows, vocab), np.float32), slots, params, None, rng="talker")  # unseeded
        for t in range(6):
            x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
            u = np.array([host[r].NextDouble() if params["do_sample"][r] else 0.0 for r in range(rows)])
            want = ctx.sample_batch(a, x, slots, params, u)
            got = ctx.sample_batch(b, x, slots, params, None, rng="talker")
            assert np.array_equal(got, want), f"step {t}"
        for r in range(rows):  # greedy rows drew nothing
            nxt = b.draw(int(slots[r]), "talker", 3)
            assert nxt.tolist() == [host[r].NextDouble() for _ in range(3)], r


@pytest.mark.parametrize("max_batch", [2, 5])
def test_generate_batch_with_device_generators(ctx, max_batch):
    jobs = _jobs()
    model = SyntheticTalker(seed=9)
    done = {}
    generate_batch(jobs, max_batch, lambda j, f: done.__setitem__(j, f), model, context=ctx, device_rng=True)
    for j, job in enumerate(jobs):
        if job.Options.Seed is None and job.Options.Talker.DoSample:
            continue  # unseeded sampling: no fixed answer
        alone = generate(j, job.Options, model, context=ctx)
        assert len(done[j]) == len(alone), f"job {j}"
        for t, (a, b) in enumerate(zip(done[j], alone)):
            assert np.array_equal(a, b), f"job {j} frame {t}: device generators {a} vs host {b}"
