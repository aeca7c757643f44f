"""GPU: contexts used from several host threads at once (one context per thread, as the binding
documents), through the C ABI: every call's ids equal the same call made alone, for polled
single-row and small calls, staged larger calls and the streaming kernel, and every thread's own
resident history store ends as its host copy."""
import threading

import numpy as np
import pytest

from voxwerk_amd._lib import PARAMS_DTYPE
from voxwerk_amd.sampler import Context

pytestmark = pytest.mark.gpu


def _calls(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        vocab = int(rng.choice([2048, 3072, 9000]))
        rows = int(rng.choice([1, 3, 16, 300])) if vocab <= 3072 else int(rng.integers(1, 9))
        x = (rng.standard_normal((rows, vocab)) * 2.0).astype(np.float32)
        hl = rng.integers(0, 300, size=rows)
        off = np.zeros(rows + 1, np.int32)
        off[1:] = np.cumsum(hl)
        hist = rng.integers(0, vocab, size=int(off[-1])).astype(np.int32)
        p = np.zeros(rows, dtype=PARAMS_DTYPE)
        p["do_sample"] = 1
        p["top_k"] = rng.choice([0, 50], size=rows)
        p["top_p"] = rng.choice([1.0, 0.9], size=rows).astype(np.float32)
        p["temperature"] = np.float32(0.9)
        p["rep_penalty"] = np.float32(1.05)
        p["keep_id"], p["ban_id"] = -1, -1
        out.append((x, p, rng.random(rows), off, hist))
    return out


def _run(ctx, calls):
    return [ctx.sample(x, p, u, off, hist) for x, p, u, off, hist in calls]


def _store_run(ctx, seed, steps=12, rows=8, vocab=3072):
    rng = np.random.default_rng(seed)
    hist = [[] for _ in range(rows)]
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"], p["top_k"], p["temperature"], p["rep_penalty"] = 1, 50, np.float32(0.9), np.float32(1.05)
    p["top_p"], p["keep_id"], p["ban_id"] = np.float32(1.0), -1, -1
    ids_all = []
    with ctx.history(rows, steps + 1) as store:
        for _ in range(steps):
            x = (rng.standard_normal((rows, vocab)) * 2.0).astype(np.float32)
            ids = ctx.sample_batch(store, x, np.arange(rows, dtype=np.int32), p, rng.random(rows))
            ids_all.append(ids)
            for r in range(rows):
                hist[r].append(int(ids[r]))
        stored = [store.get(r).tolist() for r in range(rows)]
    return ids_all, stored == hist


def test_contexts_in_threads_match_calls_alone(ctx):
    threads_n, calls_n = 8, 40
    work = [_calls(100 + t, calls_n) for t in range(threads_n)]
    alone = [_run(ctx, w) for w in work]
    alone_store = [_store_run(ctx, 200 + t) for t in range(threads_n)]
    got, got_store, errors = [None] * threads_n, [None] * threads_n, []

    def worker(t):
        try:
            c = Context(0)
            try:
                got[t] = _run(c, work[t])
                got_store[t] = _store_run(c, 200 + t)
            finally:
                c.close()
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append((t, repr(e)))

    print(f"{threads_n} threads x {calls_n} calls", flush=True)
    ts = [threading.Thread(target=worker, args=(t,)) for t in range(threads_n)]
    for th in ts:
        th.start()
    for th in ts:
        th.join(timeout=120)
    assert not errors, errors
    for t in range(threads_n):
        assert got[t] is not None, f"thread {t} did not finish"
        for i, (a, b) in enumerate(zip(got[t], alone[t])):
            assert np.array_equal(a, b), f"thread {t} call {i}"
        ids_t, ok_t = got_store[t]
        assert ok_t, f"thread {t}: store differs from its host copy"
        for a, b in zip(ids_t, alone_store[t][0]):
            assert np.array_equal(a, b), f"thread {t}: batched stage"
