"""GPU: vxs_sample_noalloc (the entry point that allocates nothing; its staging lives in a fixed
device scratch) against vxs_sample on the same inputs, through the C ABI: ids identical, on two
calls in a row, the second smaller (a different shape, histories whose offsets do not start at 0,
a leading dimension above the vocabulary, strided params), then a call too large for the scratch,
which must fail cleanly and leave the next call working; a wide-vocabulary call (the streaming
kernel), and two contexts calling from two threads at once."""
import numpy as np
import pytest

from voxwerk_amd import workloads
from voxwerk_amd._lib import PARAMS_DTYPE, ptr

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20
ERR_UNSUPPORTED = -5


def reference(ctx, logits, vocab, params, stride, u, off=None, hist=None):
    rows = logits.shape[0]
    ids = np.full(rows, -98, np.int32)
    rc = ctx._lib.vxs_sample(ctx.handle, rows, vocab, ptr(logits), logits.shape[1], ptr(off), ptr(hist), ptr(params),
                             stride, ptr(u), ptr(ids), None, None, 0)
    return rc, ids


def test_noalloc_matches_sample_on_two_calls(ctx):
    # call 1: 1024 rows of the full-vocabulary batch (12 MiB of logits: the one-wave path)
    w = workloads.workload(4)
    b = w.generate(rows=1024)
    print(f"noalloc call 1: {b.rows} x {w.vocab}", flush=True)
    rc0, want = reference(ctx, b.logits, w.vocab, b.params, 1, b.u, b.hist_off, b.hist_ids)
    ids = np.full(b.rows, -99, np.int32)
    rc = ctx._lib.vxs_sample_noalloc(ctx.handle, b.rows, w.vocab, ptr(b.logits), w.vocab, ptr(b.hist_off),
                                     ptr(b.hist_ids), ptr(b.params), 1, ptr(b.u), ptr(ids), 0)
    assert rc == rc0 == 0, ctx.last_error()
    assert np.array_equal(ids, want)

    # call 2, smaller: 40 rows of 3000 entries in rows of 3072 floats, history offsets starting at
    # 17, params every second record, one row with an id outside the vocabulary
    rng = np.random.default_rng(12)
    rows, vocab, ld = 40, 3000, 3072
    x = np.zeros((rows, ld), np.float32)
    x[:, :vocab] = rng.standard_normal((rows, vocab)) * 2.0
    x[:, vocab:] = np.nan  # never read
    hl = rng.integers(0, 80, rows)
    off = (17 + np.concatenate([[0], np.cumsum(hl)])).astype(np.int32)
    hist = np.full(off[-1], -1, np.int32)
    hist[17:] = rng.integers(0, vocab, off[-1] - 17)
    bad = int(np.argmax(hl > 0) + 5) % rows
    p2 = np.zeros(2 * rows, dtype=PARAMS_DTYPE)
    p2["do_sample"] = 1
    p2["top_k"] = rng.choice([0, 50, 200], 2 * rows)
    p2["top_p"] = rng.choice([1.0, 0.9], 2 * rows).astype(np.float32)
    p2["temperature"] = np.float32(0.9)
    p2["rep_penalty"] = np.float32(1.1)
    p2["keep_id"], p2["ban_id"] = -1, -1
    if hl[bad] > 0:
        hist[off[bad]] = vocab
    u = rng.random(rows)
    print(f"noalloc call 2: {rows} x {vocab} (ld {ld})", flush=True)
    stride_params = np.ascontiguousarray(p2)  # records 0, 2, 4, ... used with stride 2
    want = np.full(rows, -98, np.int32)
    rc_w = ctx._lib.vxs_sample(ctx.handle, rows, vocab, ptr(x), ld, ptr(off), ptr(hist), ptr(stride_params), 2,
                               ptr(u), ptr(want), None, None, 0)
    ids = np.full(rows, -99, np.int32)
    rc = ctx._lib.vxs_sample_noalloc(ctx.handle, rows, vocab, ptr(x), ld, ptr(off), ptr(hist), ptr(stride_params), 2,
                                     ptr(u), ptr(ids), 0)
    assert rc == rc_w
    assert np.array_equal(ids, want)
    if hl[bad] > 0:
        assert ids[bad] == -2 and rc == -2


def test_noalloc_rejects_calls_beyond_the_scratch(ctx):
    rows, vocab = 1400, 3072  # 16.4 MiB of logits
    assert rows * vocab * 4 > SCRATCH_BYTES
    x = np.zeros((rows, vocab), np.float32)
    p = np.zeros((), dtype=PARAMS_DTYPE)
    p["keep_id"], p["ban_id"], p["rep_penalty"], p["temperature"] = -1, -1, 1.0, 1.0
    ids = np.full(rows, -99, np.int32)
    print("noalloc oversize call", flush=True)
    rc = ctx._lib.vxs_sample_noalloc(ctx.handle, rows, vocab, ptr(x), vocab, None, None, ptr(p), 0, None, ptr(ids), 0)
    assert rc == ERR_UNSUPPORTED
    assert "fixed scratch" in ctx.last_error()
    assert (ids == -99).all()
    # the next call works
    small = np.zeros((3, vocab), np.float32)
    small[:, 7] = 1.0
    ids = np.full(3, -99, np.int32)
    rc = ctx._lib.vxs_sample_noalloc(ctx.handle, 3, vocab, ptr(small), vocab, None, None, ptr(p), 0, None, ptr(ids), 0)
    assert rc == 0 and (ids == 7).all()


def test_noalloc_wide_vocabulary(ctx):
    """16 rows of the 151936-entry workload with 4096-id histories (about 9.8 MB staged): the
    streaming kernel reading its inputs from the fixed scratch."""
    w = workloads.workload(5)
    b = w.generate(rows=16)
    print(f"noalloc wide call: {b.rows} x {w.vocab}", flush=True)
    rc0, want = reference(ctx, b.logits, w.vocab, b.params, 1, b.u, b.hist_off, b.hist_ids)
    ids = np.full(b.rows, -99, np.int32)
    rc = ctx._lib.vxs_sample_noalloc(ctx.handle, b.rows, w.vocab, ptr(b.logits), w.vocab, ptr(b.hist_off),
                                     ptr(b.hist_ids), ptr(b.params), 1, ptr(b.u), ptr(ids), 0)
    assert rc == rc0 == 0, ctx.last_error()
    assert np.array_equal(ids, want)


def test_noalloc_two_contexts_two_threads(ctx):
    """Two contexts on one GPU calling from two threads at once, with inputs of different shapes:
    the per-device lock keeps the calls from overlapping in the shared scratch, so every call
    returns vxs_sample's ids."""
    import threading

    from voxwerk_amd.sampler import Context

    rng = np.random.default_rng(99)
    jobs = []
    for rows, vocab in ((512, 3072), (300, 2000)):
        x = (rng.standard_normal((rows, vocab)) * 2.0).astype(np.float32)
        off = (np.arange(rows + 1) * 30).astype(np.int32)
        hist = rng.integers(0, vocab, off[-1]).astype(np.int32)
        p = np.zeros(rows, dtype=PARAMS_DTYPE)
        p["do_sample"] = 1
        p["top_p"] = np.float32(0.9)
        p["temperature"] = np.float32(0.8)
        p["rep_penalty"] = np.float32(1.1)
        p["keep_id"], p["ban_id"] = -1, -1
        u = rng.random(rows)
        rc, want = reference(ctx, x, vocab, p, 1, u, off, hist)
        assert rc == 0
        jobs.append((x, vocab, off, hist, p, u, want))
    other = Context(0)
    calls = 40
    bad = []
    start = threading.Barrier(2)

    def run(c, job, tag):
        x, vocab, off, hist, p, u, want = job
        start.wait()
        for i in range(calls):
            ids = np.full(x.shape[0], -99, np.int32)
            rc = c._lib.vxs_sample_noalloc(c.handle, x.shape[0], vocab, ptr(x), vocab, ptr(off), ptr(hist), ptr(p), 1,
                                           ptr(u), ptr(ids), 0)
            if rc != 0 or not np.array_equal(ids, want):
                bad.append((tag, i, rc))

    print(f"noalloc two threads: {calls} calls each", flush=True)
    try:
        ts = [threading.Thread(target=run, args=(c, j, t)) for c, j, t in ((ctx, jobs[0], "a"), (other, jobs[1], "b"))]
        for t in ts:
            t.start()
        for t in ts:
            t.join(timeout=100)
        assert not any(t.is_alive() for t in ts), "a thread did not finish"
    finally:
        if not any(t.is_alive() for t in ts):
            other.close()
    assert not bad, bad[:5]
