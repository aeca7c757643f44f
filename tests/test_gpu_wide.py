"""GPU parity of the streaming kernel for vocabularies above 8192: the wide workload (1024 rows x
151936, top-k 200, top-p 0.8, temperature 0.7, penalty over 4096 ids, suppression) and option mixes
that take its general multi-pass path (top-k off or above 256, ties, greedy, degenerate rows),
with write-back logits and probabilities against the CPU oracle."""
import numpy as np
import pytest

from oracle import ref
from parity import PROB_RTOL, comparable_rows, compare_ids, prob_rel_error, signed_zero_batch
from voxwerk_amd import workloads
from voxwerk_amd._lib import PARAMS_DTYPE

pytestmark = pytest.mark.gpu
U32 = np.uint32


def check_rows(ctx, logits, params, u=None, off=None, hist=None, label="", outputs=True):
    if outputs:
        ids, lg, pr = ctx.sample(logits, params, u, off, hist, want_logits=True, want_probs=True, raise_on_error=False)
    else:
        ids = ctx.sample(logits, params, u, off, hist, raise_on_error=False)
    ora = ref.sample(logits, params, u, off, hist, threads=8, want_logits=outputs, want_probs=outputs)
    rep = compare_ids(ids, ora)
    print(f"{label}: {rep}", flush=True)
    assert not rep.unexplained, f"{label}: ids differ at rows {rep.unexplained[:10]}"
    if outputs:
        ok = ids >= 0
        assert np.array_equal(lg[ok].view(U32), ora["logits"][ok].view(U32)), f"{label}: write-back logits differ"
        rel = prob_rel_error(pr, ora["probs"], comparable_rows(ids, ora) & ok)
        assert rel <= PROB_RTOL, f"{label}: probability relative error {rel:.3e}"
    return ids, ora


def test_wide_workload(ctx):
    """The full 1024-row batch the wide-vocabulary throughput figure is measured on."""
    w = workloads.workload(5)
    b = w.generate()
    assert b.rows == 1024
    print(f"{w.name} rows={b.rows} vocab={w.vocab} digest={b.digest()[:16]}", flush=True)
    check_rows(ctx, b.logits, b.params, b.u, b.hist_off, b.hist_ids, label=w.name, outputs=False)


def test_wide_workload_outputs(ctx):
    w = workloads.workload(5)
    b = w.generate(rows=16)
    check_rows(ctx, b.logits, b.params, b.u, b.hist_off, b.hist_ids, label=w.name + " outputs")


@pytest.mark.parametrize("vocab", [8193, 20000, 151936])
def test_wide_option_mixes(ctx, vocab):
    rng = np.random.default_rng(3000 + vocab)
    rows = 24
    logits = (rng.standard_normal((rows, vocab)) * rng.choice([0.5, 2.0, 4.0], size=(rows, 1))).astype(np.float32)
    logits[:, :50] += 4.0
    logits[3] = np.round(logits[3])  # many ties
    hl = rng.integers(0, 600, size=rows)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = rng.integers(0, vocab, size=off[-1]).astype(np.int32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["do_sample"][::6] = 0
    p["top_k"] = rng.choice([0, 1, 50, 200, 256, 257, 1000], size=rows)
    p["top_p"] = rng.choice([1.0, 0.95, 0.8, 0.3, 1e-6], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.7, 1.0, 1.3], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.05, 1.1], size=rows).astype(np.float32)
    supp = rng.random(rows) < 0.4
    p["supp_begin"] = np.where(supp, vocab - 1024, 0)
    p["supp_end"] = np.where(supp, vocab, 0)
    p["keep_id"] = np.where(supp, vocab - 1024 + 102, -1)
    p["ban_id"] = -1
    check_rows(ctx, logits, p, rng.random(rows), off, hist, label=f"wide mixed V={vocab}")


def test_wide_special_rows(ctx):
    vocab = 40000
    rows = 8
    x = np.full((rows, vocab), -1.0, np.float32)
    x[0] = -np.inf                    # all masked: V-1
    x[1] = 0.5                        # uniform: top-k ties, top-p by index order
    x[2, 123] = np.nan                # rejected
    x[3, 7] = 3.0
    x[3, 39999] = 3.0                 # tied maxima
    x[4] = np.linspace(-5, 5, vocab).astype(np.float32)
    x[5, ::2] = -np.inf
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = [1, 1, 1, 1, 1, 1, 0, 1]
    p["top_k"] = [50, 100, 0, 0, 0, 300, 0, 1]
    p["top_p"] = [1.0, 0.5, 1.0, 1e-7, 0.9, 0.9, 1.0, 1.0]
    p["temperature"] = 1.0
    p["rep_penalty"] = 1.0
    p["keep_id"] = -1
    p["ban_id"] = -1
    ids, ora = check_rows(ctx, x, p, np.linspace(0.05, 0.95, rows), label="wide special")
    assert ids[0] == vocab - 1 and ids[2] == -3 and ids[3] == 39999


def test_wide_penalty_only(ctx):
    rng = np.random.default_rng(77)
    vocab = 151936
    x = rng.standard_normal((4, vocab)).astype(np.float32)
    off = np.array([0, 100, 4196, 4196, 5000], np.int32)
    hist = rng.integers(0, vocab, size=5000).astype(np.int32)
    y = x.copy()
    ctx.apply_repetition_penalty(y, off, hist, 1.05)
    z = x.copy()
    assert ref.apply_penalty(z, off, hist, 1.05) == 0
    assert np.array_equal(y.view(U32), z.view(U32))


def test_wide_topp_ranks_by_probability_on_near_ties(ctx):
    """Candidates whose probabilities tie while d = x - max differs (values within 1e-38 of the
    maximum, or far enough below it for exp to underflow): the ordered kernel must rank by p."""
    rng = np.random.default_rng(654)
    rows, vocab = 8, 20000
    x = (rng.standard_normal((rows, vocab)) * 0.5 - 3.0).astype(np.float32)
    for r in range(rows):
        cols = rng.choice(vocab, size=12, replace=False)
        x[r, cols[:6]] = np.array([1e-38, 0.0, 5e-39, -1e-38, 2e-38, 0.0], np.float32)
        x[r, cols[6:]] = np.array([-900.0, -800.0, -1000.0, -760.0, -3.0e4, -850.0], np.float32)
        if r % 2:  # a sparse row: 50 ordinary values, the six above and 44 that underflow exp
            keep = rng.choice(vocab, size=100, replace=False)
            y = np.full(vocab, -np.inf, np.float32)
            y[keep[:50]] = rng.standard_normal(50).astype(np.float32)
            y[keep[50:56]] = x[r, cols[:6]]
            y[keep[56:]] = (-800.0 - 10.0 * rng.random(44)).astype(np.float32)
            x[r] = y
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = [40, 100, 60, 100, 100, 100, 256, 100]
    p["top_p"] = [0.9, 0.5, 0.999, 0.3, 0.3, 0.9, 0.3, 0.999]
    p["temperature"] = 1.0
    p["rep_penalty"] = 1.0
    p["keep_id"] = -1
    p["ban_id"] = -1
    check_rows(ctx, x, p, np.linspace(0.03, 0.97, rows), label="wide near ties")


def test_wide_topp_threshold_on_a_prefix_sum(ctx):
    """Top-p thresholds equal to a running sum of the sorted probabilities (m equal candidates, so
    every p is 1/m exactly and 1 - top_p lands on a prefix sum): the cut is decided by cum <= thr
    with equality, where the kernel's parallel prefix sums cannot decide and its sequential form
    must. Also thresholds just above and below such a sum, and rows whose candidates all survive."""
    rows, vocab = 12, 20000
    rng = np.random.default_rng(77)
    x = np.full((rows, vocab), -2000.0, np.float32)  # exp(x - max) underflows to 0 in double
    m = [4, 8, 8, 16, 4, 4, 32, 2, 64, 8, 128, 256]
    top_p = [0.75, 0.5, 0.625, 0.75, 0.7500001, 0.7499999, 0.875, 0.5, 0.9375, 0.9999999, 0.5, 0.25]
    for r in range(rows):
        cols = rng.choice(vocab, size=m[r], replace=False)
        x[r, cols] = 10.0
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = m
    p["top_p"] = np.array(top_p, np.float32)
    p["temperature"] = 1.0
    p["rep_penalty"] = 1.0
    p["keep_id"] = -1
    p["ban_id"] = -1
    for u in (np.linspace(0.01, 0.99, rows), np.full(rows, 0.5)):
        ids, ora = check_rows(ctx, x, p, u, label="wide top-p on a prefix sum")
        assert (ids >= 0).all()


def test_wide_handback_next_to_ordered_rows(ctx):
    """Rows of the wide workload's options (top-k 200, penalty, suppression) next to rows the ordered
    pass must hand back to the general algorithm in the same workgroup: 2000 entries tied at the
    maximum overflow its buffers, 300 tied at the k-th value exceed the exact regime's capacity."""
    w = workloads.workload(5)
    b = w.generate(rows=48)
    x = b.logits.copy()
    rng = np.random.default_rng(515)
    vocab = w.vocab
    for r in range(0, 48, 3):
        cols = rng.choice(vocab - 1024, size=2000, replace=False)
        if r % 2 == 0:
            x[r, cols] = x[r].max() + 1.0              # 2000 ties at the maximum
        else:
            x[r, cols[:300]] = np.float32(x[r].max() + 0.5)  # 300 ties at the k-th value
            x[r, cols[300:350]] = np.float32(x[r].max() + 2.0)
    check_rows(ctx, x, b.params, b.u, b.hist_off, b.hist_ids, label="wide hand-back mix")


def test_wide_signed_zero_at_kth(ctx):
    """+0 and -0 at the k-th value of 151936-entry rows (K = 1 over zeros, ties of zeros after a few
    positive entries), with write-back logits and probabilities against the oracle."""
    x, p, u, off, hist = signed_zero_batch(np.random.default_rng(5151), 24, 151936)
    ids, _ = check_rows(ctx, x, p, u, off, hist, label="wide signed zeros")
    assert (ids >= 0).all()
    assert (x[np.arange(0, 24, 3), ids[::3]] == 0.0).all()
