"""GPU parity: the HIP sampler (through the C ABI) against the CPU oracle on the same inputs.

Bar: sampled ids identical except rows whose draw or top-p cutoff lies within 1e-6 of a boundary
(counted); write-back logits bit-identical; final probabilities within 1e-5 relative.
"""
import os

import numpy as np
import pytest

from oracle import ref
from parity import PROB_RTOL, comparable_rows, compare_ids, prob_rel_error
from voxwerk_amd import workloads
from voxwerk_amd._lib import PARAMS_DTYPE
from voxwerk_amd.sampler import HistoryIdOutOfRange, NonFiniteLogits, SamplingOptions, make_params

pytestmark = pytest.mark.gpu

U32 = np.uint32


def both(ctx, logits, params, u=None, hist_off=None, hist_ids=None):
    ids, lg, pr = ctx.sample(logits, params, u, hist_off, hist_ids, want_logits=True, want_probs=True)
    ora = ref.sample(logits, params, u, hist_off, hist_ids, threads=8, want_logits=True, want_probs=True)
    assert ora["rc"] == 0
    return ids, lg, pr, ora


def check(ids, lg, pr, ora, label=""):
    rep = compare_ids(ids, ora)
    print(f"{label}: {rep}", flush=True)
    assert not rep.unexplained, f"{label}: ids differ away from boundaries at rows {rep.unexplained[:10]}"
    assert np.array_equal(lg.view(U32), ora["logits"].view(U32)), f"{label}: write-back logits differ"
    rel = prob_rel_error(pr, ora["probs"], comparable_rows(ids, ora))
    assert rel <= PROB_RTOL, f"{label}: probability relative error {rel:.3e}"
    return rep


@pytest.mark.parametrize("wid", [1, 3, 4])
def test_workload_parity(ctx, wid):
    w = workloads.workload(wid)
    b = w.generate()
    print(f"workload {w.name} rows={b.rows} vocab={w.vocab} digest={b.digest()[:16]}", flush=True)
    check(*both(ctx, b.logits, b.params, b.u, b.hist_off, b.hist_ids), label=w.name)


def test_code_predictor_frame(ctx):
    w = workloads.workload(2)
    for step in range(w.steps):
        b = w.generate(step=step)
        check(*both(ctx, b.logits, b.params, b.u, b.hist_off, b.hist_ids), label=f"{w.name}[{step}]")


def _params(rows, rng, **fixed):
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = rng.choice([0, 1, 2, 5, 50, 200, 255, 256, 257, 1000], size=rows)
    p["top_p"] = rng.choice([1.0, 0.95, 0.9, 0.5, 0.1, 1e-6], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.7, 0.9, 1.0, 1.3], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.05, 1.1, 0.9], size=rows).astype(np.float32)
    p["supp_begin"] = 0
    p["supp_end"] = 0
    p["keep_id"] = -1
    p["ban_id"] = -1
    for k, v in fixed.items():
        p[k] = v
    return p


@pytest.mark.parametrize("vocab", [7, 64, 1000, 2048, 3001, 3072, 5000, 8192])
def test_mixed_options(ctx, vocab):
    """Per-row option mixes over several vocab sizes (odd sizes take the scalar-load kernel)."""
    rng = np.random.default_rng(1000 + vocab)
    rows = 96
    logits = (rng.standard_normal((rows, vocab)) * rng.choice([0.5, 2.0, 4.0], size=(rows, 1))).astype(np.float32)
    hl = rng.integers(0, 300, size=rows)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = rng.integers(0, vocab, size=off[-1]).astype(np.int32)
    p = _params(rows, rng)
    p["do_sample"][::7] = 0
    u = rng.random(rows)
    check(*both(ctx, logits, p, u, off, hist), label=f"mixed V={vocab}")


@pytest.mark.parametrize("vocab", [3072, 5000, 9000])
def test_tiny_probabilities_keep_their_value(ctx, vocab):
    """Rows whose logits span more than 87 after temperature, so that exp(x - max) of the smallest
    kept entries is below fp32's normal range (the reference's fp64 Math.Exp still gives them a
    positive probability, down to d = -745): every probability the oracle keeps, those included,
    within 1e-5 relative, on the one-workgroup path (3072, 5000) and the streaming path (9000)."""
    rng = np.random.default_rng(7000 + vocab)
    rows = 32
    logits = np.round(rng.standard_normal((rows, vocab)) * 4.0).astype(np.float32)
    logits[:, ::97] -= 40.0  # a far tail: d down to about -200 at T = 0.3
    p = _params(rows, rng, top_k=0, rep_penalty=1.0)
    p["top_p"] = np.where(np.arange(rows) % 2 == 0, 1.0, rng.choice([0.999999, 0.9999], size=rows)).astype(np.float32)
    p["temperature"] = rng.choice([0.3, 0.5], size=rows).astype(np.float32)
    ids, lg, pr, ora = both(ctx, logits, p, rng.random(rows))
    tiny = (ora["probs"] > 0) & (ora["probs"] < 1e-38)
    assert tiny.sum() > 0, "the rows must hold kept entries below fp32's normal range"
    check(ids, lg, pr, ora, label=f"tiny probabilities V={vocab}")


def test_greedy_ties_and_signed_zero(ctx):
    x = np.array([[0.0, -0.0, 0.0, -1.0], [-0.0, 0.0, -5.0, -0.0], [1.0, 3.0, 3.0, 2.0]], dtype=np.float32)
    p = make_params(SamplingOptions.Greedy())
    ids = ctx.sample(x, p)
    assert ids.tolist() == [0, 0, 1]
    assert ctx.argmax(x).tolist() == [0, 0, 1]


def test_all_masked_row_returns_last_id(ctx):
    vocab = 3072
    x = np.zeros((2, vocab), np.float32)
    p = np.zeros(2, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = 50
    p["top_p"] = [1.0, 0.9]
    p["temperature"] = 0.9
    p["rep_penalty"] = 1.0
    p["supp_begin"] = 0
    p["supp_end"] = vocab
    p["keep_id"] = -1
    p["ban_id"] = -1
    ids, lg, pr, ora = both(ctx, x, p, np.array([0.3, 0.7]))
    assert ids.tolist() == [vocab - 1, vocab - 1] == ora["ids"].tolist()
    assert np.isnan(pr).all()


def test_uniform_row_ties(ctx):
    """Equal logits: top-k keeps every tie, top-p resolves the cut by index order."""
    vocab = 3072
    rows = 8
    x = np.full((rows, vocab), 0.25, np.float32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = [0, 50, 0, 0, 3000, 0, 0, 10]
    p["top_p"] = [0.5, 0.5, 0.999, 1e-6, 0.3, 0.75, 1.0, 1.0]
    p["temperature"] = 1.0
    p["rep_penalty"] = 1.0
    p["keep_id"] = -1
    p["ban_id"] = -1
    u = np.linspace(0.01, 0.97, rows)
    ids, lg, pr, ora = both(ctx, x, p, u)
    check(ids, lg, pr, ora, label="uniform ties")


def test_k1_and_tiny_top_p(ctx):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((64, 3072)).astype(np.float32)
    x[:, 100] = x.max(axis=1) + 1.0
    x[:32, 2000] = x[:32, 100]  # tied maxima on half of the rows
    p = np.zeros(64, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = np.where(np.arange(64) % 2 == 0, 1, 0)
    p["top_p"] = np.where(np.arange(64) % 2 == 0, 1.0, 1e-7)
    p["temperature"] = 0.9
    p["rep_penalty"] = 1.0
    p["keep_id"] = -1
    p["ban_id"] = -1
    ids, lg, pr, ora = both(ctx, x, p, rng.random(64))
    check(ids, lg, pr, ora, label="k1/tiny-p")
    # top-p -> 0 keeps only the highest-index maximum
    odd = np.arange(64) % 2 == 1
    expect = np.where(np.arange(64) < 32, 2000, 100)
    assert np.array_equal(ids[odd], expect[odd])


def test_history_id_out_of_range(ctx):
    x = np.zeros((2, 2048), np.float32)
    p = make_params(SamplingOptions(), rep_penalty=1.05)
    off = np.array([0, 2, 4], np.int32)
    hist = np.array([1, 2, 3, 2048], np.int32)
    with pytest.raises(HistoryIdOutOfRange):
        ctx.sample(x, p, np.array([0.5, 0.5]), off, hist)
    ids = ctx.sample(x, p, np.array([0.5, 0.5]), off, hist, raise_on_error=False)
    assert ids[1] == -2 and ids[0] >= 0
    hist[3] = -1
    with pytest.raises(HistoryIdOutOfRange):
        ctx.sample(x, p, np.array([0.5, 0.5]), off, hist)


@pytest.mark.parametrize("vocab", [3072, 8192])
def test_long_histories_block_path(ctx, vocab):
    """Histories around and past the 2048 ids a workgroup takes in one pass (the rest go through the
    bitmap), with ids repeated within and across the two parts, on the one-workgroup kernel; then an
    id out of range in each part."""
    rng = np.random.default_rng(9000 + vocab)
    lens = [0, 1, 2047, 2048, 2049, 3000, 6000, 9000]
    rows = len(lens)
    x = (rng.standard_normal((rows, vocab)) * 2.0).astype(np.float32)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(lens)
    pool = rng.integers(0, vocab, size=700)  # few distinct ids: most are repeats
    hist = pool[rng.integers(0, pool.size, size=off[-1])].astype(np.int32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = [0, 50, 0, 50, 0, 50, 0, 50]
    p["top_p"] = np.float32(0.9)
    p["temperature"] = np.float32(0.9)
    p["rep_penalty"] = np.array([1.1, 0.9] * 4, np.float32)
    p["keep_id"] = -1
    p["ban_id"] = -1
    u = rng.random(rows)
    ids, lg, pr = ctx.sample(x, p, u, off, hist, want_logits=True, want_probs=True, path="block")
    ora = ref.sample(x, p, u, off, hist, threads=8, want_logits=True, want_probs=True)
    check(ids, lg, pr, ora, label=f"long histories V={vocab}")
    for at in (100, 2500):  # in the first 2048 ids of the 3000-id row, then past them
        bad = hist.copy()
        bad[off[5] + at] = vocab
        got = ctx.sample(x, p, u, off, bad, raise_on_error=False, path="block")
        assert got[5] == -2, (at, got[5])
        assert np.array_equal(np.delete(got, 5), np.delete(ids, 5))


def test_nonfinite_rejected(ctx):
    x = np.zeros((3, 1024), np.float32)
    x[0, 5] = np.nan
    x[1, 7] = np.inf
    p = make_params(SamplingOptions())
    ids = ctx.sample(x, p, np.array([0.1, 0.2, 0.3]), raise_on_error=False)
    assert ids[0] == -3 and ids[1] == -3 and ids[2] >= 0
    with pytest.raises(NonFiniteLogits):
        ctx.sample(x[:1], p, np.array([0.1]))


def test_deterministic_and_batch_independent(ctx):
    w = workloads.workload(4)
    b = w.generate(rows=256)
    a1 = ctx.sample(b.logits, b.params, b.u, b.hist_off, b.hist_ids)
    a2 = ctx.sample(b.logits, b.params, b.u, b.hist_off, b.hist_ids)
    assert np.array_equal(a1, a2)
    for r in (0, 17, 255):
        h = b.hist_ids[b.hist_off[r]:b.hist_off[r + 1]]
        one = ctx.sample(b.logits[r:r + 1], b.params[r], b.u[r:r + 1], np.array([0, h.size], np.int32), h)
        assert one[0] == a1[r]


def test_device_api_matches_host(ctx):
    from voxwerk_amd.hip import DeviceArray

    w = workloads.workload(4)
    b = w.generate(rows=512)
    host = ctx.sample(b.logits, b.params, b.u, b.hist_off, b.hist_ids)
    d_logits = DeviceArray.from_numpy(b.logits)
    d_off = DeviceArray.from_numpy(b.hist_off)
    d_ids = DeviceArray.from_numpy(b.hist_ids)
    d_params = DeviceArray.from_numpy(b.params)
    d_u = DeviceArray.from_numpy(b.u)
    out = DeviceArray((b.rows,), np.int32)
    ctx.sample_device(b.rows, w.vocab, d_logits, w.vocab, d_params, 1, d_u, out, d_off, d_ids)
    ctx.synchronize()
    assert np.array_equal(out.numpy(), host)


def test_torch_interop_subprocess():
    """A caller holding torch tensors: torch imported first, the library bound to torch's HIP runtime,
    launched on torch's current stream."""
    import subprocess
    import sys

    script = os.path.join(os.path.dirname(__file__), "torch_interop.py")
    p = subprocess.run([sys.executable, script], capture_output=True, text=True, timeout=300)
    print(p.stdout[-2000:], p.stderr[-2000:])
    assert p.returncode == 0


def _near_tie_rows(rows, vocab, rng):
    """Rows whose top-k candidates include values within 1e-38 of the maximum and values far below
    it (exp underflows): their probabilities tie while d = x - max differs, so the (d, index) order
    of the candidates is not the reference's (p, index) order and the kernels must rank by p."""
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
    return x


def test_topp_ranks_by_probability_on_near_ties(ctx):
    rng = np.random.default_rng(321)
    rows, vocab = 16, 3072
    x = _near_tie_rows(rows, vocab, rng)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = [40, 100, 60, 100, 100, 100, 256, 100] * 2
    p["top_p"] = [0.9, 0.5, 0.999, 0.3, 0.3, 0.9, 0.3, 0.999] * 2
    p["temperature"] = 1.0
    p["rep_penalty"] = 1.0
    p["keep_id"] = -1
    p["ban_id"] = -1
    check(*both(ctx, x, p, np.linspace(0.02, 0.98, rows)), label="near ties")
