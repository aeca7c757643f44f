"""GPU parity of the one-wave nucleus beyond the sampled id.

vxs_sample_stats_device reports, for every row the one-wave nucleus regime samples, the kept fraction
of the probability mass, the smallest kept probability (the top-p cut) and the kept count. They are
checked against the oracle's kept set (its final probabilities > 0) and fp64 softmax probabilities
of the oracle's write-back logits: both masses within 1e-5 relative, counts equal, on rows whose
top-p cut is away from its 1e-6 boundary. The device computes masses as fp32 exp2 values on a 2^-F
grid with exact fp64 sums, so agreement here pins that arithmetic, not only the draw.
"""
import numpy as np
import pytest

from oracle import ref
from parity import comparable_rows, compare_ids
from voxwerk_amd import workloads
from voxwerk_amd._lib import PARAMS_DTYPE

pytestmark = pytest.mark.gpu

STATS_RTOL = 1e-5


def stats_call(ctx, logits, params, u, off=None, hist=None):
    from voxwerk_amd.hip import DeviceArray

    rows, vocab = logits.shape
    d_logits = DeviceArray.from_numpy(np.ascontiguousarray(logits))
    d_params = DeviceArray.from_numpy(params)
    d_u = DeviceArray.from_numpy(np.asarray(u, np.float64))
    d_off = DeviceArray.from_numpy(off) if off is not None else None
    d_hist = DeviceArray.from_numpy(hist) if hist is not None else None
    d_ids = DeviceArray((rows,), np.int32)
    d_stats = DeviceArray((rows, 4), np.float64)
    ctx.sample_stats_device(rows, vocab, d_logits, vocab, d_params, 1, d_u, d_ids, d_stats, d_off, d_hist,
                            path="wave")
    ctx.synchronize()
    return d_ids.numpy(), d_stats.numpy()


def oracle_nucleus(ora):
    """Kept fraction, smallest kept probability and kept count from the oracle's outputs: softmax in
    fp64 of its write-back logits, over the entries its final probabilities keep."""
    lw = ora["logits"].astype(np.float64)
    mx = np.max(np.where(np.isfinite(lw), lw, -np.inf), axis=1, keepdims=True)
    p = np.exp(lw - mx)
    p /= p.sum(axis=1, keepdims=True)
    kept = ora["probs"] > 0
    frac = np.where(kept, p, 0.0).sum(axis=1)
    cut = np.where(kept, p, np.inf).min(axis=1)
    return frac, cut, kept.sum(axis=1)


def check_stats(ctx, logits, params, u, off=None, hist=None, label="", min_wave_rows=1):
    ids, st = stats_call(ctx, logits, params, u, off, hist)
    ora = ref.sample(logits, params, u, off, hist, threads=8, want_logits=True, want_probs=True)
    rep = compare_ids(ids, ora)
    wave = st[:, 3] == 0
    print(f"{label}: {rep} one-wave nucleus rows={int(wave.sum())}", flush=True)
    assert not rep.unexplained, f"{label}: ids differ away from boundaries at rows {rep.unexplained[:10]}"
    # a row is either a one-wave nucleus row (path 0) or all NaN
    other = ~wave
    assert np.isnan(st[other]).all(), f"{label}: stats written for rows outside the one-wave nucleus"
    assert wave.sum() >= min_wave_rows, f"{label}: only {int(wave.sum())} rows took the one-wave nucleus"
    frac, cut, cnt = oracle_nucleus(ora)
    ok = wave & comparable_rows(ids, ora)
    topp = params["top_p"] < 1.0
    ef = np.abs(st[ok, 0] - frac[ok]) / frac[ok]
    assert ef.max(initial=0.0) <= STATS_RTOL, f"{label}: kept fraction off by {ef.max():.3e}"
    okp = ok & topp
    ec = np.abs(st[okp, 1] - cut[okp]) / cut[okp]
    assert ec.max(initial=0.0) <= STATS_RTOL, f"{label}: cut probability off by {ec.max():.3e}"
    bad = np.nonzero(st[okp, 2] != cnt[okp])[0]
    assert bad.size == 0, f"{label}: kept counts differ at rows {np.nonzero(okp)[0][bad][:10]}"
    # without top-p the whole mass is kept
    assert np.all(st[ok & ~topp, 0] == 1.0)
    print(f"{label}: kept-fraction rel err {ef.max(initial=0.0):.2e}, cut rel err {ec.max(initial=0.0):.2e} "
          f"over {int(okp.sum())} top-p rows", flush=True)
    return ids, st, ora


def test_headline_batch_nucleus(ctx):
    """The full 4096-row batch of 3072-entry rows that the throughput figure is measured on."""
    w = workloads.workload(4)
    b = w.generate()
    print(f"workload {w.name} rows={b.rows} vocab={w.vocab} digest={b.digest()[:16]}", flush=True)
    check_stats(ctx, b.logits, b.params, b.u, b.hist_off, b.hist_ids, label=w.name, min_wave_rows=b.rows * 9 // 10)


@pytest.mark.parametrize("vocab", [1000, 2048, 3072])
def test_option_mix_nucleus(ctx, vocab):
    """top-p from 1e-6 to 1, temperatures, penalties and -inf entries over three row shapes."""
    rng = np.random.default_rng(4400 + vocab)
    rows = 1024
    logits = (rng.standard_normal((rows, vocab)) * rng.choice([0.5, 2.0, 4.0, 8.0], size=(rows, 1))).astype(np.float32)
    logits[::7, -64:] = -np.inf
    hl = rng.integers(0, 200, size=rows)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = rng.integers(0, vocab, size=off[-1]).astype(np.int32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_p"] = rng.choice([1.0, 0.99, 0.95, 0.9, 0.8, 0.5, 0.1, 1e-6], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.5, 0.7, 0.9, 1.0, 1.3], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.05, 1.3, 0.9], size=rows).astype(np.float32)
    p["keep_id"] = -1
    p["ban_id"] = -1
    check_stats(ctx, logits, p, rng.random(rows), off, hist, label=f"mix V={vocab}", min_wave_rows=rows // 2)


def test_equal_mass_cut_nucleus(ctx):
    """Cuts inside groups of equal masses: equal logits, and logits one ulp apart 3 below the max (a
    single rounding of d * log2 e merges most of those pairs, so the kept members are chosen by d)."""
    vocab = 3072
    rng = np.random.default_rng(91)
    rows = 64
    x = np.full((rows, vocab), -np.inf, np.float32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["temperature"] = 1.0
    p["rep_penalty"] = 1.0
    p["keep_id"] = -1
    p["ban_id"] = -1
    for r in range(rows):
        pos = rng.permutation(vocab)
        x[r, pos[:400]] = rng.uniform(-14.0, -9.0, 400).astype(np.float32)
        x[r, pos[400]] = 0.0
        group = pos[401:441]
        if r % 2 == 0:
            x[r, group] = np.float32(-5.0)
            p["top_p"][r] = rng.choice([0.85, 0.9])
        else:
            base = np.float32(-3.0)
            x[r, group] = np.nextafter(np.full(40, base), np.float32(0.0)).astype(np.float32)
            x[r, group[::2]] = base
            p["top_p"][r] = rng.choice([0.4, 0.6, 0.7])
    check_stats(ctx, x, p, rng.random(rows), label="equal-mass cuts", min_wave_rows=rows // 2)


def _per_entry(ctx, logits, params, u, off, hist, label):
    from voxwerk_amd.hip import DeviceArray

    rows, vocab = logits.shape
    d = [DeviceArray.from_numpy(np.ascontiguousarray(a)) for a in (logits, params, np.asarray(u, np.float64))]
    d_off = DeviceArray.from_numpy(off) if off is not None else None
    d_hist = DeviceArray.from_numpy(hist) if hist is not None else None
    d_ids, d_stats = DeviceArray((rows,), np.int32), DeviceArray((rows, 4), np.float64)
    d_probs = DeviceArray((rows, vocab), np.float64)
    ctx.sample_stats_device(rows, vocab, d[0], vocab, d[1], 1, d[2], d_ids, d_stats, d_off, d_hist, path="wave",
                            probs=d_probs)
    ctx.synchronize()
    ids, st, pr = d_ids.numpy(), d_stats.numpy(), d_probs.numpy()
    ora = ref.sample(logits, params, u, off, hist, threads=8, want_probs=True)
    wave = st[:, 3] == 0
    assert np.isnan(pr[~wave]).all(), f"{label}: probabilities written for rows outside the one-wave nucleus"
    ok = wave & comparable_rows(ids, ora)
    po, pk = ora["probs"][ok], pr[ok]
    # masses live on a 2^-F grid of exp(d) (F = 41 at 3072 entries): an entry whose exp(d) is below
    # half a step gets mass 0, and one near the grid's step carries its rounding; above 2^-41 * 1e5
    # every probability agrees within 1e-5 relative, and every one within one step absolute
    F = min(51, 53 - int(np.ceil(np.log2(vocab))))
    big = po >= 2.0 ** -F * 1e5
    rel = np.abs(pk[big] - po[big]) / po[big]
    assert rel.max(initial=0.0) <= 1e-5, f"{label}: probability rel error {rel.max():.3e}"
    assert np.all(np.abs(pk - po) <= 2.0 ** -F + 1e-5 * po), f"{label}: probability abs error"
    assert np.all(((pk > 0) == (po > 0)) | (po < 2.0 ** -F)), f"{label}: kept sets differ"
    print(f"{label}: {int(ok.sum())} rows, {int(big.sum())} probabilities, max rel err {rel.max(initial=0.0):.2e}, "
          f"{int(((pk == 0) & (po > 0)).sum())} below the grid", flush=True)


def test_per_entry_probabilities_headline(ctx):
    """Every entry's final probability from the one-wave nucleus kernel (the timed kernel's stats
    build) against the oracle's, on the first 1024 rows of the headline batch."""
    w = workloads.workload(4)
    b = w.generate(rows=1024)
    _per_entry(ctx, b.logits, b.params, b.u, b.hist_off, b.hist_ids, w.name)


def test_per_entry_probabilities_option_mix(ctx):
    rng = np.random.default_rng(4711)
    rows, vocab = 512, 3072
    logits = (rng.standard_normal((rows, vocab)) * rng.choice([0.5, 2.0, 4.0], size=(rows, 1))).astype(np.float32)
    hl = rng.integers(0, 300, size=rows)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = rng.integers(0, vocab, size=off[-1]).astype(np.int32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_p"] = rng.choice([1.0, 0.99, 0.95, 0.8, 0.5], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.7, 1.0, 1.3], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.05, 1.3], size=rows).astype(np.float32)
    p["keep_id"], p["ban_id"] = -1, -1
    _per_entry(ctx, logits, p, rng.random(rows), off, hist, "per-entry option mix")
