"""GPU parity of the one-wave-per-row path (VXS_FLAG_PATH_WAVE): ids against the CPU oracle and
identical to the one-workgroup-per-row path on the same rows, over the workloads, option mixes and the
rows the wave path hands back to the general algorithm (top-k, few candidates, crowded or degenerate
top-p cuts, requested outputs)."""
import numpy as np
import pytest

from oracle import ref
from parity import compare_ids, signed_zero_batch
from voxwerk_amd import workloads
from voxwerk_amd._lib import PARAMS_DTYPE

pytestmark = pytest.mark.gpu


def run_both_paths(ctx, logits, params, u=None, off=None, hist=None, label=""):
    wave = ctx.sample(logits, params, u, off, hist, path="wave", raise_on_error=False)
    block = ctx.sample(logits, params, u, off, hist, path="block", raise_on_error=False)
    ora = ref.sample(logits, params, u, off, hist, threads=8)
    rep = compare_ids(wave, ora)
    print(f"{label}: wave {rep}", flush=True)
    assert not rep.unexplained, f"{label}: wave path ids differ at rows {rep.unexplained[:10]}"
    assert np.array_equal(wave, block), f"{label}: wave and block paths disagree"
    return wave, ora


@pytest.mark.parametrize("wid", [1, 3, 4])
def test_wave_workloads(ctx, wid):
    w = workloads.workload(wid)
    b = w.generate()
    run_both_paths(ctx, b.logits, b.params, b.u, b.hist_off, b.hist_ids, label=w.name)


def test_wave_code_predictor(ctx):
    w = workloads.workload(2)
    for step in range(0, w.steps, 4):
        b = w.generate(step=step)
        run_both_paths(ctx, b.logits, b.params, b.u, b.hist_off, b.hist_ids, label=f"{w.name}[{step}]")


@pytest.mark.parametrize("vocab,rows", [(v, 256) for v in (7, 64, 300, 1000, 2048, 2500, 3001, 3072)] +
                         [(3072, 2049), (1000, 2050)])  # two rows per wave from 2048 rows, odd end
def test_wave_option_mixes(ctx, vocab, rows):
    """Mostly full-vocabulary rows (the wave path's own work), some top-k and greedy rows."""
    rng = np.random.default_rng(2000 + vocab + rows)
    scale = rng.choice([0.3, 1.0, 3.0, 8.0], size=(rows, 1))
    logits = (rng.standard_normal((rows, vocab)) * scale).astype(np.float32)
    logits[rng.random((rows, vocab)) < 0.02] += 5.0
    hl = rng.integers(0, 700, size=rows)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = rng.integers(0, vocab, size=off[-1]).astype(np.int32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = (rng.random(rows) > 0.1).astype(np.int32)
    p["top_k"] = np.where(rng.random(rows) < 0.15, rng.integers(1, 300, rows), 0)
    p["top_p"] = rng.choice([1.0, 0.99, 0.95, 0.9, 0.8, 0.5, 0.2, 1e-6], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.5, 0.7, 0.9, 1.0, 1.3], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.05, 1.1, 0.9], size=rows).astype(np.float32)
    supp = rng.random(rows) < 0.3
    p["supp_begin"] = np.where(supp, vocab // 3, 0)
    p["supp_end"] = np.where(supp, vocab, 0)
    p["keep_id"] = np.where(supp, vocab // 2, -1)
    p["ban_id"] = np.where(rng.random(rows) < 0.1, vocab // 2, -1)
    run_both_paths(ctx, logits, p, rng.random(rows), off, hist, label=f"mixed V={vocab}")


def test_wave_deferred_and_special_rows(ctx):
    vocab = 3072
    rng = np.random.default_rng(31)
    rows = 12
    x = (rng.standard_normal((rows, vocab)) * 2).astype(np.float32)
    x[0] = 0.25                 # uniform row: one crowded crossing bucket
    x[1, :] = -np.inf           # all masked
    x[1, 5] = 1.0
    x[2, 7] = np.nan            # rejected
    x[3, 9] = np.inf            # rejected
    x[4, :3000] = -np.inf       # 72 candidates: exact regime
    x[5] = np.round(x[5])       # many exact ties
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_p"] = [0.5, 0.9, 0.9, 0.9, 0.9, 0.7, 1e-7, 0.0, 1.0, 0.95, 0.95, 0.95]
    p["temperature"] = [1.0] * 9 + [-1.0, 1e-3, 1e3]
    p["rep_penalty"] = 1.0
    p["keep_id"] = -1
    p["ban_id"] = -1
    u = np.linspace(0.02, 0.98, rows)
    wave, ora = run_both_paths(ctx, x, p, u, label="special rows")
    assert wave[2] == -3 and wave[3] == -3


def test_wave_history_errors(ctx):
    x = np.zeros((1024, 2048), np.float32)
    p = np.zeros(1024, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_p"] = 0.9
    p["temperature"] = 1.0
    p["rep_penalty"] = 1.1
    p["keep_id"] = -1
    p["ban_id"] = -1
    off = (np.arange(1025) * 2).astype(np.int32)
    hist = np.tile(np.array([1, 2], np.int32), 1024)
    hist[7] = 2048
    hist[100] = -5
    ids = ctx.sample(x, p, np.full(1024, 0.5), off, hist, path="wave", raise_on_error=False)
    assert ids[3] == -2 and ids[50] == -2
    assert (np.delete(ids, [3, 50]) >= 0).all()


def test_wave_equal_mass_cuts(ctx):
    """Top-p cuts that fall inside a group of equal logits (equal masses): the wave path keeps the
    group's higher indices where equal masses imply equal logits (logits 4 to 11 below the max) and
    hands the row back elsewhere; groups of logits one ulp apart near the max share masses without
    sharing logits, which only the general path orders correctly."""
    vocab = 3072
    rng = np.random.default_rng(77)
    rows = 48
    x = np.full((rows, vocab), -np.inf, np.float32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["temperature"] = 1.0
    p["rep_penalty"] = 1.0
    p["keep_id"] = -1
    p["ban_id"] = -1
    for r in range(rows):
        pos = rng.permutation(vocab)
        x[r, pos[:400]] = rng.uniform(-14.0, -9.0, 400).astype(np.float32)  # background
        x[r, pos[400]] = 0.0                                                  # the max
        kind = r % 3
        group = pos[401:441]
        if kind == 0:    # equal logits 5 below the max: handled by the wave path
            x[r, group] = np.float32(-5.0)
            p["top_p"][r] = 0.9
        elif kind == 1:  # equal logits 2 below the max: masses outside the safe range
            x[r, group] = np.float32(-2.0)
            p["top_p"][r] = 0.8
        else:            # logits one ulp apart 0.3 below the max: equal masses, distinct logits
            base = np.float32(-0.3)
            x[r, group] = np.nextafter(np.full(40, base), np.float32(0.0)).astype(np.float32)
            x[r, group[::2]] = base
            p["top_p"][r] = 0.6
    u = rng.random(rows)
    run_both_paths(ctx, x, p, u, label="equal-mass cuts")


def test_wave_all_rows_top_k(ctx):
    """Every row samples with top-k 50 (the talker default), which the one-wave path now takes itself."""
    rng = np.random.default_rng(77)
    rows, vocab = 2050, 3072
    logits = (rng.standard_normal((rows, vocab)) * 2.5).astype(np.float32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"], p["top_k"], p["top_p"], p["temperature"] = 1, 50, np.float32(0.95), np.float32(0.9)
    p["rep_penalty"], p["keep_id"], p["ban_id"] = np.float32(1.0), -1, -1
    run_both_paths(ctx, logits, p, rng.random(rows), label="all top-k")


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_wave_full_batches_mixed(ctx, seed):
    """4096-row batches (both halves of the launch, the second starting its loads later) with the
    headline's full-vocabulary options varied per row: ids against the oracle and the block path."""
    rng = np.random.default_rng(seed)
    rows, vocab = 4096, 3072
    mix = rng.random((rows, vocab)) < rng.uniform(0.02, 0.2, size=(rows, 1))
    logits = (rng.standard_normal((rows, vocab)) * rng.choice([0.5, 1.0, 2.0], size=(rows, 1)) + 4.0 * mix)
    logits = logits.astype(np.float32)
    hl = rng.integers(0, 513, size=rows)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = rng.integers(0, vocab, size=off[-1]).astype(np.int32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_p"] = rng.choice([1.0, 0.98, 0.95, 0.9, 0.7], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.8, 1.0, 1.2], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.1, 1.3], size=rows).astype(np.float32)
    p["keep_id"], p["ban_id"] = -1, -1
    run_both_paths(ctx, logits, p, rng.random(rows), off, hist, label=f"4096 rows seed {seed}")


@pytest.mark.parametrize("seed,vocab", [(0, 1000), (1, 2048), (2, 2500), (3, 3072)])
def test_wave_random_option_mix(ctx, seed, vocab):
    """2048 rows whose options are drawn per row over everything the one-wave path takes or hands
    back: greedy rows, top-k 1..80 on 60 % of the rows (above 64 handed back), top-p from 0.05 to
    1, temperatures below and above 1, penalties below and above 1 over histories of 0-2499 ids
    (above 2048 handed back), suppression ranges with a kept id, a banned id, and a fifth of the
    rows rounded to integers (ties): ids against the oracle and the block path."""
    rng = np.random.default_rng(9000 + seed)
    rows = 2048
    logits = (rng.standard_normal((rows, vocab)) * rng.choice([0.5, 2.0, 5.0], size=(rows, 1))).astype(np.float32)
    tied = rng.random(rows) < 0.2
    logits[tied] = np.round(logits[tied])
    hl = rng.integers(0, 2500, size=rows)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = rng.integers(0, vocab, size=off[-1]).astype(np.int32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = (rng.random(rows) > 0.05).astype(np.int32)
    p["top_k"] = np.where(rng.random(rows) < 0.6, rng.integers(1, 81, rows), 0)
    p["top_p"] = rng.choice([1.0, 0.95, 0.9, 0.5, 0.05], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.6, 0.9, 1.0, 1.4], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.05, 1.2, 0.9], size=rows).astype(np.float32)
    supp = rng.random(rows) < 0.3
    p["supp_begin"] = np.where(supp, rng.integers(0, vocab // 2, rows), 0)
    p["supp_end"] = np.where(supp, vocab, 0)
    p["keep_id"] = np.where(supp, vocab - 3, -1)
    p["ban_id"] = np.where(rng.random(rows) < 0.1, 7, -1)
    run_both_paths(ctx, logits, p, rng.random(rows), off, hist, label=f"random mix seed {seed} V {vocab}")


@pytest.mark.parametrize("vocab", [300, 1000, 2048, 3072])
def test_wave_top_k_edges(ctx, vocab):
    """Top-k on one wave at its edges: K = 1, 64 and 65 (the last handed back), logits quantised so
    that ties at the k-th value push the candidates past 64 (handed back) or not, rows whose
    suppression leaves fewer finite entries than K (no masking, the exact regime over them), and
    top-p, temperature and penalty mixes; ids against the oracle and the block path."""
    rng = np.random.default_rng(4000 + vocab)
    rows = 1024
    logits = (rng.standard_normal((rows, vocab)) * rng.choice([0.5, 2.0, 4.0], size=(rows, 1))).astype(np.float32)
    quant = rng.random(rows) < 0.3
    logits[quant] = np.round(logits[quant] * 2.0) / 2.0  # many exact ties
    hl = rng.integers(0, 400, size=rows)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = rng.integers(0, vocab, size=off[-1]).astype(np.int32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = rng.choice([1, 2, 17, 50, 64, 65], size=rows)
    p["top_p"] = rng.choice([1.0, 0.95, 0.8, 0.3], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.7, 0.9, 1.0], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.05, 1.3], size=rows).astype(np.float32)
    few = rng.random(rows) < 0.15  # suppress all but a few dozen entries
    p["supp_begin"] = np.where(few, 40, 0)
    p["supp_end"] = np.where(few, vocab, 0)
    p["keep_id"] = np.where(few, vocab - 1, -1)
    p["ban_id"] = -1
    run_both_paths(ctx, logits, p, rng.random(rows), off, hist, label=f"top-k edges V={vocab}")


def test_wave_long_histories(ctx):
    """Histories of 513 to 2048 ids on the one-wave path (taken in chunks, kept distinct by an LDS
    bitmap), with ids repeated within and across chunks, rows whose bad id sits past the first 512,
    and histories over 2048 (handed back): ids against the oracle and the block path."""
    rng = np.random.default_rng(808)
    rows, vocab = 1024, 3072
    logits = (rng.standard_normal((rows, vocab)) * 2.5).astype(np.float32)
    hl = rng.integers(400, 2300, size=rows)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = np.empty(off[-1], np.int32)
    for r in range(rows):
        pool = rng.integers(0, vocab, size=rng.choice([40, 600, 3000]))  # few distinct ids: many repeats
        hist[off[r]:off[r + 1]] = rng.choice(pool, size=hl[r])
    bad_rows = rng.choice(rows, 12, replace=False)
    for r in bad_rows:
        if hl[r] > 600:
            hist[off[r] + 550 + (r % 40)] = vocab + (r % 3)  # outside the vocabulary, past the first chunk
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = rng.choice([0, 0, 50], size=rows)
    p["top_p"] = rng.choice([1.0, 0.95, 0.8], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.9, 1.0], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.05, 1.3, 0.8], size=rows).astype(np.float32)
    p["keep_id"], p["ban_id"] = -1, -1
    wave, _ = run_both_paths(ctx, logits, p, rng.random(rows), off, hist, label="long histories")
    for r in bad_rows:
        if hl[r] > 600:
            assert wave[r] == -2, (r, wave[r])  # VXS_ERR_ID_OUT_OF_RANGE


def test_wave_signed_zero_at_kth(ctx):
    """+0 and -0 at the k-th value: the forced wave path on 96 rows and the default path on a full
    1024-row batch (which takes the one-wave kernel), against the oracle and the block path."""
    rng = np.random.default_rng(4242)
    x, p, u, off, hist = signed_zero_batch(rng, 96, 3072)
    wave, _ = run_both_paths(ctx, x, p, u, off, hist, label="signed zeros (wave)")
    assert (wave >= 0).all()
    assert (x[np.arange(0, 96, 3), wave[::3]] == 0.0).all()  # K = 1 rows draw one of the zeros
    x, p, u, off, hist = signed_zero_batch(rng, 1024, 3072)
    ids = ctx.sample(x, p, u, off, hist, raise_on_error=False)
    block = ctx.sample(x, p, u, off, hist, path="block", raise_on_error=False)
    rep = compare_ids(ids, ref.sample(x, p, u, off, hist, threads=8))
    print(f"signed zeros (1024 rows): {rep}", flush=True)
    assert not rep.unexplained, f"ids differ at rows {rep.unexplained[:10]}"
    assert np.array_equal(ids, block)


def test_wave_top_k_at_tiny_penalised_logits(ctx):
    """Positive logits below 2^-60 in the history (penalised by rho 1.1 or 0.9) next to entries one
    ulp either side of their quotients and a maximum of 1, with the k-th largest value among the
    tiny ones: the k-th value and the kept set depend on the quotients being correctly rounded."""
    rng = np.random.default_rng(977)
    rows, vocab = 64, 3072
    x = rng.uniform(-9.0, -1.0, (rows, vocab)).astype(np.float32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_p"] = 1.0
    p["temperature"] = 1.0
    p["keep_id"], p["ban_id"] = -1, -1
    off = np.zeros(rows + 1, np.int32)
    hist = []
    for r in range(rows):
        rho = np.float32(1.1 if r % 2 == 0 else 0.9)
        p["rep_penalty"][r] = rho
        pos = rng.permutation(vocab)
        n = 12
        t = (np.float32(2.0 ** -70) * rng.uniform(1.0, 2.0 ** 9, n)).astype(np.float32)  # 2^-70 .. 2^-61
        x[r, pos[:n]] = t
        q = (t / rho).astype(np.float32)  # the correctly rounded penalised values
        up = np.nextafter(q, np.float32(1.0))
        dn = np.nextafter(q, np.float32(0.0))
        x[r, pos[n:2 * n]] = np.where(rng.random(n) < 0.5, up, dn)
        x[r, pos[2 * n:3 * n]] = q
        x[r, pos[3 * n]] = 1.0  # the maximum, well above 2^-30
        hist.append(pos[:n].astype(np.int32))
        off[r + 1] = off[r] + n
        p["top_k"][r] = int(rng.integers(2, 3 * n + 1))
    u = rng.random(rows)
    run_both_paths(ctx, x, p, u, off, np.concatenate(hist), label="tiny penalised logits at the k-th value")


@pytest.mark.parametrize("rows", [1024, 2048])
def test_wave_handback_rows_take_one_wave_exact_in_turn(ctx, rows):
    """Every row of the batch handed back by the one-wave kernel (more than 256 entries at or above
    the K-th largest lane maximum: five lanes hold only large values), yet with 50 candidates after
    top-k, so each of a workgroup's four rows in turn reaches the one-wave exact regime of the
    one-workgroup algorithm (one wave samples while the others wait for the next row): ids against
    the oracle and the block path. 1024 rows (one workgroup per CU) run the kernel instance with
    oldest-first issue, 2048 rows the one whose waves step their priority."""
    rng = np.random.default_rng(5050 + rows)
    vocab = 3072
    lane_of = (np.arange(vocab) % 256) // 4  # lane l holds entries c * 256 + 4 l + j
    x = rng.uniform(-3.0, 0.0, (rows, vocab)).astype(np.float32)
    hist = []
    off = np.zeros(rows + 1, np.int32)
    for r in range(rows):
        hot = rng.choice(64, 5, replace=False)
        hot_e = np.isin(lane_of, hot)
        x[r, hot_e] = rng.uniform(5.0, 6.0, hot_e.sum()).astype(np.float32)
        for l in np.setdiff1d(np.arange(64), hot):
            e = rng.choice(np.flatnonzero(lane_of == l))
            x[r, e] = np.float32(rng.uniform(4.0, 4.99))
        lane_max = np.array([x[r, lane_of == l].max() for l in range(64)])
        tf = np.sort(lane_max)[::-1][49]
        assert (x[r] >= tf).sum() > 256  # the one-wave gather overflows: handed back
        h = rng.choice(np.flatnonzero(~hot_e), 40, replace=False).astype(np.int32)
        hist.append(h)
        off[r + 1] = off[r] + len(h)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_k"] = 50
    p["top_p"] = rng.choice([1.0, 0.9], size=rows).astype(np.float32)
    p["temperature"] = np.float32(0.9)
    p["rep_penalty"] = np.float32(1.05)
    p["keep_id"], p["ban_id"] = -1, -1
    u = rng.random(rows)
    wave, _ = run_both_paths(ctx, x, p, u, off, np.concatenate(hist), label="handed-back top-k rows")
    assert (wave >= 0).all()
