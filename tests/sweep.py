"""Randomised parity sweep: random batches over every path of the sampler (one-wave, one-workgroup,
streaming), each compared with the CPU oracle on the same inputs.

A batch draws its vocabulary (7 to 151,936 entries), its row count, the shape of its logits (normal
at several scales, Zipf-like, integer ties, sparse spikes, the headline's two-component mixture,
signed zeros), histories of 0 to 5000 ids and per-row options over everything the reference's
sampler takes (greedy rows, top-k 1-299, top-p from 1e-6 to 1, temperatures 0.3-2, penalties below
and above 1, suppression ranges with a kept id, a banned id), some rows outside the contract (NaN
or +inf logits, a history id past the vocabulary: their error codes must match), a forced or
automatic path, one of three entry points (host buffers; device buffers with a padded leading
dimension and possibly a base one float past 16-byte alignment; the entry point that allocates
nothing), and for some batches the final probabilities or the write-back logits. Bar: ids and
error codes identical except counted boundary draws and cuts, write-back logits bit-identical,
probabilities within 1e-5 relative (the bar of tests/test_gpu_parity.py).

    python tests/sweep.py --seconds 300 --seed 1      # a long run on the GPU, one line per batch
    python tests/sweep.py --heads 500 --seconds 0     # random logit-head calls (bf16 and int8)
    python tests/sweep.py --sequences 50 --seconds 0  # random batched stages over a history store
    python tests/sweep.py --stats 200 --seconds 0     # the one-wave kernel's per-entry probabilities
    python tests/sweep.py --misc 200 --seconds 0      # penalty and argmax host calls
The GPU suite runs a short seeded sweep of each (tests/test_gpu_sweep.py). Head calls: rows 1-64,
k a multiple of 8 up to 2048, n up to 5200, padded leading dimensions, bf16 or int8 weights (packed
on the GPU, bit-identical to the oracle's packing), real, integer-valued or partly non-finite hidden
values; bar: within the fp32 bound of the exact product (exact on integer data), the IEEE pattern
of non-finite results, nothing written past n.
"""
from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.dirname(HERE), HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import ref  # noqa: E402
from parity import PROB_RTOL, comparable_rows, compare_ids, prob_rel_error  # noqa: E402
from voxwerk_amd._lib import PARAMS_DTYPE  # noqa: E402

VOCABS = [7, 64, 300, 1000, 2048, 2500, 3001, 3072, 3072, 3072, 4096, 8192, 9000, 32000, 151936]


def random_batch(rng):
    """One random batch: (logits, params, u, hist_off, hist_ids, path, want_probs, want_logits,
    (entry point, leading-dimension pad, base shift), label)."""
    V = int(rng.choice(VOCABS))
    if V <= 3072:
        rows = int(rng.choice([1, 2, 3, 17, 64, 255, 1024, 2049, 4096]))
    else:
        rows = int(rng.integers(1, (512 if V <= 32000 else 48) + 1))
    kind = int(rng.integers(0, 5))
    if kind == 0:
        x = rng.standard_normal((rows, V)) * rng.choice([0.3, 1.0, 3.0, 8.0], size=(rows, 1))
    elif kind == 1:  # Zipf-like: -log(rank), shuffled per row
        r = np.log(np.arange(1, V + 1))
        x = np.stack([-r[rng.permutation(V)] * rng.uniform(0.5, 2.0) for _ in range(rows)])
        x += rng.standard_normal((rows, V)) * 0.1
    elif kind == 2:  # integer values: many exact ties
        x = np.round(rng.standard_normal((rows, V)) * rng.choice([1.0, 2.0, 4.0], size=(rows, 1)))
    elif kind == 3:  # sparse spikes over a normal background
        x = rng.standard_normal((rows, V))
        x[rng.random((rows, V)) < 0.01] += rng.uniform(3, 12)
    else:  # 0.9 N(0, 1) + 0.1 N(4, 1)
        x = 0.9 * rng.standard_normal((rows, V)) + (4.0 + rng.standard_normal((rows, V))) * (rng.random((rows, V)) < 0.1)
    x = x.astype(np.float32)
    if rng.random() < 0.05:  # zeros of both signs
        z = rng.random((rows, V)) < 0.2
        x[z] = np.where(rng.random(int(z.sum())) < 0.5, np.float32(0.0), np.float32(-0.0))
    hmax = int(rng.choice([0, 16, 256, 512, 2048, 3000, 5000]))
    hl = rng.integers(0, hmax + 1, size=rows) if hmax else np.zeros(rows, np.int64)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = rng.integers(0, V, size=int(off[-1])).astype(np.int32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = (rng.random(rows) > 0.05).astype(np.int32)
    p["top_k"] = np.where(rng.random(rows) < rng.uniform(0, 1), rng.integers(1, 300, rows), 0)
    p["top_p"] = rng.choice([1.0, 0.999, 0.99, 0.95, 0.9, 0.8, 0.5, 0.1, 1e-6], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.3, 0.7, 0.9, 1.0, 1.3, 2.0], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.05, 1.1, 1.3, 0.9, 2.0], size=rows).astype(np.float32)
    supp = rng.random(rows) < 0.2
    sb = rng.integers(0, V, rows)
    p["supp_begin"] = np.where(supp, sb, 0)
    p["supp_end"] = np.where(supp, np.minimum(V, sb + rng.integers(1, V + 1, rows)), 0)
    p["keep_id"] = np.where(supp & (rng.random(rows) < 0.5), rng.integers(0, V, rows), -1)
    p["ban_id"] = np.where(rng.random(rows) < 0.1, rng.integers(0, V, rows), -1)
    if rng.random() < 0.05:  # rows outside the contract: NaN or +inf logits, a history id past V
        for r in rng.integers(0, rows, size=int(rng.integers(1, 4))):
            x[r, rng.integers(0, V)] = rng.choice([np.nan, np.inf])
        if hist.size:
            hist[rng.integers(0, hist.size)] = V + int(rng.integers(0, 3))
    u = rng.random(rows)
    path = str(rng.choice(["auto", "auto", "block", "wave"])) if V <= 3072 else "auto"
    small = rows * V <= 4_000_000
    want_probs = bool(rng.random() < 0.15) and small
    want_logits = bool(rng.random() < 0.15) and small
    # the entry point: host buffers (vxs_sample), device buffers with a padded leading dimension and
    # possibly a base one float past 16-byte alignment (vxs_sample_device), or the entry point that
    # allocates nothing (vxs_sample_noalloc); the last two return ids only
    api = "host" if want_probs or want_logits else str(rng.choice(["host", "host", "host", "device", "noalloc"]))
    pad, shift = int(rng.choice([0, 1, 3, 64])), int(rng.choice([0, 1]))
    label = (f"kind {kind} rows {rows} V {V} hmax {hmax} path {path} probs {int(want_probs)} "
             f"logits {int(want_logits)} api {api}" + (f" pad {pad} shift {shift}" if api == "device" else ""))
    return x, p, u, off, hist, path, want_probs, want_logits, (api, pad, shift), label


NOALLOC_UNSUPPORTED = -5  # VXS_ERR_UNSUPPORTED: the call does not fit the entry point's scratch


def gpu_ids(ctx, batch):
    """The batch through the chosen entry point; None when vxs_sample_noalloc declines its size."""
    x, p, u, off, hist, path, want_probs, want_logits, (api, pad, shift), _ = batch
    rows, V = x.shape
    if api == "host":
        return ctx.sample(x, p, u, off, hist, path=path, raise_on_error=False, want_probs=want_probs,
                          want_logits=want_logits)
    if api == "noalloc":
        from voxwerk_amd._lib import ptr

        ids = np.full(rows, -99, np.int32)
        rc = ctx._lib.vxs_sample_noalloc(ctx.handle, rows, V, ptr(x), V, ptr(off), ptr(hist), ptr(p), 1, ptr(u),
                                         ptr(ids), 0)
        if rc == NOALLOC_UNSUPPORTED and (ids == -99).all():
            return None
        bad = np.nonzero(ids < 0)[0]
        assert rc == (int(ids[bad[0]]) if bad.size else 0), (rc, ctx.last_error())  # the lowest failing row's code
        return ids
    from voxwerk_amd.hip import DeviceArray

    ld = V + pad
    buf = np.full(shift + rows * ld, np.nan, np.float32)  # pads hold NaN: never read
    buf[shift:].reshape(rows, ld)[:, :V] = x
    arrs = [DeviceArray.from_numpy(a) for a in (buf, p, u, off, hist if hist.size else np.zeros(1, np.int32))]
    d_ids = DeviceArray((rows,), np.int32)
    try:
        ctx.sample_device(rows, V, arrs[0].ptr + 4 * shift, ld, arrs[1], 1, arrs[2], d_ids, arrs[3], arrs[4],
                          path=path)
        ctx.synchronize()
        return d_ids.numpy()
    finally:
        for a in arrs + [d_ids]:
            a.free()


def run_batch(ctx, batch, threads: int = 16):
    """Sample one batch on the GPU and with the oracle; returns the parity report (write-back
    logits that differ from the oracle's on a row that did not fail count as unexplained)."""
    x, p, u, off, hist, path, want_probs, want_logits = batch[:8]
    out = gpu_ids(ctx, batch)
    if out is None:
        return None
    ids = out[0] if isinstance(out, tuple) else out
    ora = ref.sample(x, p, u, off, hist, threads=threads, want_probs=want_probs, want_logits=want_logits)
    rep = compare_ids(ids, ora)
    if want_probs:
        rep.max_prob_rel = prob_rel_error(out[2], ora["probs"], comparable_rows(ids, ora) & (ora["ids"] >= 0))
    if want_logits:
        ok = ora["ids"] >= 0
        same = (out[1].view(np.uint32) == ora["logits"].view(np.uint32)).all(axis=1)
        rep.unexplained += [int(r) for r in np.nonzero(ok & ~same)[0] if int(r) not in rep.unexplained]
    return rep


def sweep(ctx, seed: int, batches: int = 0, seconds: float = 0.0, threads: int = 16, log=print):
    """Run `batches` random batches (or as many as fit in `seconds`); stops at the first batch that
    misses the bar. Returns (totals, failing report or None)."""
    rng = np.random.default_rng(seed)
    end = time.time() + seconds
    tot = {"batches": 0, "rows": 0, "exact": 0, "draw_boundary": 0, "topp_boundary": 0, "max_prob_rel": 0.0}
    while (batches and tot["batches"] < batches) or (seconds and time.time() < end):
        batch = random_batch(rng)
        log(batch[-1])
        rep = run_batch(ctx, batch, threads)
        log(f"  {rep}" if rep is not None else "  (larger than the no-alloc scratch: skipped)")
        if rep is None:
            continue
        tot["batches"] += 1
        tot["rows"] += rep.rows
        tot["exact"] += rep.exact
        tot["draw_boundary"] += rep.draw_boundary
        tot["topp_boundary"] += rep.topp_boundary
        tot["max_prob_rel"] = max(tot["max_prob_rel"], rep.max_prob_rel)
        if rep.unexplained or rep.max_prob_rel > PROB_RTOL:
            return tot, rep
    return tot, None


def random_head_case(rng):
    """One random logit-head call: rows, k (a multiple of 8 up to 2048), n, leading-dimension pads,
    bf16 or int8 weights, real, integer-valued or partly non-finite hidden values."""
    rows = int(rng.choice([1, 2, 3, 5, 8, 9, 16, 24, 31, 32, 33, 48, 64]))
    k = 8 * int(rng.integers(1, 257))
    n = int(rng.integers(1, 400)) if rng.random() < 0.4 else int(rng.integers(2000, 5200))
    data = str(rng.choice(["real", "real", "integer", "nonfinite"]))
    return dict(rows=rows, k=k, n=n, padx=4 * int(rng.integers(0, 5)), padw=8 * int(rng.integers(0, 3)),
                pado=int(rng.integers(0, 9)), int8=bool(rng.random() < 0.3), data=data,
                seed=int(rng.integers(0, 2**31)))


def run_head_case(ctx, c) -> str:
    """Run one head call on the GPU and check it against the oracle; returns '' or what failed."""
    from oracle.head_np import head_bound, head_exact, head_int8_bound, head_int8_exact, pack_int8
    from voxwerk_amd.hip import DeviceArray

    rng = np.random.default_rng(c["seed"])
    rows, k, n = c["rows"], c["k"], c["n"]
    ldx, ldw, ldo = k + c["padx"], k + c["padw"], n + c["pado"]
    if c["data"] == "integer":
        x = rng.integers(-8, 9, (rows, k)).astype(np.float32)
        wf = rng.integers(-8, 9, (n, k)).astype(np.float32)
    else:
        x = rng.standard_normal((rows, k)).astype(np.float32)
        wf = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    if c["data"] == "nonfinite":
        for _ in range(int(rng.integers(1, 4))):
            x[rng.integers(0, rows), rng.integers(0, k)] = rng.choice([np.inf, -np.inf, np.nan])
    w = (wf.view(np.uint32) >> 16).astype(np.uint16)
    xp = np.zeros((rows, ldx), np.float32)
    xp[:, :k] = x
    wp = np.zeros((n, ldw), np.uint16)
    wp[:, :k] = w
    arrs = [DeviceArray.from_numpy(xp), DeviceArray.from_numpy(wp),
            DeviceArray.from_numpy(np.full((rows, ldo), 7.0, np.float32))]
    try:
        if c["int8"]:
            d_q = DeviceArray.from_numpy(np.full((n, ldw), 99, np.int8))
            d_s = DeviceArray((n,), np.float32)
            arrs += [d_q, d_s]
            ctx.head_pack_int8_device(k, n, arrs[1], ldw, d_q, ldw, d_s)
            ctx.head_int8_device(rows, k, n, arrs[0], ldx, d_q, ldw, d_s, arrs[2], ldo)
        else:
            ctx.head_device(rows, k, n, arrs[0], ldx, arrs[1], ldw, arrs[2], ldo)
        ctx.synchronize()
        out = arrs[2].numpy()
        if c["int8"]:
            q, scale = d_q.numpy()[:, :k], d_s.numpy()
    finally:
        for a in arrs:
            a.free()
    if not np.all(out[:, n:] == 7.0):
        return "wrote past n"
    got = out[:, :n].astype(np.float64)
    if c["int8"]:
        wq, ws = pack_int8(w)
        if not (np.array_equal(q, wq) and np.array_equal(scale.view(np.uint32), ws.view(np.uint32))):
            return "int8 packing differs from the oracle's"
        exact, bound = head_int8_exact(x, q, scale), head_int8_bound(x, q, scale)
    else:
        with np.errstate(invalid="ignore", over="ignore"):
            exact, bound = head_exact(x, w), head_bound(x, w)
    fin = np.isfinite(exact)
    for cls in (np.isnan, np.isposinf, np.isneginf):
        if not np.array_equal(cls(got), cls(exact)):
            return f"non-finite pattern differs ({cls.__name__})"
    if c["data"] == "integer" and not c["int8"] and not np.array_equal(got, exact):
        return "integer data not exact"
    err = np.abs(got[fin] - exact[fin])
    if not np.all(err <= bound[fin]):
        return f"outside the fp32 bound (max err/bound {np.max(err / np.maximum(bound[fin], 1e-300)):.3f})"
    return ""


def head_sweep(ctx, seed: int, cases: int, log=print) -> list:
    """`cases` random head calls; returns the failing cases with what failed."""
    rng = np.random.default_rng(seed)
    bad = []
    for _ in range(cases):
        c = random_head_case(rng)
        log(f"head {c}")
        why = run_head_case(ctx, c)
        if why:
            log(f"  FAILED: {why}")
            bad.append((c, why))
    return bad


def run_stats_batch(ctx, batch, counts=None) -> str:
    """The batch (vocabulary <= 3072) through the one-wave kernel's statistics build
    (vxs_sample_stats_device): ids equal to the timed kernel's (vxs_sample_device) and classified
    against the oracle; for the rows the one-wave nucleus regime samples, every entry's final
    probability against the oracle's: within 1e-5 relative above 2^-F * 1e5 (masses live on a 2^-F
    grid of exp(d)), within one grid step absolute everywhere, the kept sets equal except entries
    below one step; NaN for every other row. Returns '' or what failed."""
    from voxwerk_amd.hip import DeviceArray

    x, p, u, off, hist = batch[:5]
    rows, V = x.shape
    arrs = [DeviceArray.from_numpy(np.ascontiguousarray(a)) for a in (x, p, u, off, hist if hist.size else off)]
    d_ids, d_ids2 = DeviceArray((rows,), np.int32), DeviceArray((rows,), np.int32)
    d_st, d_pr = DeviceArray((rows, 4), np.float64), DeviceArray((rows, V), np.float64)
    try:
        ctx.sample_stats_device(rows, V, arrs[0], V, arrs[1], 1, arrs[2], d_ids, d_st, arrs[3], arrs[4], path="wave",
                                probs=d_pr)
        ctx.sample_device(rows, V, arrs[0], V, arrs[1], 1, arrs[2], d_ids2, arrs[3], arrs[4], path="wave")
        ctx.synchronize()
        ids, ids2, st, pr = d_ids.numpy(), d_ids2.numpy(), d_st.numpy(), d_pr.numpy()
    finally:
        for a in arrs + [d_ids, d_ids2, d_st, d_pr]:
            a.free()
    if not np.array_equal(ids, ids2):
        return "statistics build drew differently from the timed kernel"
    ora = ref.sample(x, p, u, off, hist, threads=16, want_probs=True)
    rep = compare_ids(ids, ora)
    if rep.unexplained:
        return f"ids: {rep}"
    wave = st[:, 3] == 0
    if not np.isnan(pr[~wave]).all():
        return "probabilities written for rows outside the one-wave nucleus regime"
    ok = wave & comparable_rows(ids, ora) & (ora["ids"] >= 0)
    po, pk = ora["probs"][ok], pr[ok]
    F = min(51, 53 - int(np.ceil(np.log2(V))))
    big = po >= 2.0 ** -F * 1e5
    rel = np.abs(pk[big] - po[big]) / po[big]
    if rel.max(initial=0.0) > 1e-5:
        return f"probability rel error {rel.max():.3e}"
    if not np.all(np.abs(pk - po) <= 2.0 ** -F + 1e-5 * po):
        return "probability abs error beyond one grid step"
    if not np.all(((pk > 0) == (po > 0)) | (po < 2.0 ** -F)):
        return "kept sets differ above the grid"
    if counts is not None:
        counts["rows"] += int(ok.sum())
        counts["probabilities"] += int(big.sum())
    return ""


def stats_sweep(ctx, seed: int, batches: int, log=print) -> list:
    """`batches` random batches of at most 3072 entries through run_stats_batch."""
    rng = np.random.default_rng(seed)
    bad, n = [], 0
    counts = {"rows": 0, "probabilities": 0}
    while n < batches:
        b = random_batch(rng)
        if b[0].shape[1] > 3072 or b[0].shape[0] > 2049:
            continue
        n += 1
        log("stats " + b[-1])
        why = run_stats_batch(ctx, b, counts)
        if why:
            log(f"  FAILED: {why}")
            bad.append((b[-1], why))
    log(f"one-wave nucleus rows compared: {counts['rows']}, probabilities above the grid: {counts['probabilities']}")
    return bad


def misc_sweep(ctx, seed: int, calls: int, log=print) -> list:
    """Random calls of the two other host entry points against the oracle: vxs_apply_repetition_penalty
    (rows 1-64, vocabularies up to 151,936, histories with repeats, penalties below, at and above 1
    and extreme ones, logits with zeros of both signs and subnormals): the rows bit-identical;
    vxs_argmax (ties, -inf entries, all -inf rows): the ids identical. Returns the failing calls."""
    rng = np.random.default_rng(seed)
    bad = []
    for _ in range(calls):
        V = int(rng.choice(VOCABS))
        rows = int(rng.integers(1, 65 if V <= 32000 else 5))
        x = (rng.standard_normal((rows, V)) * rng.choice([0.5, 3.0, 30.0])).astype(np.float32)
        if rng.random() < 0.3:
            x = np.round(x)
        special = rng.random((rows, V))
        x[special < 0.01] = np.float32(0.0)
        x[(special >= 0.01) & (special < 0.02)] = np.float32(-0.0)
        x[(special >= 0.02) & (special < 0.025)] = np.float32(1e-40)  # subnormal
        what = str(rng.choice(["penalty", "argmax"]))
        log(f"{what} rows {rows} V {V}")
        if what == "penalty":
            hl = rng.integers(0, 3000, size=rows)
            off = np.zeros(rows + 1, np.int32)
            off[1:] = np.cumsum(hl)
            hist = rng.integers(0, min(V, int(rng.choice([64, V]))), size=int(off[-1])).astype(np.int32)
            rho = float(rng.choice([1.0, 1.05, 1.3, 0.9, 2.0, 1e-30, 1e30, -1.5]))
            got, want = x.copy(), x.copy()
            ctx.apply_repetition_penalty(got, off, hist, rho)
            rc = ref.apply_penalty(want, off, hist, rho)
            if rc != 0 or not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
                log(f"  FAILED: penalty {rho} (oracle rc {rc})")
                bad.append(("penalty", rows, V, rho))
        else:
            x[rng.random((rows, V)) < 0.05] = -np.inf
            if rows > 1 and rng.random() < 0.2:
                x[0] = -np.inf
            got = ctx.argmax(x)
            want = np.array([ref.argmax(x[r]) for r in range(rows)], np.int32)
            if not np.array_equal(got, want):
                log(f"  FAILED: argmax {got[:8]} vs {want[:8]}")
                bad.append(("argmax", rows, V))
    return bad


def _i32(v: int) -> int:
    return ((v + 0x80000000) & 0xFFFFFFFF) - 0x80000000


def batch_sequence(ctx, seed: int, log=print) -> str:
    """One random sequence of batched stages over a resident history store (vxs_sample_batch): slots
    with random initial histories and seeds, then 3-12 stages, each over a random subset of the
    slots in a random order, with random options, append on or off and the uniforms from the host or
    from the slots' device generators. Each stage's ids must equal the CSR-history call on the
    host's copy of the histories (same kernels) and the oracle's (counted boundaries aside); after
    the sequence every slot's history must equal the host copy and every generator must continue as
    .NET's Random(seed) / Random(seed + 1) does. Returns '' or what failed."""
    from voxwerk_amd.sampler import DotNetRandom

    rng = np.random.default_rng(seed)
    nslots = int(rng.integers(1, 65))
    steps = int(rng.integers(3, 13))
    cap = int(rng.integers(steps + 1, 3000))
    V = int(rng.choice([2048, 3072, 3072, 8192, 151936]))
    maxrows = nslots if V <= 8192 else min(nslots, 8)
    hist = [list(rng.integers(0, V, size=int(rng.integers(0, cap - steps + 1)))) for _ in range(nslots)]
    seeds = [int(v) for v in rng.integers(-2**31, 2**31, nslots)]
    gens = {(s, st): DotNetRandom(sd if st == "talker" else _i32(sd + 1))
            for s, sd in enumerate(seeds) for st in ("talker", "sub")}
    log(f"batch sequence: {nslots} slots, cap {cap}, {steps} stages, V {V}")
    with ctx.history(nslots, cap) as store:
        for s in range(nslots):
            store.set(s, hist[s])
            store.seed(s, seeds[s])
        for t in range(steps):
            rows = int(rng.integers(1, maxrows + 1))
            slots = rng.permutation(nslots)[:rows].astype(np.int32)
            x = (rng.standard_normal((rows, V)) * rng.choice([1.0, 3.0])).astype(np.float32)
            x[:, :64] += 3.0  # ids the histories often hold: the penalty decides draws
            p = np.zeros(rows, dtype=PARAMS_DTYPE)
            p["do_sample"] = (rng.random(rows) > 0.1).astype(np.int32)
            p["top_k"] = rng.choice([0, 1, 20, 50, 256, 300], size=rows)
            p["top_p"] = rng.choice([1.0, 0.95, 0.8, 0.3], size=rows).astype(np.float32)
            p["temperature"] = rng.choice([0.7, 0.9, 1.0, 1.3], size=rows).astype(np.float32)
            p["rep_penalty"] = rng.choice([1.05, 1.3, 0.9, 1.0], size=rows).astype(np.float32)
            p["supp_begin"], p["supp_end"] = max(V - 1024, 0), V
            p["keep_id"], p["ban_id"] = min(2150, V - 1), -1
            append = bool(rng.random() < 0.7)
            mode = str(rng.choice(["host", "talker", "sub"]))
            path = str(rng.choice(["auto", "block", "wave"])) if V <= 3072 else "auto"
            if mode == "host":
                u = rng.random(rows)
            else:
                u = np.array([gens[(int(s), mode)].NextDouble() if p["do_sample"][r] else 0.0
                              for r, s in enumerate(slots)])
            off = np.zeros(rows + 1, np.int32)
            off[1:] = np.cumsum([len(hist[s]) for s in slots])
            ids_csr = np.array([i for s in slots for i in hist[s]], np.int32)
            want = ctx.sample(x, p, u, off, ids_csr, path=path)
            got = ctx.sample_batch(store, x, slots, p, None if mode != "host" else u, append=append, path=path,
                                   rng=None if mode == "host" else mode)
            if not np.array_equal(got, want):
                return f"stage {t} ({mode}, append {append}): resident {got[:8]} vs CSR {want[:8]}"
            c = ref.classify(got, ref.sample(x, p, u, off, ids_csr))
            if c["unexplained"]:
                return f"stage {t}: {c}"
            if append:
                for r, s in enumerate(slots):
                    hist[s].append(int(got[r]))
        for s in range(nslots):
            if store.get(s).tolist() != [int(i) for i in hist[s]]:
                return f"slot {s}: history differs from the host copy"
            for st in ("talker", "sub"):
                if store.draw(s, st, 2).tolist() != [gens[(s, st)].NextDouble() for _ in range(2)]:
                    return f"slot {s}: generator {st} out of step"
    return ""


def batch_sweep(ctx, seed: int, sequences: int, log=print) -> list:
    rng = np.random.default_rng(seed)
    bad = []
    for _ in range(sequences):
        sd = int(rng.integers(0, 2**31))
        why = batch_sequence(ctx, sd, log)
        if why:
            log(f"  FAILED (sequence seed {sd}): {why}")
            bad.append((sd, why))
    return bad


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--seconds", type=float, default=60.0)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--threads", type=int, default=16, help="oracle threads (at most one GPU's share of the host)")
    ap.add_argument("--heads", type=int, default=0, help="random logit-head calls to check first")
    ap.add_argument("--sequences", type=int, default=0, help="random batched-stage sequences to check first")
    ap.add_argument("--misc", type=int, default=0, help="random penalty and argmax host calls to check first")
    ap.add_argument("--stats", type=int, default=0,
                    help="random batches through the one-wave kernel's statistics build to check first")
    args = ap.parse_args()
    from voxwerk_amd.sampler import Context

    ctx = Context(0)
    if args.heads:
        bad = head_sweep(ctx, args.seed, args.heads, log=lambda s: print(s, flush=True))
        print(f"HEADS {args.heads} calls, {len(bad)} failed", flush=True)
        if bad:
            sys.exit(1)
    if args.stats:
        bad = stats_sweep(ctx, args.seed, args.stats, log=lambda s: print(s, flush=True))
        print(f"STATS {args.stats} batches, {len(bad)} failed", flush=True)
        if bad:
            sys.exit(1)
    if args.misc:
        bad = misc_sweep(ctx, args.seed, args.misc, log=lambda s: print(s, flush=True))
        print(f"MISC {args.misc} calls, {len(bad)} failed", flush=True)
        if bad:
            sys.exit(1)
    if args.sequences:
        bad = batch_sweep(ctx, args.seed, args.sequences, log=lambda s: print(s, flush=True))
        print(f"SEQUENCES {args.sequences}, {len(bad)} failed", flush=True)
        if bad:
            sys.exit(1)
    tot, bad = sweep(ctx, args.seed, seconds=args.seconds, threads=args.threads, log=lambda s: print(s, flush=True))
    print("TOTAL", tot, flush=True)
    if bad is not None:
        print("FAILED", bad, "rows", bad.unexplained[:20], flush=True)
        sys.exit(1)


if __name__ == "__main__":
    main()
