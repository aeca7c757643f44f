"""GPU: the draw of the exact regime (rows with at most 64 candidates, e.g. top-k 50) with u placed
on the running sums of the row's own probabilities.

A call that returns probabilities runs the reference's sequential sums (Sampler.cs:51-75) and hands
back every final probability; the running sum over them in index order is the value the reference's
draw compares u against (Sampler.cs:77-86: the first entry with u < acc, skipping p <= 0, else the
last entry with p > 0). Calls without outputs decide the draw (and, under top-p, the second sum) by
wave sums unless u lies within their rounding band of a deciding running sum, where the sequential
form runs. With u on such a sum, one ulp either side of it, or 2^-44 either side (inside the band),
both paths must draw exactly the entry the sequential rule names, as must the call with outputs.
"""
import math

import numpy as np
import pytest

from voxwerk_amd._lib import PARAMS_DTYPE

pytestmark = pytest.mark.gpu


def sequential_draw(prob_row: np.ndarray, u: float) -> int:
    """Sampler.cs:77-86 over one row of final probabilities (Python floats: IEEE double adds in
    index order)."""
    acc, last = 0.0, 0
    for i in np.flatnonzero(prob_row > 0.0):
        acc += float(prob_row[i])
        last = int(i)
        if u < acc:
            return int(i)
    return last


def edge_uniforms(probs: np.ndarray) -> np.ndarray:
    """One u per row on (or next to) one of the row's running sums, cycling over the placements."""
    rows = probs.shape[0]
    u = np.empty(rows, dtype=np.float64)
    for r in range(rows):
        kept = np.flatnonzero(probs[r] > 0.0)
        acc = []
        a = 0.0
        for i in kept:
            a += float(probs[r, i])
            acc.append(a)
        at = acc[(r * 7) % len(acc)]
        mode = r % 6
        u[r] = (at, math.nextafter(at, -math.inf), math.nextafter(at, math.inf), at - 2.0 ** -44, at + 2.0 ** -44,
                acc[-1])[mode]
    return u


@pytest.mark.parametrize("vocab", [2048, 3072])
@pytest.mark.parametrize("top_p", [1.0, 0.9])
def test_exact_draw_on_running_sums(ctx, vocab, top_p):
    rows = 192
    rng = np.random.default_rng(vocab + int(top_p * 100))
    x = (rng.standard_normal((rows, vocab)) * 2.5).astype(np.float32)
    x[::5, 7] = x[::5, 9]  # some exact ties inside the candidates
    p = np.zeros(1, dtype=PARAMS_DTYPE)
    p["do_sample"], p["top_k"], p["top_p"], p["temperature"] = 1, 50, np.float32(top_p), np.float32(0.9)
    p["rep_penalty"], p["keep_id"], p["ban_id"] = np.float32(1.0), -1, -1
    _, _, probs = ctx.sample(x, p, rng.random(rows), want_probs=True, path="block")
    assert np.all((probs > 0).sum(axis=1) <= 64), "rows must stay in the exact regime"
    u = edge_uniforms(probs)
    want = np.array([sequential_draw(probs[r], u[r]) for r in range(rows)], dtype=np.int32)
    for path in ("block", "wave"):
        got = ctx.sample(x, p, u, path=path)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"{path}: rows {bad[:10].tolist()} drew {got[bad[:10]].tolist()}, want {want[bad[:10]].tolist()}"
    ids_seq, _, probs2 = ctx.sample(x, p, u, want_probs=True, path="block")
    assert np.array_equal(ids_seq, want)
    assert np.array_equal(probs2, probs)


@pytest.mark.parametrize("top_p", [1.0, 0.9])
def test_exact_draw_out_of_range_uniforms(ctx, top_p):
    """u outside [0, 1) (a caller's, never NextDouble's): the reference's loop still defines the id
    (u >= every running sum or NaN: the last entry with p > 0; u < 0: the first), and the wave-sum
    draw must give it on both paths."""
    rows, vocab = 64, 2048
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((rows, vocab)) * 2.5).astype(np.float32)
    p = np.zeros(1, dtype=PARAMS_DTYPE)
    p["do_sample"], p["top_k"], p["top_p"], p["temperature"] = 1, 50, np.float32(top_p), np.float32(0.9)
    p["rep_penalty"], p["keep_id"], p["ban_id"] = np.float32(1.0), -1, -1
    _, _, probs = ctx.sample(x, p, rng.random(rows), want_probs=True, path="block")
    u = np.array([(1.0, 1.5, np.nan, -0.5, np.inf, -np.inf)[r % 6] for r in range(rows)], dtype=np.float64)
    want = np.array([sequential_draw(probs[r], u[r]) for r in range(rows)], dtype=np.int32)
    kept = [np.flatnonzero(probs[r] > 0.0) for r in range(rows)]
    assert all(want[r] == (kept[r][0] if u[r] < 0 else kept[r][-1]) for r in range(rows))
    for path in ("block", "wave"):
        got = ctx.sample(x, p, u, path=path)
        assert np.array_equal(got, want), f"{path}: rows {np.flatnonzero(got != want)[:10].tolist()}"
