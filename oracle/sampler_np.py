"""Independent numpy restatement of voxwerk's sampler (Sampler.cs:25-95, TalkerGenerator.cs:247-248).

TEST INFRASTRUCTURE ONLY: cross-checks the C oracle bit for bit. Built differently on purpose —
vectorised masks, numpy sort/lexsort, ``np.add.accumulate`` for the reference's sequential sums
(accumulate is a strictly left-to-right loop, unlike ``np.sum``'s pairwise tree) and ``math.exp``
(the platform libm, as .NET's Math.Exp) — so a slip in either restatement shows as a mismatch.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32


def penalty(x: np.ndarray, hist, rho) -> None:
    """Sampler.cs:25-33, in place on a float32 row."""
    rho = F32(rho)
    if rho == F32(1.0):
        return
    h = np.asarray(hist, dtype=np.int64)
    if h.size and (h.min() < 0 or h.max() >= x.size):
        raise IndexError("history id out of range")
    ids = np.unique(h)
    s = x[ids]
    x[ids] = np.where(s < 0, s * rho, s / rho).astype(F32)


def suppress(x: np.ndarray, supp_begin, supp_end, keep_id, ban_id) -> None:
    """TalkerGenerator.cs:247-248."""
    n = x.size
    idx = np.arange(n)
    mask = (idx >= supp_begin) & (idx < supp_end) & (idx != keep_id)
    x[mask] = -np.inf
    if 0 <= ban_id < n:
        x[ban_id] = -np.inf


def select(x: np.ndarray, do_sample, top_k, top_p, temperature, u):
    """Sampler.cs:35-88 on a float32 row (modified in place). Returns (id, probs or None)."""
    n = x.size
    if not do_sample:
        if np.isnan(x).any():
            raise ValueError("NaN logits")
        return int(np.argmax(x)), None
    inv = F32(1.0) / F32(temperature)
    x *= inv
    if np.isnan(x).any() or (x == np.inf).any():
        raise ValueError("non-finite logits")
    if 0 < top_k < n:
        kth = np.sort(x)[n - top_k]
        x[x < kth] = -np.inf
    m = x.max()
    fin = x != -np.inf
    d = (x - m).astype(F32)
    e = np.zeros(n, dtype=np.float64)
    e[fin] = [math.exp(float(v)) for v in d[fin]]
    s = np.add.accumulate(e)[-1]
    with np.errstate(invalid="ignore", divide="ignore"):
        p = e / s
    if F32(top_p) < F32(1.0):
        thr = float(F32(1.0) - F32(top_p))
        if np.isnan(p).any():
            order = np.arange(n)  # all-NaN row: equal keys, index order
        else:
            order = np.lexsort((np.arange(n), p))
        cum = np.add.accumulate(p[order])
        above = np.nonzero(~(cum[: n - 1] <= thr))[0]
        nrem = int(above[0]) if above.size else n - 1
        p[order[:nrem]] = 0.0
        s2 = np.add.accumulate(p)[-1]
        with np.errstate(invalid="ignore", divide="ignore"):
            p = p / s2
    pos = ~(p <= 0)  # NaN counts as not <= 0, like the reference's `probs[i] <= 0` skip
    if not pos.any():
        return 0, p
    idx = np.nonzero(pos)[0]
    acc = np.add.accumulate(p[idx])
    hit = np.nonzero(u < acc)[0]
    return (int(idx[hit[0]]) if hit.size else int(idx[-1])), p


def sample_row(logits, hist, params, u):
    """Full per-row path: penalty -> suppression -> select. Returns (id, processed logits, probs)."""
    x = np.array(logits, dtype=F32, copy=True)
    penalty(x, hist, params["rep_penalty"])
    suppress(x, int(params["supp_begin"]), int(params["supp_end"]), int(params["keep_id"]), int(params["ban_id"]))
    i, p = select(x, bool(params["do_sample"]), int(params["top_k"]), F32(params["top_p"]),
                  F32(params["temperature"]), float(u))
    return i, x, p
