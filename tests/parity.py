"""Parity bookkeeping shared by the GPU tests: exact-id matches, boundary-classified differences and
probability agreement against the CPU oracle."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from voxwerk_amd._lib import PARAMS_DTYPE

DRAW_BOUNDARY = 1e-6   # |u - CDF edge| below which a differing id is a counted boundary draw
TOPP_BOUNDARY = 1e-6   # |cum - (1 - top_p)| below which a differing cutoff is a counted boundary
PROB_RTOL = 1e-5       # relative tolerance on the final probabilities


@dataclass
class Report:
    rows: int
    exact: int
    draw_boundary: int
    topp_boundary: int
    unexplained: list
    max_prob_rel: float = 0.0

    def __str__(self):
        return (f"rows={self.rows} exact={self.exact} draw_boundary={self.draw_boundary} "
                f"topp_boundary={self.topp_boundary} unexplained={len(self.unexplained)} "
                f"max_prob_rel={self.max_prob_rel:.2e}")


def comparable_rows(gpu_ids: np.ndarray, ora: dict) -> np.ndarray:
    """Rows whose probabilities must agree: same id and a top-p cut away from its boundary (on the
    boundary the two cuts may keep different sets, which is counted, not a failure)."""
    return (gpu_ids == ora["ids"]) & ~(ora["info"]["topp_margin"] < TOPP_BOUNDARY)


def compare_ids(gpu_ids: np.ndarray, ora: dict) -> Report:
    ids = ora["ids"]
    info = ora["info"]
    same = gpu_ids == ids
    draw_b = info["draw_margin"] < DRAW_BOUNDARY
    topp_b = info["topp_margin"] < TOPP_BOUNDARY
    diff = ~same
    unexplained = np.nonzero(diff & ~draw_b & ~topp_b)[0].tolist()
    return Report(len(ids), int(same.sum()), int((diff & draw_b & ~topp_b).sum()), int((diff & topp_b).sum()),
                  unexplained)


def prob_rel_error(gpu_p: np.ndarray, ora_p: np.ndarray, rows_ok: np.ndarray) -> float:
    """Max relative error over entries the oracle keeps (p > 0); entries it drops must be 0 on the GPU."""
    worst = 0.0
    for r in np.nonzero(rows_ok)[0]:
        g, o = gpu_p[r], ora_p[r]
        if np.isnan(o).all():
            assert np.isnan(g).all()
            continue
        kept = o > 0
        assert np.all(g[~kept] == 0), f"row {r}: probability on an entry the oracle removed"
        rel = np.abs(g[kept] - o[kept]) / o[kept]
        if rel.size:
            worst = max(worst, float(rel.max()))
    return worst


def signed_zero_batch(rng, rows, vocab):
    """Rows whose k-th largest value is a zero present with both signs: K = 1 over zeros only,
    K at a tie of zeros after a few positive entries, and K inside the zeros, with the penalty on
    some zero entries (zeros keep their sign through it) and uniforms on both sides of 0.5. The
    reference compares floats, where -0 equals +0, so every zero ties at the k-th value."""
    x = rng.uniform(-9.0, -1.0, (rows, vocab)).astype(np.float32)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["top_p"] = rng.choice([1.0, 0.9], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([1.0, 0.7], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.1], size=rows).astype(np.float32)
    p["keep_id"], p["ban_id"] = -1, -1
    off = np.zeros(rows + 1, np.int32)
    hist = []
    for r in range(rows):
        pos = rng.permutation(vocab)
        nz = int(rng.integers(2, 9))
        zeros = pos[:nz]
        x[r, zeros] = np.where(rng.random(nz) < 0.5, np.float32(0.0), np.float32(-0.0))
        x[r, zeros[0]], x[r, zeros[1]] = np.float32(-0.0), np.float32(0.0)
        kind = r % 3
        if kind == 0:
            k = 1
        else:
            npos = int(rng.integers(1, 5))
            x[r, pos[nz:nz + npos]] = rng.uniform(0.5, 3.0, npos).astype(np.float32)
            k = npos + (1 if kind == 1 else int(rng.integers(1, nz + 1)))
        p["top_k"][r] = k
        h = np.concatenate([zeros[rng.random(nz) < 0.5], rng.integers(0, vocab, 20)]).astype(np.int32)
        hist.append(h)
        off[r + 1] = off[r] + len(h)
    u = np.where(np.arange(rows) % 2 == 0, rng.uniform(0.02, 0.48, rows), rng.uniform(0.52, 0.98, rows))
    return x, p, u, off, np.concatenate(hist)

