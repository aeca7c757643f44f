"""Parity bookkeeping shared by the GPU tests: exact-id matches, boundary-classified differences and
probability agreement against the CPU oracle."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

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
