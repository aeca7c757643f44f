"""GPU checks against the committed fixtures and against exact arithmetic: hand-derived known answers
(tests/golden/kat.json), the stored workload ids, and an exhaustive sweep of the penalty's division
over whole binades."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import ref
from parity import compare_ids
from voxwerk_amd import workloads
from voxwerk_amd._lib import PARAMS_DTYPE

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "kat.json")))["cases"]
META = json.load(open(os.path.join(HERE, "golden", "workloads.json")))


def _params(d) -> np.ndarray:
    p = np.zeros((), dtype=PARAMS_DTYPE)
    for k, v in d.items():
        p[k] = v
    return p


@pytest.mark.parametrize("case", KATS, ids=[c["name"] for c in KATS])
def test_gpu_known_answers(ctx, case):
    x = np.asarray(case["logits"], dtype=np.float32).reshape(1, -1)
    off = ids = None
    if "hist" in case:
        ids = np.asarray(case["hist"], np.int32)
        off = np.array([0, ids.size], np.int32)
    got, lg, _ = ctx.sample(x, _params(case["params"]), np.array([case["u"]]), off, ids, want_logits=True)
    assert got[0] == case["expected_id"], case["why"]
    if "expected_logits" in case:
        want = np.asarray(case["expected_logits"], dtype=np.float32)
        assert np.array_equal(lg[0].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("wid", [1, 2, 3, 4, 5])
def test_gpu_matches_stored_ids(ctx, wid):
    m = META[str(wid)]
    w = workloads.workload(wid)
    with np.load(os.path.join(HERE, "golden", "workloads.npz"), allow_pickle=False) as z:
        for step in range(w.steps):
            b = w.generate(step=step, rows=m["rows"])
            assert b.digest() == m["digests"][step]
            gpu = ctx.sample(b.logits, b.params, b.u, b.hist_off, b.hist_ids)
            stored = z[f"w{wid}_s{step}_ids"]
            info = ref.sample(b.logits, b.params, b.u, b.hist_off, b.hist_ids, threads=8)
            assert np.array_equal(info["ids"], stored)
            rep = compare_ids(gpu, info)
            print(f"{w.name}[{step}] vs stored ids: {rep}", flush=True)
            assert not rep.unexplained


@pytest.mark.parametrize("rho", [1.05, 1.1, 0.9])
def test_gpu_penalty_whole_binades(ctx, rho):
    """Every binary32 value of [1, 2) and (-2, -1] through the GPU penalty, against the correctly
    rounded quotient / product. Division and multiplication by rho commute with scaling by powers of
    two, so one binade stands for every normal magnitude the device's fast path accepts; values at
    the extremes of the range and subnormals are added as well."""
    vocab = 8192
    mant = np.arange(1 << 23, dtype=np.uint32)
    pos = (np.uint32(127 << 23) | mant).view(np.float32)
    rng = np.random.default_rng(17)
    extra = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    extra = extra[np.isfinite(extra)]
    x = np.concatenate([pos, -pos, extra, np.array([0.0, -0.0, -np.inf], np.float32)])
    x = np.concatenate([x, np.zeros((-x.size) % vocab, np.float32)])
    rows = x.size // vocab
    y = x.reshape(rows, vocab).copy()
    hist = np.tile(np.arange(vocab, dtype=np.int32), rows)
    off = (np.arange(rows + 1, dtype=np.int64) * vocab).astype(np.int32)
    print(f"penalty sweep rho={rho} rows={rows} vocab={vocab}", flush=True)
    ctx.apply_repetition_penalty(y, off, hist, rho)
    r = float(np.float32(rho))
    with np.errstate(over="ignore"):
        want = np.where(x < 0, x.astype(np.float64) * r, x.astype(np.float64) / r).astype(np.float32)
    bad = np.nonzero(y.reshape(-1).view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first at x={x[bad[0]]!r}: {y.reshape(-1)[bad[0]]!r} != {want[bad[0]]!r}"
