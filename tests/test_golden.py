"""The committed fixtures (tests/golden/, written by make_golden.py): the generator still produces the
same inputs, and the oracle still produces the same ids and probabilities on them."""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest

from oracle import ref
from voxwerk_amd import workloads

HERE = os.path.dirname(os.path.abspath(__file__))
META = json.load(open(os.path.join(HERE, "golden", "workloads.json")))


@pytest.fixture(scope="module")
def arrays():
    with np.load(os.path.join(HERE, "golden", "workloads.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("wid", [1, 2, 3, 4, 5])
def test_workload_inputs_and_oracle_ids(wid, arrays):
    m = META[str(wid)]
    w = workloads.workload(wid)
    assert (w.name, w.vocab, w.steps) == (m["name"], m["vocab"], m["steps"])
    for step in range(w.steps):
        b = w.generate(step=step, rows=m["rows"])
        assert b.digest() == m["digests"][step], f"generator output changed ({w.name} step {step})"
        o = ref.sample(b.logits, b.params, b.u, b.hist_off, b.hist_ids, threads=8, want_info=False)
        assert np.array_equal(o["ids"], arrays[f"w{wid}_s{step}_ids"])
        assert _sha(o["ids"]) == m["id_sha256"][step]


@pytest.mark.parametrize("wid", [1, 2])
def test_full_input_fixtures(wid, arrays):
    """The talker step and the first code-predictor step are stored whole: the oracle reproduces the
    stored ids and probabilities from the stored inputs alone."""
    a = {k[len(f"w{wid}_"):]: v for k, v in arrays.items() if k.startswith(f"w{wid}_")}
    o = ref.sample(a["logits"], a["params"], a["u"], a["hist_off"], a["hist_ids"], want_probs=True)
    assert np.array_equal(o["ids"], a["s0_ids"])
    assert np.array_equal(o["probs"], a["probs"])
    p = a["probs"]
    assert np.all(np.abs(p.sum(axis=1) - 1.0) < 1e-12)
