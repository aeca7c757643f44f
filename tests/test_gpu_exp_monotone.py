"""The one-wave path orders top-p candidates by their fp32 nucleus masses (vxs_wave.h). That order is
the reference's (logit, index) order only while the mass function is monotone non-decreasing, a
property of the device's exp2 instruction; this test checks both exponentials (nucleus_exp, the masses
of vocabularies up to 8192, and exp_neg, the streaming kernel's) on every float in [-128, 0] on the
device under test, with their accuracy against the double-precision exp: exp_neg within 2 ulps,
nucleus_exp within its stated bound |d| * 7.4e-8 + 1.2e-7 relative."""
from __future__ import annotations

import json
import os
import subprocess

import pytest

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "voxwerk_amd", "lib")


@pytest.mark.gpu
def test_exponentials_monotone_and_accurate():
    exe = os.path.join(LIB, "vxs_selfcheck")
    assert os.path.exists(exe), "vxs_selfcheck is not built (run __graft_entry__.build())"
    p = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    r = json.loads(p.stdout.strip().splitlines()[-1])
    print(r)
    assert r["values"] == 0x43000001
    assert r["max_step_back_ulp"] == 0, r
    assert r["max_err_ulp"] < 2.0, r
    assert r["nucleus_max_step_back_ulp"] == 0, r
    assert r["nucleus_max_excess"] <= 1.2e-7, r
