"""CPU checks of the host side: the C ABI library's exports and struct layout, the host mirror of the
reference's options and RNG, and the product/oracle separation. No GPU calls."""
from __future__ import annotations

import os
import re
import subprocess
import textwrap

import numpy as np
import pytest

from voxwerk_amd import _lib, build
from voxwerk_amd.sampler import (CODEC_EOS_ID, TALKER_VOCAB, DotNetRandom, GenerationOptions, SamplingOptions,
                                 _csr, make_params, sub_talker_params, talker_params)

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_header_symbols_are_exported():
    syms = _lib.header_symbols()
    assert {"vxs_create", "vxs_destroy", "vxs_sample", "vxs_sample_device", "vxs_last_error"} <= set(syms)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIBVXS], check=True, capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT\s+(vxs_\w+)", out))
    missing = [s for s in syms if s not in exported]
    assert not missing, f"declared in include/vxs_sampler.h but not exported: {missing}"
    assert set(_lib._SIGNATURES) | {"vxs_version"} >= set(syms)


def test_library_loads_and_reports_version():
    lib = _lib.load_vxs()
    for s in _lib.header_symbols():
        assert hasattr(lib, s)
    lib.vxs_version.restype = __import__("ctypes").c_char_p
    assert b"gfx950" in lib.vxs_version()


def test_params_struct_layout(tmp_path):
    """vxs_params as a C compiler lays it out == the numpy record the bindings pass."""
    src = tmp_path / "layout.c"
    src.write_text(textwrap.dedent("""
        #include <stdio.h>
        #include <stddef.h>
        #include "vxs_sampler.h"
        int main(void) {
            printf("%zu", sizeof(vxs_params));
            #define F(f) printf(" %s=%zu", #f, offsetof(vxs_params, f));
            F(do_sample) F(top_k) F(top_p) F(temperature) F(rep_penalty) F(supp_begin) F(supp_end) F(keep_id) F(ban_id)
            printf("\\n");
            return 0;
        }
    """))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert int(out[0]) == _lib.PARAMS_DTYPE.itemsize == 36
    for item in out[1:]:
        name, off = item.split("=")
        assert _lib.PARAMS_DTYPE.fields[name][1] == int(off)


def test_hip_build_flags():
    flags = " ".join(build.HIP_FLAGS)
    assert "--offload-arch=gfx950" in flags
    assert "-target-feature -Xclang -packed-fp32-ops" in flags
    assert "-ffp-contract=off" in flags


def test_product_never_touches_the_oracle():
    pkg = os.path.join(REPO, "voxwerk_amd")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h", ".c")):
                text = open(os.path.join(root, f), encoding="utf-8").read()
                assert not re.search(r"^\s*(from|import)\s+oracle|vxs_oracle|libvxs_oracle", text, re.M), f


# ---------------------------------------------------------------------------------------------
# options (Sampler.cs:4-13, TalkerGenerator.cs:7-22, Program.cs:217-229 defaults)
# ---------------------------------------------------------------------------------------------
def test_option_defaults():
    s = SamplingOptions()
    assert (s.DoSample, s.TopK, s.TopP, s.Temperature) == (True, 50, 1.0, 0.9)
    assert not SamplingOptions.Greedy().DoSample
    g = GenerationOptions()
    assert g.RepetitionPenalty == 1.05 and g.MaxNewTokens == 2048 and g.Seed is None
    assert not GenerationOptions.Greedy().Talker.DoSample and not GenerationOptions.Greedy().SubTalker.DoSample


def test_talker_params_suppression_and_eos_ban():
    g = GenerationOptions()
    for step in range(4):
        p = talker_params(g, step)
        assert (p["supp_begin"], p["supp_end"], p["keep_id"]) == (TALKER_VOCAB - 1024, TALKER_VOCAB, CODEC_EOS_ID)
        assert p["ban_id"] == (CODEC_EOS_ID if step < 2 else -1)
        assert p["rep_penalty"] == np.float32(1.05) and p["top_k"] == 50 and p["temperature"] == np.float32(0.9)
    c = sub_talker_params(g)
    assert c["rep_penalty"] == 1.0 and c["supp_end"] == 0 and c["ban_id"] == -1


def test_make_params_rounds_to_float32():
    p = make_params(SamplingOptions(TopP=0.95, Temperature=0.7), rep_penalty=1.1)
    assert p["top_p"] == np.float32(0.95) and p["temperature"] == np.float32(0.7)
    assert p["rep_penalty"] == np.float32(1.1)


def test_csr_histories():
    off, ids = _csr([[1, 2], [], [3, 3, 3]], 3)
    assert off.tolist() == [0, 2, 2, 5] and ids.tolist() == [1, 2, 3, 3, 3]
    with pytest.raises(ValueError):
        _csr([[1]], 2)


# ---------------------------------------------------------------------------------------------
# .NET System.Random(seed): legacy subtractive generator
# ---------------------------------------------------------------------------------------------
def test_dotnet_random_first_values():
    """First Next() of new Random(seed) for seeds 0, 1 and 42 as widely published for .NET's
    seeded generator. Recalled values, not produced by a .NET run here (none is available)."""
    assert DotNetRandom(0).Next() == 1559595546
    assert DotNetRandom(1).Next() == 534011718
    assert DotNetRandom(42).Next() == 1434747710


def test_dotnet_random_large_seeds_stay_in_range():
    """Seeds above MSEED overflow 32-bit arithmetic during seeding; C# wraps (unchecked int), and
    every InternalSample then stays in [0, int.MaxValue). A version with unbounded integers returns
    negative samples for most such seeds, which this catches."""
    rng = np.random.default_rng(0)
    seeds = [2**31 - 1, -(2**31), 10**9, 2 * 10**9, 161803399] + rng.integers(-2**31, 2**31, 200).tolist()
    for seed in seeds:
        r = DotNetRandom(int(seed))
        xs = [r.Next() for _ in range(200)]
        assert all(0 <= x < DotNetRandom.MBIG for x in xs), seed


def test_sub_seed_wraps_like_csharp():
    from voxwerk_amd.generate import _sub_seed
    from voxwerk_amd.sampler import GenerationOptions

    assert _sub_seed(GenerationOptions(Seed=7)) == 8
    assert _sub_seed(GenerationOptions(Seed=2**31 - 1)) == -(2**31)
    assert _sub_seed(GenerationOptions()) is None


def test_dotnet_random_next_double_range_and_determinism():
    a, b = DotNetRandom(7), DotNetRandom(7)
    xs = [a.NextDouble() for _ in range(10000)]
    assert xs == [b.NextDouble() for _ in range(10000)]
    assert 0.0 <= min(xs) and max(xs) < 1.0
    assert abs(np.mean(xs) - 0.5) < 0.01
    assert DotNetRandom(-5).Next() == DotNetRandom(5).Next()  # abs(seed), as .NET does


def test_committed_traffic_profile_feeds_the_roofline():
    """bench.py's roofline.traffic comes from the committed FETCH_SIZE + WRITE_SIZE summary of the
    headline kernel: it must parse, and lie within a few percent above the algorithmic bytes."""
    import bench

    traffic = bench.read_traffic()
    algorithmic = 4096 * (4 * 3072 + 4 * 512 + 4 + 8 + 4)
    assert traffic is not None, "profiles/traffic_full_vocab_nucleus_4096x3072.txt has no traffic_bytes_per_launch"
    assert algorithmic <= traffic <= 1.05 * algorithmic, (traffic, algorithmic)
