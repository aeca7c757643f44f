"""CPU checks that pin the oracle (oracle/vxs_oracle.c and oracle/sampler_np.py) to the reference's
sampling rules (src/Voxwerk/Talker/Sampler.cs:25-95, TalkerGenerator.cs:247-248).

Each rule is checked against something other than its own formula: hand-derived known answers
(tests/golden/kat.json), exact rational arithmetic, Hugging Face's logits processors (an independent
implementation of the same penalty / top-k / top-p rules) on CPU torch, brute force on tiny rows,
textbook special cases (k = 1, p -> 0, uniform rows, u = 0), a chi-square test of the draw, and a
second, differently built restatement (sampler_np) that must agree bit for bit.
"""
from __future__ import annotations

import itertools
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import ref, sampler_np

F32 = np.float32
NINF = -np.inf
HERE = os.path.dirname(os.path.abspath(__file__))


def P(do_sample=1, top_k=0, top_p=1.0, temperature=1.0, rep_penalty=1.0, supp_begin=0, supp_end=0, keep_id=-1,
      ban_id=-1) -> np.ndarray:
    p = np.zeros((), dtype=ref.PARAMS_DTYPE)
    p["do_sample"], p["top_k"], p["top_p"], p["temperature"] = do_sample, top_k, top_p, temperature
    p["rep_penalty"], p["supp_begin"], p["supp_end"] = rep_penalty, supp_begin, supp_end
    p["keep_id"], p["ban_id"] = keep_id, ban_id
    return p


def run1(x, p, u=0.0, hist=None, **kw):
    x = np.asarray(x, dtype=F32).reshape(1, -1)
    off = ids = None
    if hist is not None:
        ids = np.asarray(hist, dtype=np.int32)
        off = np.array([0, ids.size], np.int32)
    return ref.sample(x, p, np.array([u]), off, ids, **kw)


@pytest.fixture(scope="module", autouse=True)
def _built():
    ref.build()


# ---------------------------------------------------------------------------------------------
# hand-derived known answers
# ---------------------------------------------------------------------------------------------
KATS = json.load(open(os.path.join(HERE, "golden", "kat.json")))["cases"]


@pytest.mark.parametrize("case", KATS, ids=[c["name"] for c in KATS])
def test_known_answers(case):
    p = P(**case["params"])
    o = run1(case["logits"], p, case["u"], case.get("hist"), want_logits=True)
    assert o["rc"] == 0
    assert o["ids"][0] == case["expected_id"], case["why"]
    if "expected_logits" in case:
        want = np.asarray(case["expected_logits"], dtype=F32)
        got = o["logits"][0]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (got, want)
    # the numpy restatement agrees
    i, xs, _ = sampler_np.sample_row(case["logits"], case.get("hist", []), p, case["u"])
    assert i == case["expected_id"]


# ---------------------------------------------------------------------------------------------
# S1 repetition penalty
# ---------------------------------------------------------------------------------------------
def _penalised(x, hist, rho):
    y = np.array(x, dtype=F32, copy=True).reshape(1, -1)
    assert ref.apply_penalty(y, np.array([0, len(hist)], np.int32), np.asarray(hist, np.int32), rho) == 0
    return y[0]


@pytest.mark.parametrize("rho", [1.05, 1.1, 0.9, 1.3333, 7.77, 0.123])
def test_penalty_correctly_rounded(rho):
    """Every penalised value is the correctly rounded binary32 quotient / product (checked through
    binary64, which is exact-then-round for one op on binary32 operands)."""
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(F32) * F32(30),
                        (rng.standard_normal(2000) * 1e-30).astype(F32),
                        np.array([0.0, -0.0, NINF, 3.4e38, -3.4e38, 1e-45, -1e-45], F32)])
    y = _penalised(x, np.arange(x.size), rho)
    r = float(F32(rho))
    want = np.where(x < 0, (x.astype(np.float64) * r), (x.astype(np.float64) / r)).astype(F32)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_penalty_matches_hf_processor():
    torch = pytest.importorskip("torch")
    lp = pytest.importorskip("transformers.generation.logits_process")
    rng = np.random.default_rng(2)
    for rho in (1.05, 1.1, 1.3):
        x = (rng.standard_normal(3072) * 4).astype(F32)
        hist = rng.integers(0, 3072, 700)
        y = _penalised(x, hist, rho)
        proc = lp.RepetitionPenaltyLogitsProcessor(penalty=float(F32(rho)))
        hf = proc(torch.from_numpy(hist.reshape(1, -1)), torch.from_numpy(x.reshape(1, -1).copy()))[0].numpy()
        assert np.array_equal(y, hf)


def test_penalty_invariances():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(512) * 3).astype(F32)
    hist = rng.integers(0, 512, 300)
    a = _penalised(x, hist, 1.05)
    b = _penalised(x, rng.permutation(hist), 1.05)
    c = _penalised(x, np.concatenate([hist, hist, hist[:50]]), 1.05)
    d = _penalised(x, np.unique(hist), 1.05)
    assert np.array_equal(a, b) and np.array_equal(a, c) and np.array_equal(a, d)
    assert np.array_equal(_penalised(x, hist, 1.0), x)  # rho = 1 is the identity
    untouched = np.setdiff1d(np.arange(512), hist)
    assert np.array_equal(a[untouched], x[untouched])


def test_penalty_rejects_out_of_range_ids():
    x = np.zeros((1, 8), F32)
    assert ref.apply_penalty(x, np.array([0, 1], np.int32), np.array([8], np.int32), 1.1) == -2
    o = run1(np.zeros(8), P(rep_penalty=1.1), 0.5, hist=[3, -1])
    assert o["rc"] == -2 and o["ids"][0] == -2


# ---------------------------------------------------------------------------------------------
# S3 greedy, S4 temperature
# ---------------------------------------------------------------------------------------------
def test_greedy_is_first_index_argmax():
    rng = np.random.default_rng(4)
    for n in (1, 2, 7, 3072):
        for _ in range(20):
            x = rng.integers(-3, 4, n).astype(F32)  # many ties
            assert run1(x, P(do_sample=0))["ids"][0] == int(np.argmax(x)) == ref.argmax(x)


def test_temperature_constants():
    """fl32(1/T) at the benchmarked temperatures, from exact rationals."""
    for t, bits in ((0.9, 0x3F8E38E4), (0.7, 0x3FB6DB6E), (1.0, 0x3F800000)):
        inv = F32(float(1 / Fraction(float(F32(t)))))
        assert int(inv.view(np.uint32)) == bits
        o = run1([1.0, 2.0], P(temperature=t), want_logits=True)
        assert o["logits"][0][0] == inv


def test_temperature_scales_every_entry():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(3000) * 5).astype(F32)
    for t in (0.9, 0.7, 1.3, 0.05):
        inv = float(F32(float(1 / Fraction(float(F32(t))))))
        want = (x.astype(np.float64) * inv).astype(F32)  # exact product, one rounding
        o = run1(x, P(temperature=t), want_logits=True)
        assert np.array_equal(o["logits"][0], want)


def test_nonfinite_rejected():
    assert run1([1.0, np.nan, 0.0], P())["rc"] == -3
    assert run1([1.0, np.inf, 0.0], P())["rc"] == -3
    assert run1([1.0, np.nan, 0.0], P(do_sample=0))["rc"] == -3
    assert run1([1.0, np.inf, 0.0], P(do_sample=0))["ids"][0] == 1  # +inf is an ordinary greedy maximum
    assert run1([3e38, 1.0], P(temperature=0.1))["rc"] == -3  # overflow to +inf after temperature


# ---------------------------------------------------------------------------------------------
# S5 top-k
# ---------------------------------------------------------------------------------------------
def _mask_after(x, **kw):
    o = run1(x, P(**kw), want_logits=True, want_info=True)
    return o["logits"][0] != NINF, o


def test_top_k_brute_force_and_invariants():
    rng = np.random.default_rng(6)
    for n in (5, 64, 3072):
        for k in (1, 2, 3, min(50, n - 1), n - 1):
            x = np.round(rng.standard_normal(n) * 2, 1).astype(F32)  # rounded: ties
            kept, o = _mask_after(x, top_k=k)
            kth = sorted(x.tolist())[n - k]  # k-th largest with multiplicity
            assert o["info"]["kth"][0] == F32(kth)
            assert np.array_equal(kept, x >= F32(kth))
            assert kept.sum() >= k
            assert x[kept].min() >= (x[~kept].max() if (~kept).any() else NINF)


def test_top_k_matches_hf_warper():
    torch = pytest.importorskip("torch")
    lp = pytest.importorskip("transformers.generation.logits_process")
    rng = np.random.default_rng(7)
    for k in (1, 50, 200):
        x = (rng.standard_normal(3072) * 3).astype(F32)
        kept, _ = _mask_after(x, top_k=k)
        hf = lp.TopKLogitsWarper(top_k=k)(None, torch.from_numpy(x.reshape(1, -1).copy()))[0].numpy()
        assert np.array_equal(kept, hf != NINF)


def test_top_k_one_without_ties_is_argmax():
    rng = np.random.default_rng(8)
    for _ in range(50):
        x = rng.standard_normal(100).astype(F32)
        o = run1(x, P(top_k=1), u=float(rng.random()))
        assert o["ids"][0] == int(np.argmax(x))


def test_top_k_disabled_outside_range():
    x = np.arange(6, dtype=F32)
    for k in (0, 6, 7, -1):
        kept, o = _mask_after(x, top_k=k)
        assert kept.all() and o["info"]["flags"][0] & 1 == 0


# ---------------------------------------------------------------------------------------------
# S6 softmax
# ---------------------------------------------------------------------------------------------
def test_softmax_closed_form():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(3072) * 3).astype(F32)
    o = run1(x, P(), want_probs=True)
    p = o["probs"][0]
    assert abs(math.fsum(p) - 1.0) < 1e-13  # each of the V quotients rounds once
    # extended precision reference of exp(fl32(x - m)) / sum
    d = (x - x.max()).astype(F32).astype(np.longdouble)
    e = np.exp(d)
    q = e / e.sum()
    assert np.max(np.abs(p - q.astype(np.float64)) / q.astype(np.float64)) < 1e-14


# ---------------------------------------------------------------------------------------------
# S7 top-p
# ---------------------------------------------------------------------------------------------
def _topp_brute(p: np.ndarray, top_p: float) -> np.ndarray:
    """Kept mask by brute force over every prefix length of the stable ascending order."""
    thr = float(F32(1.0) - F32(top_p))
    order = sorted(range(p.size), key=lambda i: (p[i], i))
    best = 0
    for r in range(p.size):  # remove the r smallest (never all)
        if r <= p.size - 1 and math.fsum(p[order[:r]]) <= thr:
            best = r
        else:
            break
    kept = np.ones(p.size, bool)
    kept[order[:best]] = False
    return kept


def test_top_p_brute_force_tiny_rows():
    rng = np.random.default_rng(10)
    checked = 0
    for n in range(2, 8):
        for _ in range(150):
            x = (rng.standard_normal(n) * 2).astype(F32)
            top_p = float(rng.choice([0.3, 0.5, 0.8, 0.9, 0.95]))
            base = run1(x, P(), want_probs=True)["probs"][0]
            o = run1(x, P(top_p=top_p), want_probs=True)
            if o["info"]["topp_margin"][0] < 1e-9:
                continue  # fsum and the sequential sum may round differently on the boundary
            assert np.array_equal(o["probs"][0] > 0, _topp_brute(base, top_p))
            checked += 1
    assert checked > 700


def test_top_p_limits():
    x = np.array([1, 5, 5, 2, 5, 0], F32)
    o = run1(x, P(top_p=1e-7), want_probs=True)
    assert np.nonzero(o["probs"][0])[0].tolist() == [4]  # highest-index maximum only
    a = run1(x, P(top_p=1.0), want_probs=True)["probs"][0]
    b = run1(x, P(), want_probs=True)["probs"][0]
    assert np.array_equal(a, b)


def test_top_p_matches_hf_warper_away_from_ties():
    torch = pytest.importorskip("torch")
    lp = pytest.importorskip("transformers.generation.logits_process")
    rng = np.random.default_rng(11)
    compared = 0
    for top_p in (0.5, 0.8, 0.9, 0.95):
        for _ in range(10):
            x = (rng.standard_normal(3072) * 2).astype(F32)
            if np.unique(x).size != x.size:
                continue
            o = run1(x, P(top_p=top_p), want_probs=True)
            if o["info"]["topp_margin"][0] < 1e-5:
                continue  # HF sums in fp32: only cuts well away from the threshold are comparable
            warper = lp.TopPLogitsWarper(top_p=float(F32(top_p)))
            hf = warper(None, torch.from_numpy(x.reshape(1, -1).copy()))[0].numpy()
            assert np.array_equal(o["probs"][0] > 0, hf != NINF)
            compared += 1
    assert compared >= 30


# ---------------------------------------------------------------------------------------------
# S8 draw
# ---------------------------------------------------------------------------------------------
def test_draw_u_zero_and_uniform_rows():
    rng = np.random.default_rng(12)
    for m in (1, 2, 3, 10, 64, 3072):
        x = np.full(m, 0.25, F32)
        for u in rng.random(30):
            j = math.floor(u * m)
            if abs(u * m - round(u * m)) < 1e-6:
                continue
            assert run1(x, P(), float(u))["ids"][0] == j
    x = np.array([NINF, NINF, 0.5, 3.0, NINF, 1.0], F32)
    assert run1(x, P(), 0.0)["ids"][0] == 2


def test_draw_chi_square():
    stats = pytest.importorskip("scipy.stats")
    rng = np.random.default_rng(13)
    x = np.array([0.0, 1.0, -0.5, 2.0, 0.3, -2.0, 1.5, 0.7], F32)
    rows = 200000
    o = ref.sample(np.tile(x, (rows, 1)), P(temperature=0.9), rng.random(rows), threads=8, want_info=False)
    counts = np.bincount(o["ids"], minlength=x.size)
    p = run1(x, P(temperature=0.9), want_probs=True)["probs"][0]
    chi2, pv = stats.chisquare(counts, p * rows)
    assert pv > 1e-4, (chi2, pv)


def test_draw_is_inverse_cdf_in_index_order():
    rng = np.random.default_rng(14)
    for _ in range(200):
        n = int(rng.integers(2, 40))
        x = (rng.standard_normal(n) * 2).astype(F32)
        x[rng.random(n) < 0.3] = NINF
        if (x == NINF).all():
            continue
        u = float(rng.random())
        o = run1(x, P(), u, want_probs=True)
        p = o["probs"][0]
        if o["info"]["draw_margin"][0] < 1e-12:
            continue
        cum = np.add.accumulate(p)
        assert o["ids"][0] == int(np.searchsorted(cum, u, side="right"))


# ---------------------------------------------------------------------------------------------
# the two restatements agree bit for bit
# ---------------------------------------------------------------------------------------------
def _np_rows(b, rows):
    ids, probs = [], []
    for r in rows:
        h = b.hist_ids[b.hist_off[r]:b.hist_off[r + 1]]
        i, _, p = sampler_np.sample_row(b.logits[r], h, b.params[r], b.u[r])
        ids.append(i)
        probs.append(p)
    return np.array(ids), probs


@pytest.mark.parametrize("wid,rows", [(1, 1), (2, 16), (3, 24), (4, 24), (5, 2)])
def test_c_and_numpy_restatements_agree(wid, rows):
    from voxwerk_amd import workloads

    b = workloads.workload(wid).generate(rows=rows)
    o = ref.sample(b.logits, b.params, b.u, b.hist_off, b.hist_ids, threads=4, want_probs=True)
    ids, probs = _np_rows(b, range(rows))
    assert np.array_equal(ids, o["ids"])
    for r in range(rows):
        if probs[r] is not None:
            assert np.array_equal(probs[r], o["probs"][r])


def test_c_and_numpy_agree_on_mixed_options():
    rng = np.random.default_rng(15)
    for _ in range(300):
        n = int(rng.choice([3, 17, 100, 1000]))
        x = (rng.standard_normal(n) * rng.choice([0.5, 3, 20])).astype(F32)
        x[rng.random(n) < 0.05] = NINF
        p = P(do_sample=int(rng.random() < 0.85), top_k=int(rng.choice([0, 1, 5, 50, n])),
              top_p=float(rng.choice([1.0, 0.9, 0.5, 0.05])), temperature=float(rng.choice([1.0, 0.9, 0.7, 1.5])),
              rep_penalty=float(rng.choice([1.0, 1.05, 1.3])), supp_begin=n // 2, supp_end=n if rng.random() < 0.3 else 0,
              keep_id=n // 2 + 1, ban_id=int(rng.choice([-1, 0])))
        hist = rng.integers(0, n, int(rng.integers(0, 40)))
        u = float(rng.random())
        o = run1(x, p, u, hist, want_probs=True, want_logits=True)
        i, xs, pr = sampler_np.sample_row(x, hist, p, u)
        assert o["ids"][0] == i
        assert np.array_equal(o["logits"][0].view(np.uint32), xs.view(np.uint32))
        if pr is not None:
            assert np.array_equal(o["probs"][0], pr, equal_nan=True)


def test_planted_mistake_is_caught():
    """The cross-checks above fail on a plausible slip: dividing by T instead of multiplying by
    fl32(1/T), or summing top-p mass in descending order."""
    x = np.array([1.0009765625, 1.01171875, 1.0234375], F32)  # values where x/T != x*fl32(1/T)
    inv = F32(1.0) / F32(0.9)
    assert not np.array_equal(x * inv, (x / F32(0.9)).astype(F32))
    o = run1(x, P(temperature=0.9), want_logits=True)
    assert np.array_equal(o["logits"][0], x * inv)
    assert not np.array_equal(o["logits"][0], (x / F32(0.9)).astype(F32))


# ---------------------------------------------------------------------------------------------
# Embedding lookups of sampled ids (oracle/embedding_np.py)
# ---------------------------------------------------------------------------------------------
def test_embedding_widen_special_encodings():
    from oracle.embedding_np import widen

    got = widen(np.array([0x3F80, 0xC000, 0x7F80, 0xFF80, 0x0001, 0x8000, 0x4B80], np.uint16))
    assert got[0] == 1.0 and got[1] == -2.0
    assert np.isposinf(got[2]) and np.isneginf(got[3])
    assert got[4] == math.ldexp(1.0, -133)  # smallest bf16 subnormal: 2^-126 * 2^-7
    assert got[5] == 0.0 and math.copysign(1.0, float(got[5])) == -1.0
    assert got[6] == 2.0**24


def test_frame_embed_order_and_precision():
    """2^24 + 1 + 1 is 2^24 left to right in fp32 (each +1 ties to even), 2^24 + 2 in any other
    grouping or in fp64; (1 + 1) + 2^24 with the text row last is 2^24 + 2, 2^24 if it came first."""
    from oracle.embedding_np import embed, frame_embed

    codec = np.array([[0x4B80, 0x3F80]], np.uint16)  # row 0: [2^24, 1]
    cp = np.array([[[0x3F80, 0x3F80]], [[0x3F80, 0x0000]]], np.uint16)  # two code-predictor tables, 1 row each
    out, st = frame_embed(np.array([[0, 0, 0]]), codec, cp)
    assert st.tolist() == [0]
    assert out[0, 0] == 2.0**24 and out[0, 1] == 2.0
    out, _ = frame_embed(np.array([[0, 0]]), np.array([[0x3F80, 0x3F80]], np.uint16), cp[:1],
                         addend=np.array([[2.0**24, 0.0]], np.float32))
    assert out[0, 0] == 2.0**24 + 2 and out[0, 1] == 2.0
    prev = np.full((2, 2), 7.0, np.float32)
    out, st = frame_embed(np.array([[0, 0, 1], [1, 0, 0]]), codec, cp, out=prev.copy())
    assert st.tolist() == [-2, -2] and np.all(out == 7.0)  # bad ids: rows untouched
    o = np.full((2, 2), 2.0**24, np.float32)
    st = embed([0, 5], np.array([[0x3F80, 0x4000]], np.uint16), o, add=True)
    assert st.tolist() == [0, -2] and o[0].tolist() == [2.0**24, 2.0**24 + 2] and o[1, 0] == 2.0**24


# ---------------------------------------------------------------------------------------------
# Logit heads (oracle/head_np.py)
# ---------------------------------------------------------------------------------------------
def _bf16(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_head_exact_on_integers():
    """Small integers: every partial sum is exact in fp32, so any order gives the exact value."""
    from oracle.head_np import head_exact

    rng = np.random.default_rng(0)
    x = rng.integers(-8, 9, (3, 1024)).astype(np.float32)
    w = rng.integers(-8, 9, (40, 1024)).astype(np.float32)
    want = x.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(head_exact(x, _bf16(w)), want.astype(np.float64))


def test_head_bound_holds_for_fp32_sums_in_two_orders():
    from oracle.embedding_np import widen
    from oracle.head_np import head_bound, head_exact

    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 1024)).astype(np.float32)
    w = _bf16(rng.standard_normal((16, 1024)))
    exact, bound = head_exact(x, w), head_bound(x, w)
    wf = widen(w)
    for r in range(2):
        for n in range(16):
            prods = x[r] * wf[n]  # fp32 products (rounded once each)
            seq = np.float32(0)
            for p in prods:  # left to right
                seq = np.float32(seq + p)
            pair = prods.copy()  # pairwise tree
            while pair.size > 1:
                pair = (pair[0::2] + pair[1::2]).astype(np.float32)
            for got in (float(seq), float(pair[0])):
                assert abs(got - exact[r, n]) <= bound[r, n], (r, n)
    assert np.all(bound > 0) and np.all(bound < 1e-3 * np.abs(x).sum() * 4)


def test_pack_int8_hand_derived_rows():
    """FromBf16LinearInt8 on rows whose scale is exact: ties go to even, the extreme maps to 127."""
    from oracle.head_np import pack_int8

    w = _bf16(np.array([[127.0, -63.5, 2.5, 3.5, -0.5, 0.0, 1.5, -126.5],  # amax 127: scale 1
                        [254.0, 3.0, 5.0, -254.0, 1.0, -3.0, 0.0, 7.0],  # amax 254: scale 2, w/2
                        [0.0] * 8,  # all zero: scale 1, q 0
                        [-0.25, 0.125, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]], np.float32))  # amax 1/4
    q, scale = pack_int8(w)
    assert scale.tolist()[:3] == [1.0, 2.0, 1.0]
    assert q[0].tolist() == [127, -64, 2, 4, 0, 0, 2, -126]
    assert q[1].tolist() == [127, 2, 2, -127, 0, -2, 0, 4]
    assert q[2].tolist() == [0] * 8
    assert scale[3] == np.float32(0.25) / np.float32(127.0) and q[3].tolist()[:2] == [-127, 64]


def test_pack_int8_row_whose_inverse_scale_overflows():
    """amax below ~3.7e-37: scale = amax / 127 is tiny, 1 / scale overflows to +inf, so w * inf is
    +-inf (or NaN for w = 0); .NET 9+ saturating (int) casts and the clamp give +-127 and 0."""
    from oracle.head_np import pack_int8

    tiny = np.float32(2.0**-125)  # normal; tiny / 127 is subnormal and 1 / that overflows
    w = _bf16(np.array([[tiny, -tiny, 0.0, tiny / 2]], np.float32))
    q, scale = pack_int8(w)
    assert scale[0] == np.float32(tiny) / np.float32(127.0) and np.isinf(np.float32(1.0) / scale[0])
    assert q[0].tolist() == [127, -127, 0, 127]


def test_pack_int8_against_python_floats():
    """Per element in Python: the fp32 quotient and product as the correctly rounded value of the
    exact rational (fractions), round-half-even by Python's round(); differently computed."""
    from fractions import Fraction

    from oracle.embedding_np import widen
    from oracle.head_np import pack_int8

    rng = np.random.default_rng(5)
    w = _bf16(rng.standard_normal((12, 64)) * np.exp(rng.uniform(-6, 6, (12, 1))))
    q, scale = pack_int8(w)
    wf = widen(w)

    def f32(fr):  # nearest fp32 to a rational (fp32-normal range): exact via scaling
        e = int(np.floor(np.log2(abs(float(fr))))) if fr != 0 else 0
        m = fr / Fraction(2) ** (e - 23)
        n = round(m)  # ties to even
        return float(Fraction(n) * Fraction(2) ** (e - 23))

    for r in range(12):
        amax = max(abs(Fraction(float(v))) for v in wf[r])
        s = f32(amax / 127) if amax > 0 else 1.0
        inv = f32(1 / Fraction(s))
        assert float(scale[r]) == s
        for c in range(64):
            p = f32(Fraction(float(wf[r, c])) * Fraction(inv)) if wf[r, c] != 0 else 0.0
            assert int(q[r, c]) == max(-127, min(127, round(p))), (r, c)


def test_head_int8_bound_holds_for_both_reference_forms():
    from oracle.head_np import (head_int8_batched_fp32, head_int8_bound, head_int8_decode_fp32, head_int8_exact,
                                pack_int8)

    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    q, scale = pack_int8(_bf16(rng.standard_normal((20, 256)) * 0.05))
    exact, bound = head_int8_exact(x, q, scale), head_int8_bound(x, q, scale)
    for got in (head_int8_decode_fp32(x, q, scale), head_int8_batched_fp32(x, q, scale)):
        assert np.all(np.abs(got.astype(np.float64) - exact) <= bound)
    # integers with a power-of-two scale: exact in every order
    xi = rng.integers(-8, 9, (2, 256)).astype(np.float32)
    qi = rng.integers(-127, 128, (5, 256)).astype(np.int8)
    si = np.full(5, 0.5, np.float32)
    want = (xi.astype(np.int64) @ qi.astype(np.int64).T) * 0.5
    assert np.array_equal(head_int8_exact(xi, qi, si), want)
    assert np.array_equal(head_int8_decode_fp32(xi, qi, si).astype(np.float64), want)
