"""GPU tests of the host-pointer calls a managed binding makes one row at a time: write-back Select,
the repetition penalty and argmax complete by polling (the kernel stores ids and rows into coherent
host memory), with results bit-identical to the oracle's and failing rows left as the caller had them.
"""
import numpy as np
import pytest

from oracle import ref
from parity import compare_ids
from voxwerk_amd._lib import PARAMS_DTYPE, ptr
from voxwerk_amd.sampler import Sampler, SamplingOptions

pytestmark = pytest.mark.gpu
U32 = np.uint32


def _params(rows, rng):
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"] = 1
    p["do_sample"][::5] = 0
    p["top_k"] = rng.choice([0, 1, 50, 200], size=rows)
    p["top_p"] = rng.choice([1.0, 0.95, 0.8], size=rows).astype(np.float32)
    p["temperature"] = rng.choice([0.7, 0.9, 1.3], size=rows).astype(np.float32)
    p["rep_penalty"] = rng.choice([1.0, 1.05, 1.1], size=rows).astype(np.float32)
    p["supp_begin"] = 0
    p["supp_end"] = 0
    p["keep_id"] = -1
    p["ban_id"] = -1
    return p


@pytest.mark.parametrize("rows,vocab", [(1, 2048), (1, 3072), (16, 2048), (24, 3072), (40, 8192)])
def test_polled_write_back(ctx, rows, vocab):
    """Write-back without probabilities: up to 2 MiB of rows, written by the kernel into host memory.
    A row with a history id outside the vocabulary fails and keeps the caller's contents."""
    rng = np.random.default_rng(rows * 10007 + vocab)
    x = (rng.standard_normal((rows, vocab)) * 2.0).astype(np.float32)
    hl = rng.integers(0, 100, size=rows)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(hl)
    hist = rng.integers(0, vocab, size=off[-1]).astype(np.int32)
    bad_row = rows // 2 if rows > 1 and hl[rows // 2] > 0 else -1
    if bad_row >= 0:
        hist[off[bad_row]] = vocab
    p = _params(rows, rng)
    if bad_row >= 0:
        p["rep_penalty"][bad_row] = np.float32(1.1)  # a penalty of 1 reads no history (Sampler.cs:27)
    u = rng.random(rows)
    out = np.full((rows, vocab), 7.0, np.float32)
    ids, lg, _ = ctx.sample(x, p, u, off, hist, raise_on_error=False, logits_out=out, path="block")
    assert lg is out
    ora = ref.sample(x, p, u, off, hist, threads=8, want_logits=True)
    rep = compare_ids(ids, ora)
    print(f"write-back {rows}x{vocab}: {rep}", flush=True)
    assert not rep.unexplained
    ok = ids >= 0
    assert np.array_equal(out[ok].view(U32), ora["logits"][ok].view(U32))
    if bad_row >= 0:
        assert ids[bad_row] == -2
        assert np.all(out[bad_row] == 7.0), "a failed row's write-back buffer was overwritten"


def test_polled_penalty_strided_rows(ctx):
    """vxs_apply_repetition_penalty on rows with a leading dimension above the vocabulary: the
    penalised entries are bit-identical to the oracle's and the pads between rows are not touched;
    a call with an id outside the vocabulary changes nothing."""
    rng = np.random.default_rng(5)
    rows, vocab, ld = 12, 3000, 3072
    buf = rng.standard_normal((rows, ld)).astype(np.float32)
    buf[:, vocab:] = 99.0
    off = np.arange(rows + 1, dtype=np.int32) * 300
    hist = rng.integers(0, vocab, size=off[-1]).astype(np.int32)
    want = np.ascontiguousarray(buf[:, :vocab])
    assert ref.apply_penalty(want, off, hist, 1.1) == 0
    y = buf.copy()
    rc = ctx._lib.vxs_apply_repetition_penalty(ctx.handle, rows, vocab, ptr(y), ld, ptr(off), ptr(hist),
                                               float(np.float32(1.1)))
    assert rc == 0, ctx.last_error()
    assert np.array_equal(y[:, :vocab].view(U32), want.view(U32))
    assert np.all(y[:, vocab:] == 99.0)
    bad = hist.copy()
    bad[700] = -1
    z = buf.copy()
    rc = ctx._lib.vxs_apply_repetition_penalty(ctx.handle, rows, vocab, ptr(z), ld, ptr(off), ptr(bad),
                                               float(np.float32(1.1)))
    assert rc == -2
    assert np.array_equal(z.view(U32), buf.view(U32))


def test_sampler_select_sequence(ctx):
    """The managed Sampler's call pattern for one frame: 15 in-place Select calls on 2048-entry rows
    with one seeded generator, ids and rows against the oracle fed the same uniforms; then ArgMax
    and the static penalty on a talker row."""
    rng = np.random.default_rng(8)
    s = Sampler(seed=1234, context=ctx)
    shadow = Sampler(seed=1234, context=ctx)  # only its uniforms are used
    opts = SamplingOptions(DoSample=True, TopK=50, TopP=1.0, Temperature=0.9)
    from voxwerk_amd.sampler import make_params

    for g in range(15):
        row = (rng.standard_normal(2048) * 3.0).astype(np.float32)
        orig = row.copy()
        tok = s.Select(row, opts)
        u = np.array([shadow.NextUniform(opts)])
        ora = ref.sample(orig.reshape(1, -1), make_params(opts), u, threads=1, want_logits=True)
        rep = compare_ids(np.array([tok], np.int32), ora)
        assert not rep.unexplained, f"Select {g}: {tok} vs {ora['ids'][0]}"
        assert np.array_equal(row.view(U32), ora["logits"][0].view(U32)), f"Select {g}: row differs"
    talker = (rng.standard_normal(3072) * 2.0).astype(np.float32)
    assert Sampler.ArgMax(talker, context=ctx) == ref.argmax(talker)
    hist = rng.integers(0, 3072, 256)
    y = talker.copy()
    Sampler.ApplyRepetitionPenalty(y, hist, 1.05, context=ctx)
    z = talker.copy()
    assert ref.apply_penalty(z, np.array([0, hist.size], np.int32), hist.astype(np.int32), 1.05) == 0
    assert np.array_equal(y.view(U32), z.view(U32))
