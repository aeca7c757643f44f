"""GPU: the logit heads (vxs_head_device, and the int8 form vxs_head_int8_device with its packing
vxs_head_pack_int8_device) through the C ABI against the oracle (oracle/head_np.py), and the
device-resident step head -> sampler -> embedding.

Bar: exact on integer data (every order is exact); within gamma_K * sum|x w| of the exact dot
product otherwise (the bound the reference's own fp32 order also satisfies); sampled ids on the
head's logits identical to the oracle's on the same logits (boundary rows counted); embeddings
bit-identical."""
import numpy as np
import pytest

from oracle import ref
from oracle.embedding_np import embed
from oracle.head_np import (head_bound, head_exact, head_int8_batched_fp32, head_int8_bound, head_int8_decode_fp32,
                            head_int8_exact, pack_int8)
from voxwerk_amd._lib import PARAMS_DTYPE
from voxwerk_amd.hip import DeviceArray

pytestmark = pytest.mark.gpu


def _bf16(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _run(ctx, x, w, ldx=None, ldw=None, ldo=None):
    rows, k = x.shape
    n = w.shape[0]
    ldx, ldw, ldo = ldx or k, ldw or k, ldo or n
    xp = np.zeros((rows, ldx), np.float32)
    xp[:, :k] = x
    wp = np.zeros((n, ldw), np.uint16)
    wp[:, :k] = w
    d_x, d_w = DeviceArray.from_numpy(xp), DeviceArray.from_numpy(wp)
    d_o = DeviceArray.from_numpy(np.full((rows, ldo), 7.0, np.float32))
    print(f"head rows={rows} k={k} n={n} ldx={ldx} ldw={ldw} ldo={ldo}", flush=True)
    ctx.head_device(rows, k, n, d_x, ldx, d_w, ldw, d_o, ldo)
    ctx.synchronize()
    out = d_o.numpy()
    assert np.all(out[:, n:] == 7.0)
    return out[:, :n]


@pytest.mark.parametrize("rows,k,n", [(1, 1024, 3072), (24, 1024, 2048), (5, 1024, 3001), (24, 1024, 3072),
                                      (8, 2048, 2560), (32, 64, 4099)])
def test_head_exact_on_integers(ctx, rows, k, n):
    rng = np.random.default_rng(rows + n)
    x = rng.integers(-8, 9, (rows, k)).astype(np.float32)
    w = rng.integers(-8, 9, (n, k)).astype(np.float32)
    got = _run(ctx, x, _bf16(w))
    assert np.array_equal(got.astype(np.float64), (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float64))


@pytest.mark.parametrize("rows,k,n,pad", [(24, 1024, 3072, 0), (1, 1024, 2048, 0), (64, 1024, 3072, 8),
                                          (3, 200, 100, 0), (7, 776, 1000, 16), (9, 1536, 513, 0),
                                          (2, 2048, 3072, 0), (4, 8, 7, 0), (2, 1024, 5, 0), (1, 1536, 3001, 8),
                                          (1, 512, 64, 0), (32, 776, 3001, 16), (9, 1536, 2560, 8), (17, 64, 4096, 0)])
def test_head_within_fp32_bound(ctx, rows, k, n, pad):
    rng = np.random.default_rng(rows * 1000 + k + n)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    w = _bf16(rng.standard_normal((n, k)) * 0.05)
    got = _run(ctx, x, w, ldx=k + pad, ldw=k + pad, ldo=n + pad)
    err = np.abs(got - head_exact(x, w))
    bound = head_bound(x, w)
    assert np.all(err <= bound), f"max err/bound {np.max(err / bound):.3f}"
    print(f"max err/bound {np.max(err / bound):.4f}", flush=True)


def test_head_rejects_unsupported_shapes(ctx):
    from voxwerk_amd.sampler import SamplerError

    d = DeviceArray((4, 4096), np.float32)
    w = DeviceArray((4, 4096), np.uint16)
    o = DeviceArray((4, 4), np.float32)
    for k, ldx, ldw in ((2056, 2056, 2056), (12, 12, 12), (16, 18, 16), (16, 16, 20)):
        with pytest.raises(SamplerError):
            ctx.head_device(1, k, 4, d, ldx, w, ldw, o, 4)


def test_step_on_device_head_sampler_embedding(ctx):
    """Hidden rows -> CodecHead -> sampler (logits never leave the GPU) -> CodecEmbedding of the ids."""
    rng = np.random.default_rng(42)
    rows, hidden, vocab = 24, 1024, 3072
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    w = _bf16(rng.standard_normal((vocab, hidden)) * 0.1)
    emb = _bf16(rng.standard_normal((vocab, hidden)))
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"], p["top_k"], p["top_p"], p["temperature"] = 1, 50, np.float32(0.95), np.float32(0.9)
    p["rep_penalty"], p["supp_begin"], p["supp_end"], p["keep_id"], p["ban_id"] = np.float32(1.0), 2048, 3072, 2150, -1
    u = rng.random(rows)
    d_x, d_w, d_emb = DeviceArray.from_numpy(x), DeviceArray.from_numpy(w), DeviceArray.from_numpy(emb)
    d_logits = DeviceArray((rows, vocab), np.float32)
    d_p, d_u = DeviceArray.from_numpy(p), DeviceArray.from_numpy(u)
    d_ids, d_out, d_st = DeviceArray((rows,), np.int32), DeviceArray((rows, hidden), np.float32), DeviceArray((rows,), np.int32)
    ctx.head_device(rows, hidden, vocab, d_x, hidden, d_w, hidden, d_logits, vocab)
    ctx.sample_device(rows, vocab, d_logits, vocab, d_p, 1, d_u, d_ids)
    ctx.embed_device(rows, hidden, d_ids, d_emb, vocab, d_out, hidden, False, d_st)
    ctx.synchronize()
    logits = d_logits.numpy()
    assert np.all(np.abs(logits - head_exact(x, w)) <= head_bound(x, w))
    ids = d_ids.numpy()
    c = ref.classify(ids, ref.sample(logits, p, u))
    assert c["unexplained"] == 0, c
    want = np.zeros((rows, hidden), np.float32)
    st = embed(ids, emb, want, add=False)
    assert np.array_equal(d_st.numpy(), st)
    assert np.array_equal(d_out.numpy().view(np.uint32), want.view(np.uint32))


# ---- int8 weights (WeightPrecision.Int8)
def _run_int8(ctx, x, q, scale, ldx=None, ldq=None, ldo=None):
    rows, k = x.shape
    n = q.shape[0]
    ldx, ldq, ldo = ldx or k, ldq or k, ldo or n
    xp = np.zeros((rows, ldx), np.float32)
    xp[:, :k] = x
    qp = np.zeros((n, ldq), np.int8)
    qp[:, :k] = q
    d_x, d_q, d_s = DeviceArray.from_numpy(xp), DeviceArray.from_numpy(qp), DeviceArray.from_numpy(scale.astype(np.float32))
    d_o = DeviceArray.from_numpy(np.full((rows, ldo), 7.0, np.float32))
    print(f"int8 head rows={rows} k={k} n={n} ldx={ldx} ldq={ldq} ldo={ldo}", flush=True)
    ctx.head_int8_device(rows, k, n, d_x, ldx, d_q, ldq, d_s, d_o, ldo)
    ctx.synchronize()
    out = d_o.numpy()
    assert np.all(out[:, n:] == 7.0)
    return out[:, :n]


def _pack_on_gpu(ctx, w, ldw=None, ldq=None):
    n, k = w.shape
    ldw, ldq = ldw or k, ldq or k
    wp = np.zeros((n, ldw), np.uint16)
    wp[:, :k] = w
    d_w = DeviceArray.from_numpy(wp)
    d_q = DeviceArray.from_numpy(np.full((n, ldq), 99, np.int8))
    d_s = DeviceArray((n,), np.float32)
    print(f"int8 pack n={n} k={k} ldw={ldw} ldq={ldq}", flush=True)
    ctx.head_pack_int8_device(k, n, d_w, ldw, d_q, ldq, d_s)
    ctx.synchronize()
    qv = d_q.numpy()
    assert np.all(qv[:, k:] == 99)
    return qv[:, :k], d_s.numpy()


@pytest.mark.parametrize("n,k,ldw,ldq", [(3072, 1024, 1024, 1024), (2048, 1024, 1032, 1040), (7, 300, 301, 300),
                                         (1, 2048, 2048, 2048)])
def test_pack_int8_bit_exact(ctx, n, k, ldw, ldq):
    rng = np.random.default_rng(n + k)
    wf = rng.standard_normal((n, k)) * np.exp(rng.uniform(-8, 3, (n, 1)))
    if n >= 4:
        wf[0] = 0.0  # all-zero row: scale 1
        wf[1, :8] = [127.0, -63.5, 2.5, 3.5, -0.5, 0.0, 1.5, -126.5]  # ties at scale 1
        wf[1, 8:] = np.clip(wf[1, 8:], -100, 100)
        wf[2] = np.round(wf[2] * 4) / 4
        wf[3] = 0.0  # a row whose inverse scale overflows (amax 2^-125): q saturates to +-127 / 0
        wf[3, :4] = [2.0**-125, -(2.0**-125), 0.0, 2.0**-126]
    w = _bf16(wf)
    q, scale = _pack_on_gpu(ctx, w, ldw, ldq)
    wq, ws = pack_int8(w)
    assert np.array_equal(scale.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(q, wq)


@pytest.mark.parametrize("rows,k,n,scale", [(1, 1024, 3072, 1.0), (24, 1024, 2048, 0.5), (5, 1024, 3001, 0.25),
                                            (3, 2048, 100, 1.0), (24, 1024, 3072, 0.5), (32, 1536, 2560, 2.0)])
def test_head_int8_exact_on_integers(ctx, rows, k, n, scale):
    """Small integers and a power-of-two scale: every partial sum and the scaling are exact."""
    rng = np.random.default_rng(rows * 7 + n)
    x = rng.integers(-8, 9, (rows, k)).astype(np.float32)
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sc = np.full(n, scale, np.float32)
    got = _run_int8(ctx, x, q, sc)
    want = (x.astype(np.int64) @ q.astype(np.int64).T).astype(np.float64) * scale
    assert np.array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("rows,k,n,pad", [(24, 1024, 3072, 0), (1, 1024, 2048, 0), (64, 1024, 3072, 8),
                                          (3, 200, 100, 0), (7, 776, 1000, 16), (9, 1536, 513, 0),
                                          (2, 2048, 3072, 0), (4, 8, 7, 0), (1, 1536, 3001, 8), (16, 776, 3001, 16)])
def test_head_int8_within_bound(ctx, rows, k, n, pad):
    """Weights packed on the GPU, then the head: within gamma_{K+1} * scale * sum|x q| of the exact
    value, the bound both reference forms (decode and batched) satisfy."""
    rng = np.random.default_rng(rows * 1000 + k + n + 1)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    w = _bf16(rng.standard_normal((n, k)) * 0.05)
    q, scale = _pack_on_gpu(ctx, w, ldw=k + pad, ldq=k + pad)
    got = _run_int8(ctx, x, q, scale, ldx=k + pad, ldq=k + pad, ldo=n + pad)
    exact, bound = head_int8_exact(x, q, scale), head_int8_bound(x, q, scale)
    err = np.abs(got - exact)
    assert np.all(err <= bound), f"max err/bound {np.max(err / bound):.3f}"
    if rows * n * k <= 2_000_000:  # the reference's own two fp32 forms on the same packed weight
        for ref_form in (head_int8_decode_fp32, head_int8_batched_fp32):
            assert np.all(np.abs(ref_form(x, q, scale).astype(np.float64) - exact) <= bound)


def test_head_int8_rejects_unsupported_shapes(ctx):
    from voxwerk_amd.sampler import SamplerError

    d = DeviceArray((4, 4096), np.float32)
    q = DeviceArray((4, 4096), np.int8)
    s = DeviceArray((4,), np.float32)
    o = DeviceArray((4, 4), np.float32)
    for k, ldx, ldq in ((2056, 2056, 2056), (12, 12, 12), (16, 18, 16), (16, 16, 20)):
        with pytest.raises(SamplerError):
            ctx.head_int8_device(1, k, 4, d, ldx, q, ldq, s, o, 4)


def test_step_on_device_int8_head_sampler(ctx):
    """Hidden rows -> int8 CodecHead (weights packed on the GPU) -> sampler, the logits never leaving
    the GPU (WeightPrecision.Int8): logits within the int8 bound, ids equal to the oracle's on them."""
    rng = np.random.default_rng(43)
    rows, hidden, vocab = 24, 1024, 3072
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    w = _bf16(rng.standard_normal((vocab, hidden)) * 0.1)
    p = np.zeros(rows, dtype=PARAMS_DTYPE)
    p["do_sample"], p["top_k"], p["top_p"], p["temperature"] = 1, 50, np.float32(0.95), np.float32(0.9)
    p["rep_penalty"], p["supp_begin"], p["supp_end"], p["keep_id"], p["ban_id"] = np.float32(1.0), 2048, 3072, 2150, -1
    u = rng.random(rows)
    q, scale = _pack_on_gpu(ctx, w)
    d_x, d_q, d_s = DeviceArray.from_numpy(x), DeviceArray.from_numpy(q), DeviceArray.from_numpy(scale)
    d_logits = DeviceArray((rows, vocab), np.float32)
    d_p, d_u, d_ids = DeviceArray.from_numpy(p), DeviceArray.from_numpy(u), DeviceArray((rows,), np.int32)
    ctx.head_int8_device(rows, hidden, vocab, d_x, hidden, d_q, hidden, d_s, d_logits, vocab)
    ctx.sample_device(rows, vocab, d_logits, vocab, d_p, 1, d_u, d_ids)
    ctx.synchronize()
    logits = d_logits.numpy()
    assert np.all(np.abs(logits - head_int8_exact(x, q, scale)) <= head_int8_bound(x, q, scale))
    ids = d_ids.numpy()
    c = ref.classify(ids, ref.sample(logits, p, u))
    assert c["unexplained"] == 0, c


@pytest.mark.parametrize("int8", [False, True])
def test_head_nonfinite_hidden_values(ctx, int8):
    """Matrix-core form (8 to 32 rows, 2560 outputs or more): +inf, -inf and NaN in the hidden rows
    give what IEEE products and sums give (the classes of the float64 results: +-inf, NaN)."""
    rng = np.random.default_rng(17)
    rows, k, n = 12, 1024, 2560
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[1, 5] = np.inf
    x[3, 100] = -np.inf
    x[5, 7] = np.nan
    x[7, 9], x[7, 10] = np.inf, -np.inf
    wf = rng.standard_normal((n, k)) * 0.05
    wf[:8, 5] = 0.0  # inf times a zero weight: NaN
    w = _bf16(wf)
    if int8:
        q, scale = _pack_on_gpu(ctx, w)
        got = _run_int8(ctx, x, q, scale)
        wd = q.astype(np.float64)
    else:
        got = _run(ctx, x, w)
        wd = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    want = np.empty((rows, n))
    with np.errstate(invalid="ignore"):
        for r in range(rows):  # elementwise products and a plain sum: IEEE classes, no library shortcuts
            want[r] = (x[r].astype(np.float64)[:, None] * wd.T).sum(axis=0)
    for r in (1, 3, 5, 7):
        assert np.array_equal(np.isnan(got[r]), np.isnan(want[r])), r
        assert np.array_equal(np.isposinf(got[r]), np.isposinf(want[r])), r
        assert np.array_equal(np.isneginf(got[r]), np.isneginf(want[r])), r
    fin = [0, 2, 4, 6, 8, 9, 10, 11]
    assert np.all(np.isfinite(got[fin]))
