"""GPU: the logit heads (vxs_head_device) through the C ABI against the oracle (oracle/head_np.py),
and the device-resident step head -> sampler -> embedding.

Bar: exact on integer data (every order is exact); within gamma_K * sum|x w| of the exact dot
product otherwise (the bound the reference's own fp32 order also satisfies); sampled ids on the
head's logits identical to the oracle's on the same logits (boundary rows counted); embeddings
bit-identical."""
import numpy as np
import pytest

from oracle import ref
from oracle.embedding_np import embed
from oracle.head_np import head_bound, head_exact
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


@pytest.mark.parametrize("rows,k,n", [(1, 1024, 3072), (24, 1024, 2048), (5, 1024, 3001)])
def test_head_exact_on_integers(ctx, rows, k, n):
    rng = np.random.default_rng(rows + n)
    x = rng.integers(-8, 9, (rows, k)).astype(np.float32)
    w = rng.integers(-8, 9, (n, k)).astype(np.float32)
    got = _run(ctx, x, _bf16(w))
    assert np.array_equal(got.astype(np.float64), (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float64))


@pytest.mark.parametrize("rows,k,n,pad", [(24, 1024, 3072, 0), (1, 1024, 2048, 0), (64, 1024, 3072, 8),
                                          (3, 200, 100, 0), (7, 776, 1000, 16), (9, 1536, 513, 0),
                                          (2, 2048, 3072, 0), (4, 8, 7, 0), (2, 1024, 5, 0), (1, 1536, 3001, 8),
                                          (1, 512, 64, 0)])
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
