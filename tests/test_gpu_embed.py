"""GPU: embedding lookups of sampled ids (vxs_embed_device / vxs_frame_embed_device) through the C ABI
against the numpy oracle (oracle/embedding_np.py). Bar: bit-identical rows (NaN-free tables), status
codes equal, rows with a bad id left untouched."""
import numpy as np
import pytest

from oracle.embedding_np import embed, frame_embed
from voxwerk_amd.hip import DeviceArray

pytestmark = pytest.mark.gpu


def _table(rng, vocab, hidden):
    """Random bf16 tables: normal values with a sprinkle of subnormals and zeros of both signs
    (finite, so the sums are NaN-free and compare bit for bit)."""
    t = (rng.standard_normal((vocab, hidden)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    k = max(1, t.size // 200)
    idx = rng.integers(0, t.size, k)
    t.reshape(-1)[idx] = rng.choice(np.array([0x0001, 0x8003, 0x0000, 0x8000, 0x007F], np.uint16), k)
    return t


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("rows,hidden,ld", [(24, 1024, 1024), (7, 1000, 1003), (300, 1024, 1028)])
def test_frame_embedding_matches_oracle(ctx, rows, hidden, ld):
    rng = np.random.default_rng(rows * 7 + hidden)
    groups, vocab, cp_vocab = 16, 3072, 2048
    codec = _table(rng, vocab, hidden)
    cp = np.stack([_table(rng, cp_vocab, hidden) for _ in range(groups - 1)])
    codes = np.concatenate([rng.integers(0, vocab, (rows, 1)), rng.integers(0, cp_vocab, (rows, groups - 1))], 1)
    codes = codes.astype(np.int32)
    if rows > 3:
        codes[1, 0] = vocab       # codebook 0 out of range
        codes[2, 5] = -4          # a failed sampler row's error code
        codes[3, 15] = cp_vocab
    text = rng.standard_normal((rows, ld)).astype(np.float32)
    prev = np.full((rows, ld), 5.0, np.float32)
    want, wst = frame_embed(codes, codec, cp, addend=text, out=prev[:, :hidden].copy())
    d_codes, d_codec, d_cp, d_text = (DeviceArray.from_numpy(a) for a in (codes, codec, cp, text))
    d_out = DeviceArray.from_numpy(prev)
    d_st = DeviceArray((rows,), np.int32)
    print(f"rows={rows} hidden={hidden} ld={ld}", flush=True)
    ctx.frame_embed_device(rows, groups, hidden, d_codes, groups, d_codec, vocab, d_cp, cp_vocab, d_out, ld, d_st,
                           addend=d_text, ld_addend=ld)
    ctx.synchronize()
    got = d_out.numpy()
    assert d_st.numpy().tolist() == wst.tolist()
    assert _bits_equal(got[:, :hidden], want)
    assert np.all(got[:, hidden:] == 5.0)  # beyond hidden: untouched


def test_frame_embedding_without_text_row(ctx):
    rng = np.random.default_rng(1)
    rows, groups, hidden, vocab, cp_vocab = 16, 16, 1024, 3072, 2048
    codec = _table(rng, vocab, hidden)
    cp = np.stack([_table(rng, cp_vocab, hidden) for _ in range(groups - 1)])
    codes = np.concatenate([rng.integers(0, vocab, (rows, 1)), rng.integers(0, cp_vocab, (rows, groups - 1))], 1)
    codes = np.ascontiguousarray(codes, np.int32)
    want, _ = frame_embed(codes, codec, cp)
    d = [DeviceArray.from_numpy(a) for a in (codes, codec, cp)]
    d_out, d_st = DeviceArray((rows, hidden), np.float32), DeviceArray((rows,), np.int32)
    ctx.frame_embed_device(rows, groups, hidden, d[0], groups, d[1], vocab, d[2], cp_vocab, d_out, hidden, d_st)
    ctx.synchronize()
    assert _bits_equal(d_out.numpy(), want) and not d_st.numpy().any()
    # codebook-major codes, as one sampling call per codebook leaves them: stage g at codes + g * rows
    d_cm, d_out2 = DeviceArray.from_numpy(np.ascontiguousarray(codes.T)), DeviceArray((rows, hidden), np.float32)
    ctx.frame_embed_device(rows, groups, hidden, d_cm, 1, d[1], vocab, d[2], cp_vocab, d_out2, hidden, d_st,
                           group_stride=rows)
    ctx.synchronize()
    assert _bits_equal(d_out2.numpy(), want) and not d_st.numpy().any()


@pytest.mark.parametrize("add", [False, True])
def test_embed_matches_oracle(ctx, add):
    rng = np.random.default_rng(2 + add)
    rows, hidden, vocab, ld = 40, 1024, 2048, 1040
    table = _table(rng, vocab, hidden)
    ids = rng.integers(0, vocab, rows).astype(np.int32)
    ids[3], ids[7] = vocab, -1
    out0 = rng.standard_normal((rows, ld)).astype(np.float32)
    want = out0.copy()
    wst = embed(ids, table, want, add)
    d_ids, d_tab, d_out = DeviceArray.from_numpy(ids), DeviceArray.from_numpy(table), DeviceArray.from_numpy(out0)
    d_st = DeviceArray((rows,), np.int32)
    ctx.embed_device(rows, hidden, d_ids, d_tab, vocab, d_out, ld, add, d_st)
    ctx.synchronize()
    assert d_st.numpy().tolist() == wst.tolist()
    assert _bits_equal(d_out.numpy(), want)
