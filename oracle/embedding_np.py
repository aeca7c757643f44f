"""numpy restatement of voxwerk's embedding lookups of sampled ids — TEST INFRASTRUCTURE ONLY.

- ``widen``: Bf16.ToFloat (src/Voxwerk/Numerics/Bf16.cs:13), the bf16 bits shifted into the high
  half of a binary32 (exact, NaN payloads kept).
- ``embed``: CodecEmbedding / CodePredictorEmbedding (src/Voxwerk/Talker/TalkerModel.cs:100-111,
  the row write or add of AddRow, :119-131).
- ``frame_embed``: FrameEmbedding (TalkerModel.cs:113-117) — codebook 0 written, codebooks 1..G-1
  added in order, each add one binary32 rounding — followed by the talker step's text row
  (TalkerGenerator.cs:283, :439).

Pinned in tests/test_oracle.py by closed forms: widened special encodings (1, -2, inf, the
smallest subnormal), and sums whose fp32 result depends on the order of the adds and on the
addend coming last, so a reordered, pairwise or fp64 sum fails.
"""
from __future__ import annotations

import numpy as np


def widen(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32, exactly."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def embed(ids, table: np.ndarray, out: np.ndarray, add: bool) -> np.ndarray:
    """out[r] = widen(table[ids[r]]) (add False) or out[r] += it (add True). Returns per-row status:
    0, or -2 for an id outside the table (that row is left unchanged)."""
    ids = np.asarray(ids)
    status = np.zeros(ids.shape[0], np.int32)
    vocab, hidden = table.shape
    for r, i in enumerate(ids.tolist()):
        if not 0 <= i < vocab:
            status[r] = -2
            continue
        e = widen(table[i])
        out[r, :hidden] = (out[r, :hidden] + e).astype(np.float32) if add else e
    return status


def frame_embed(codes, codec_table: np.ndarray, cp_tables: np.ndarray, addend=None, out=None):
    """Rows E0[c0] + E1[c1] + ... (+ addend), left to right in float32. cp_tables [G-1][cp_vocab][hidden].
    Returns (out, status); rows with an id outside its table keep `out`'s previous values."""
    codes = np.asarray(codes)
    rows, groups = codes.shape
    vocab, hidden = codec_table.shape
    cp_vocab = cp_tables.shape[1] if groups > 1 else 0
    if out is None:
        out = np.zeros((rows, hidden), np.float32)
    status = np.zeros(rows, np.int32)
    for r in range(rows):
        c = codes[r].tolist()
        if not (0 <= c[0] < vocab and all(0 <= x < cp_vocab for x in c[1:])):
            status[r] = -2
            continue
        acc = widen(codec_table[c[0]])
        for g in range(1, groups):
            acc = (acc + widen(cp_tables[g - 1, c[g]])).astype(np.float32)
        if addend is not None:
            acc = (acc + np.asarray(addend[r][:hidden], np.float32)).astype(np.float32)
        out[r, :hidden] = acc
    return out, status
