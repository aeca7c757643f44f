"""numpy restatement of voxwerk's logit heads — TEST INFRASTRUCTURE ONLY.

CodecHead / CodePredictorHead (src/Voxwerk/Talker/TalkerModel.cs:133-137) are Gemm.Multiply over a
bf16 PackedMatrix (Gemm.cs:602-648, PanelDot): out[r][n] = sum_k x[r][k] * W[n][k] in fp32 with
the reference's own AVX-512 order of products and sums. That order is not restated: the oracle is
the exact dot product (fp64, where the product of a bf16 and an fp32 value is exact) and the
classical bound on any fp32 evaluation of it, |fl(s) - s| <= gamma_K * sum_k |x_k w_k| with
gamma_K = K u / (1 - K u), u = 2^-24, which the reference's result and the GPU's both satisfy.

The int8 form (WeightPrecision.Int8) packs W per output row as PackedMatrix.FromBf16LinearInt8
(src/Voxwerk/Numerics/PackedMatrix.cs:124-154): amax = max |w|, scale = fp32(amax / 127) (1 for an
all-zero row), inv = fp32(1 / scale), q = clamp(round-half-even(fp32(w * inv)), -127, 127); the
decode product is scale * sum_k x q (Gemm.cs:650-680), the batched one sum_k x * fp32(q * scale)
(Gemm.cs:95-98, 650-654). Both lie within gamma_{K+1} * scale * sum_k |x q| of the exact value.

Pinned in tests/test_oracle.py: integer data whose every partial sum is exact in fp32 (so every
order gives the exact value), fp32 sums in two different orders staying inside the bound, and the
int8 packing against hand-derived rows (ties to even, all-zero rows, power-of-two scales) and a
per-element restatement in Python floats.
"""
from __future__ import annotations

import numpy as np

from .embedding_np import widen

U = 2.0**-24


def head_exact(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """x fp32 [rows][K], w bf16 bits [N][K] -> exact-ish fp64 [rows][N] (error ~K 2^-53 relative)."""
    return np.asarray(x, np.float64) @ widen(w).astype(np.float64).T


def head_bound(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """gamma_K * sum_k |x w| per entry: the worst-case error of any fp32 evaluation of the dot."""
    k = x.shape[1]
    gamma = k * U / (1 - k * U)
    return gamma * (np.abs(np.asarray(x, np.float64)) @ np.abs(widen(w).astype(np.float64)).T)


def pack_int8(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """bf16 bits [N][K] -> (q int8 [N][K], scale fp32 [N]) as FromBf16LinearInt8 (PackedMatrix.cs:129-152)."""
    wf = widen(w)
    amax = np.max(np.abs(wf), axis=1)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        scale = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)  # :142
        inv = (np.float32(1.0) / scale).astype(np.float32)  # :143; inf when amax < ~3.7e-37
        prod = (wf * inv[:, None]).astype(np.float32)
        r = np.rint(prod)  # MathF.Round: ties to even (:146)
    # (int) of a float saturates in .NET 9 and later: NaN -> 0, +-inf -> int.MaxValue / MinValue;
    # then Math.Clamp to [-127, 127]
    q = np.where(np.isnan(r), 0.0, np.clip(r, -127, 127)).astype(np.int8)
    return q, scale


def head_int8_exact(x: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """scale[n] * sum_k x[r][k] q[n][k] in fp64 (the integer-valued q makes each product exact)."""
    return (np.asarray(x, np.float64) @ q.astype(np.float64).T) * scale.astype(np.float64)[None, :]


def head_int8_bound(x: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """gamma_{K+1} * scale * sum_k |x q|: the error bound of the decode and batched fp32 forms."""
    k = x.shape[1] + 1
    gamma = k * U / (1 - k * U)
    return gamma * (np.abs(np.asarray(x, np.float64)) @ np.abs(q.astype(np.float64)).T) * scale.astype(np.float64)[None, :]


def head_int8_decode_fp32(x: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """The decode form, FMAs in k order then the scale: fl(fl(sum_k x q) * scale) (Gemm.cs:738-753).
    Each step is acc + x q in fp64 rounded to fp32 (an FMA up to rare double rounding)."""
    rows, k = x.shape
    acc = np.zeros((rows, q.shape[0]), np.float32)
    qd = q.astype(np.float64)
    for kk in range(k):
        acc = (acc.astype(np.float64) + x[:, kk : kk + 1].astype(np.float64) * qd[None, :, kk]).astype(np.float32)
    return (acc * scale[None, :]).astype(np.float32)


def head_int8_batched_fp32(x: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """The batched form, FMAs in k order over the dequantized weight: sum_k x * fl(q * scale)
    (Gemm.cs:95-98); steps as in head_int8_decode_fp32."""
    rows, k = x.shape
    wd = (q.astype(np.float32) * scale[:, None]).astype(np.float32).astype(np.float64)
    acc = np.zeros((rows, q.shape[0]), np.float32)
    for kk in range(k):
        acc = (acc.astype(np.float64) + x[:, kk : kk + 1].astype(np.float64) * wd[None, :, kk]).astype(np.float32)
    return acc
