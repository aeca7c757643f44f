"""numpy restatement of voxwerk's logit heads — TEST INFRASTRUCTURE ONLY.

CodecHead / CodePredictorHead (src/Voxwerk/Talker/TalkerModel.cs:133-137) are Gemm.Multiply over a
bf16 PackedMatrix (Gemm.cs:602-648, PanelDot): out[r][n] = sum_k x[r][k] * W[n][k] in fp32 with
the reference's own AVX-512 order of products and sums. That order is not restated: the oracle is
the exact dot product (fp64, where the product of a bf16 and an fp32 value is exact) and the
classical bound on any fp32 evaluation of it, |fl(s) - s| <= gamma_K * sum_k |x_k w_k| with
gamma_K = K u / (1 - K u), u = 2^-24, which the reference's result and the GPU's both satisfy.

Pinned in tests/test_oracle.py: integer data whose every partial sum is exact in fp32 (so every
order gives the exact value), and fp32 sums in two different orders staying inside the bound.
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
