"""ctypes wrapper of the C oracle (oracle/vxs_oracle.c). TEST INFRASTRUCTURE ONLY."""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_int64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libvxs_oracle.so")

PARAMS_DTYPE = np.dtype(
    [("do_sample", "<i4"), ("top_k", "<i4"), ("top_p", "<f4"), ("temperature", "<f4"), ("rep_penalty", "<f4"),
     ("supp_begin", "<i4"), ("supp_end", "<i4"), ("keep_id", "<i4"), ("ban_id", "<i4")]
)

INFO_DTYPE = np.dtype(
    [("draw_margin", "<f8"), ("topp_margin", "<f8"), ("n_candidates", "<i4"), ("n_kept", "<i4"),
     ("kth", "<f4"), ("flags", "<i4")],
    align=True,
)

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = ctypes.CDLL(LIB)
        lib.vxs_oracle_sample.restype = c_int
        lib.vxs_oracle_sample.argtypes = [c_int, c_int, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int,
                                          c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int]
        lib.vxs_oracle_apply_penalty.restype = c_int
        lib.vxs_oracle_apply_penalty.argtypes = [c_int, c_int, c_void_p, c_int64, c_void_p, c_void_p, c_float]
        lib.vxs_oracle_argmax.restype = c_int
        lib.vxs_oracle_argmax.argtypes = [c_int, c_void_p]
        lib.vxs_oracle_random_stream.restype = c_int
        lib.vxs_oracle_random_stream.argtypes = [c_int32, c_int64, c_void_p, c_void_p]
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def sample(logits, params, u=None, hist_off=None, hist_ids=None, threads: int = 1, want_logits=False,
           want_probs=False, want_info=True):
    """Run the oracle over [rows, vocab] logits. Returns dict(ids, logits?, probs?, info?, rc)."""
    lib = load()
    x = np.ascontiguousarray(logits, dtype=np.float32)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    rows, vocab = x.shape
    params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
    stride = 0 if params.ndim == 0 or params.size == 1 else 1
    if u is not None:
        u = np.ascontiguousarray(u, dtype=np.float64).reshape(-1)
    if hist_off is not None:
        hist_off = np.ascontiguousarray(hist_off, dtype=np.int32)
        hist_ids = np.ascontiguousarray(hist_ids, dtype=np.int32)
    ids = np.empty(rows, dtype=np.int32)
    out_l = np.empty((rows, vocab), dtype=np.float32) if want_logits else None
    out_p = np.empty((rows, vocab), dtype=np.float64) if want_probs else None
    info = np.zeros(rows, dtype=INFO_DTYPE) if want_info else None
    rc = lib.vxs_oracle_sample(rows, vocab, _p(x), vocab, _p(hist_off), _p(hist_ids), _p(params), stride, _p(u),
                               _p(ids), _p(out_l), _p(out_p), _p(info), threads)
    return {"rc": rc, "ids": ids, "logits": out_l, "probs": out_p, "info": info}


def apply_penalty(logits, hist_off, hist_ids, penalty) -> int:
    lib = load()
    assert logits.dtype == np.float32 and logits.flags.c_contiguous
    x = logits.reshape(1, -1) if logits.ndim == 1 else logits
    return lib.vxs_oracle_apply_penalty(x.shape[0], x.shape[1], _p(x), x.shape[1],
                                        _p(np.ascontiguousarray(hist_off, np.int32)),
                                        _p(np.ascontiguousarray(hist_ids, np.int32)), float(np.float32(penalty)))


def random_stream(seed: int, n: int):
    """The first n draws of .NET's new Random(seed): (Next() values int32, NextDouble() values)."""
    samples = np.empty(n, np.int32)
    doubles = np.empty(n, np.float64)
    assert load().vxs_oracle_random_stream(int(seed), int(n), _p(samples), _p(doubles)) == 0
    return samples, doubles


def argmax(x) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    return load().vxs_oracle_argmax(x.size, _p(x))


DRAW_BOUNDARY = 1e-6  # |u - CDF edge| below which differing ids count as boundary draws
TOPP_BOUNDARY = 1e-6  # |cum - (1 - top_p)| below which differing ids count as top-p boundaries


def classify(gpu_ids, ora) -> dict:
    """Exact-id matches and boundary-classified differences of GPU ids against an oracle result."""
    ids = ora["ids"]
    info = ora["info"]
    same = gpu_ids == ids
    draw_b = info["draw_margin"] < DRAW_BOUNDARY
    topp_b = info["topp_margin"] < TOPP_BOUNDARY
    diff = ~same
    bad = np.nonzero(diff & ~draw_b & ~topp_b)[0]
    return {
        "rows": int(ids.size),
        "exact": int(same.sum()),
        "draw_boundary": int((diff & draw_b & ~topp_b).sum()),
        "topp_boundary": int((diff & topp_b).sum()),
        "unexplained": int(bad.size),
        "unexplained_rows": bad[:8].tolist(),
    }
