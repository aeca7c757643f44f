"""ctypes bindings of the sampler's C ABI (include/vxs_sampler.h) and of the workload generator.

The HIP library must have been built (``__graft_entry__.build()``); there is no CPU fallback:
loading fails loudly when ``voxwerk_amd/lib/libvxs.so`` is missing.
"""
from __future__ import annotations

import ctypes
import os
import re
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_uint32, c_void_p

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG_DIR, "lib")
REPO_DIR = os.path.dirname(PKG_DIR)
HEADER = os.path.join(REPO_DIR, "include", "vxs_sampler.h")
LIBVXS = os.path.join(LIB_DIR, "libvxs.so")
LIBSYNTH = os.path.join(LIB_DIR, "libvxs_synth.so")

VXS_OK = 0
VXS_ERR_INVALID_ARG = -1
VXS_ERR_ID_OUT_OF_RANGE = -2
VXS_ERR_NONFINITE = -3
VXS_ERR_HIP = -4
VXS_ERR_UNSUPPORTED = -5
VXS_ERR_NO_DEVICE = -6
VXS_ERR_HISTORY_FULL = -7
VXS_FLAG_PATH_BLOCK = 1 << 8
VXS_FLAG_PATH_WAVE = 1 << 9
VXS_FLAG_RNG_TALKER = 1 << 10
VXS_FLAG_RNG_SUB = 1 << 11


class VxsParams(ctypes.Structure):
    """vxs_params (include/vxs_sampler.h)."""

    _fields_ = [
        ("do_sample", c_int32),
        ("top_k", c_int32),
        ("top_p", c_float),
        ("temperature", c_float),
        ("rep_penalty", c_float),
        ("supp_begin", c_int32),
        ("supp_end", c_int32),
        ("keep_id", c_int32),
        ("ban_id", c_int32),
    ]


PARAMS_DTYPE = np.dtype(
    [
        ("do_sample", "<i4"),
        ("top_k", "<i4"),
        ("top_p", "<f4"),
        ("temperature", "<f4"),
        ("rep_penalty", "<f4"),
        ("supp_begin", "<i4"),
        ("supp_end", "<i4"),
        ("keep_id", "<i4"),
        ("ban_id", "<i4"),
    ]
)
assert PARAMS_DTYPE.itemsize == ctypes.sizeof(VxsParams) == 36


class VxsWorkload(ctypes.Structure):
    """vxs_workload (voxwerk_amd/csrc/vxs_synth.c)."""

    _fields_ = [
        ("id", c_int32),
        ("rows", c_int32),
        ("vocab", c_int32),
        ("steps", c_int32),
        ("hist_len", c_int32),
        ("seed", ctypes.c_uint64),
        ("params", VxsParams),
    ]


_P = c_void_p  # raw pointers are passed as integers / c_void_p

_SIGNATURES = {
    "vxs_create": (c_int, [POINTER(c_void_p), c_int, c_int, c_int, c_int64]),
    "vxs_destroy": (None, [c_void_p]),
    "vxs_last_error": (c_char_p, [c_void_p]),
    "vxs_version": (c_char_p, []),
    "vxs_set_stream": (c_int, [c_void_p, c_void_p]),
    "vxs_get_stream": (c_void_p, [c_void_p]),
    "vxs_sample": (c_int, [c_void_p, c_int, c_int, _P, c_int64, _P, _P, _P, c_int, _P, _P, _P, _P, c_uint32]),
    "vxs_sample_device": (c_int, [c_void_p, c_int, c_int, _P, c_int64, _P, _P, _P, c_int, _P, _P, _P, _P, c_uint32]),
    "vxs_sample_noalloc": (c_int, [c_void_p, c_int, c_int, _P, c_int64, _P, _P, _P, c_int, _P, _P, c_uint32]),
    "vxs_sample_stats_device": (c_int, [c_void_p, c_int, c_int, _P, c_int64, _P, _P, _P, c_int, _P, _P, _P,
                                        _P, c_uint32]),
    "vxs_synchronize": (c_int, [c_void_p]),
    "vxs_apply_repetition_penalty": (c_int, [c_void_p, c_int, c_int, _P, c_int64, _P, _P, c_float]),
    "vxs_argmax": (c_int, [c_void_p, c_int, c_int, _P, c_int64, _P]),
    "vxs_history_create": (c_int, [c_void_p, c_int, c_int, POINTER(c_void_p)]),
    "vxs_history_destroy": (None, [c_void_p]),
    "vxs_history_set": (c_int, [c_void_p, c_void_p, c_int, _P, c_int]),
    "vxs_history_get": (c_int, [c_void_p, c_void_p, c_int, _P, c_int, POINTER(c_int)]),
    "vxs_history_seed": (c_int, [c_void_p, c_void_p, c_int, c_int32]),
    "vxs_embed_device": (c_int, [c_void_p, c_int, c_int, _P, _P, c_int, _P, c_int64, c_int, _P]),
    "vxs_head_device": (c_int, [c_void_p, c_int, c_int, c_int, _P, c_int64, _P, c_int64, _P, c_int64]),
    "vxs_head_int8_device": (c_int, [c_void_p, c_int, c_int, c_int, _P, c_int64, _P, c_int64, _P, _P, c_int64]),
    "vxs_head_pack_int8_device": (c_int, [c_void_p, c_int, c_int, _P, c_int64, _P, c_int64, _P]),
    "vxs_frame_embed_device": (c_int, [c_void_p, c_int, c_int, c_int, _P, c_int64, c_int64, _P, c_int, _P, c_int, _P,
                                       c_int64, _P, c_int64, _P]),
    "vxs_history_draw": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, _P]),
    "vxs_sample_batch": (c_int, [c_void_p, c_void_p, c_int, c_int, _P, c_int64, _P, c_int, _P, c_int, _P, _P,
                                 c_uint32]),
    "vxs_sample_batch_device": (c_int, [c_void_p, c_void_p, c_int, c_int, _P, c_int64, _P, c_int, _P, c_int, _P,
                                        _P, c_uint32]),
}


def header_symbols(path: str = HEADER) -> list[str]:
    """Names of every function the public header declares (``VXS_API <ret> <name>(``)."""
    text = open(path, encoding="utf-8").read()
    return re.findall(r"VXS_API\s+[\w\s\*]+?\b(vxs_\w+)\s*\(", text)


_vxs = None
_synth = None


def load_vxs() -> ctypes.CDLL:
    """Load the HIP sampler library (raises if it has not been built)."""
    global _vxs
    if _vxs is None:
        if not os.path.exists(LIBVXS):
            raise RuntimeError(f"{LIBVXS} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
        lib = ctypes.CDLL(LIBVXS)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _vxs = lib
    return _vxs


def load_synth() -> ctypes.CDLL:
    """Load the CPU workload generator library."""
    global _synth
    if _synth is None:
        if not os.path.exists(LIBSYNTH):
            raise RuntimeError(f"{LIBSYNTH} is missing: build the package first")
        lib = ctypes.CDLL(LIBSYNTH)
        lib.vxs_synth_workload.restype = c_int
        lib.vxs_synth_workload.argtypes = [c_int, POINTER(VxsWorkload)]
        lib.vxs_synth_generate.restype = c_int
        lib.vxs_synth_generate.argtypes = [c_int, c_int, c_int64, c_int64, _P, c_int64, _P, _P, c_int]
        lib.vxs_synth_log.restype = c_double
        lib.vxs_synth_log.argtypes = [c_double]
        lib.vxs_synth_cos_turn.restype = c_double
        lib.vxs_synth_cos_turn.argtypes = [c_double]
        _synth = lib
    return _synth


def ptr(a) -> int | None:
    """Address of a numpy array / torch tensor / None (for ctypes void* arguments)."""
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    if isinstance(a, int):
        return a
    raise TypeError(f"cannot take the address of {type(a)}")
