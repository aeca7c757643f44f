"""Python host side of the MI355X sampler, mirroring voxwerk's C# sampling surface.

``SamplingOptions`` / ``GenerationOptions`` / ``Sampler`` keep the names, argument meaning and error
behaviour of src/Voxwerk/Talker/Sampler.cs:4-96 and TalkerGenerator.cs:7-22; every computation goes
through the HIP library's C ABI (include/vxs_sampler.h). ``Context`` is the thin binding of that ABI
for batched host or device-resident calls.
"""
from __future__ import annotations

import ctypes
import os
import threading
from dataclasses import dataclass, field
from typing import Iterable, Optional

import numpy as np

from . import _lib
from ._lib import PARAMS_DTYPE, load_vxs, ptr


class SamplerError(RuntimeError):
    """A non-zero return code of the C ABI."""

    def __init__(self, code: int, message: str):
        super().__init__(f"vxs error {code}: {message}")
        self.code = code


class HistoryIdOutOfRange(SamplerError, IndexError):
    """A history id outside [0, vocab): the reference's Span indexer throws here (Sampler.cs:30)."""


class NonFiniteLogits(SamplerError, ValueError):
    """NaN or +inf after temperature scaling: outside the sampler contract."""


class HistoryFull(SamplerError, OverflowError):
    """A resident history slot already holds its capacity of ids (vxs_sample_batch)."""


def _raise(code: int, message: str) -> None:
    if code == _lib.VXS_ERR_HISTORY_FULL:
        raise HistoryFull(code, message)
    if code == _lib.VXS_ERR_ID_OUT_OF_RANGE:
        raise HistoryIdOutOfRange(code, message)
    if code == _lib.VXS_ERR_NONFINITE:
        raise NonFiniteLogits(code, message)
    if code == _lib.VXS_ERR_INVALID_ARG:
        raise SamplerError(code, message)
    raise SamplerError(code, message)


# ---------------------------------------------------------------------------------------------
# Options (Sampler.cs:4-13, TalkerGenerator.cs:7-22)
# ---------------------------------------------------------------------------------------------
@dataclass(frozen=True)
class SamplingOptions:
    DoSample: bool = True
    TopK: int = 50
    TopP: float = 1.0
    Temperature: float = 0.9

    @staticmethod
    def Greedy() -> "SamplingOptions":
        return SamplingOptions(DoSample=False)


@dataclass(frozen=True)
class GenerationOptions:
    MaxNewTokens: int = 2048
    RepetitionPenalty: float = 1.05
    Talker: SamplingOptions = field(default_factory=SamplingOptions)
    SubTalker: SamplingOptions = field(default_factory=SamplingOptions)
    NonStreamingMode: Optional[bool] = None
    Seed: Optional[int] = None

    @staticmethod
    def Greedy() -> "GenerationOptions":
        return GenerationOptions(Talker=SamplingOptions.Greedy(), SubTalker=SamplingOptions.Greedy())


# Qwen3TtsConfig.cs:28,34,49
TALKER_VOCAB = 3072
CODEC_EOS_ID = 2150
CP_VOCAB = 2048


def make_params(opts: SamplingOptions, rep_penalty: float = 1.0, supp_begin: int = 0, supp_end: int = 0,
                keep_id: int = -1, ban_id: int = -1) -> np.ndarray:
    """One vxs_params record."""
    p = np.zeros((), dtype=PARAMS_DTYPE)
    p["do_sample"] = 1 if opts.DoSample else 0
    p["top_k"] = opts.TopK
    p["top_p"] = np.float32(opts.TopP)
    p["temperature"] = np.float32(opts.Temperature)
    p["rep_penalty"] = np.float32(rep_penalty)
    p["supp_begin"] = supp_begin
    p["supp_end"] = supp_end
    p["keep_id"] = keep_id
    p["ban_id"] = ban_id
    return p


def talker_params(opts: GenerationOptions, step: int, vocab: int = TALKER_VOCAB, eos_id: int = CODEC_EOS_ID) -> np.ndarray:
    """Talker row of frame `step`: penalty, [V-1024, V) suppressed except EOS, EOS banned while step < 2
    (TalkerGenerator.cs:246-249 / :370-373)."""
    return make_params(opts.Talker, opts.RepetitionPenalty, vocab - 1024, vocab, eos_id, eos_id if step < 2 else -1)


def sub_talker_params(opts: GenerationOptions) -> np.ndarray:
    """Code-predictor row (TalkerGenerator.cs:268 / :419-420): no penalty, no suppression."""
    return make_params(opts.SubTalker)


# ---------------------------------------------------------------------------------------------
# .NET System.Random(seed) — legacy subtractive generator, so seeded runs reproduce the C# draws
# ---------------------------------------------------------------------------------------------
def _i32(x: int) -> int:
    """C#'s unchecked ``int`` arithmetic: wrap to [-2^31, 2^31)."""
    return ((x + 0x80000000) & 0xFFFFFFFF) - 0x80000000


class DotNetRandom:
    """``new Random(seed)`` as .NET constructs it for an explicit seed (Knuth's subtractive method,
    MSEED = 161803398). ``NextDouble()`` = InternalSample() / int.MaxValue. Sampler.cs:21,77 consume one
    NextDouble per sampled Select. Every step wraps to 32 bits as C#'s unchecked ``int`` arithmetic
    does: for seeds above MSEED the seeding overflows, and the draws depend on the wrap."""

    MBIG = 2147483647
    MSEED = 161803398

    def __init__(self, seed: Optional[int]):
        if seed is None:
            seed = int.from_bytes(os.urandom(4), "little") & 0x7FFFFFFF
        seed = _i32(int(seed))
        sa = [0] * 56
        sub = self.MBIG if seed == -(2**31) else abs(seed)
        mj = _i32(self.MSEED - sub)
        sa[55] = mj
        mk = 1
        ii = 0
        for _ in range(1, 55):
            ii += 21
            if ii >= 55:
                ii -= 55
            sa[ii] = mk
            mk = _i32(mj - mk)
            if mk < 0:
                mk = _i32(mk + self.MBIG)
            mj = sa[ii]
        for _ in range(1, 5):
            for i in range(1, 56):
                n = i + 30
                if n >= 55:
                    n -= 55
                sa[i] = _i32(sa[i] - sa[1 + n])
                if sa[i] < 0:
                    sa[i] = _i32(sa[i] + self.MBIG)
        self._sa = sa
        self._inext = 0
        self._inextp = 21

    def InternalSample(self) -> int:
        a = self._inext + 1
        if a >= 56:
            a = 1
        b = self._inextp + 1
        if b >= 56:
            b = 1
        r = _i32(self._sa[a] - self._sa[b])
        if r == self.MBIG:
            r -= 1
        if r < 0:
            r = _i32(r + self.MBIG)
        self._sa[a] = r
        self._inext, self._inextp = a, b
        return r

    def Next(self) -> int:
        return self.InternalSample()

    def NextDouble(self) -> float:
        return self.InternalSample() * (1.0 / self.MBIG)


# ---------------------------------------------------------------------------------------------
# Context: the C ABI
# ---------------------------------------------------------------------------------------------
def _csr(histories: Optional[Iterable[Iterable[int]]], rows: int):
    if histories is None:
        return None, None
    lists = [np.asarray(list(h), dtype=np.int32) for h in histories]
    if len(lists) != rows:
        raise ValueError("one history per row is required")
    off = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum([len(h) for h in lists], out=off[1:])
    if off[-1] >= 2**31:
        raise ValueError("history too long for int32 offsets")
    ids = np.concatenate(lists) if lists else np.zeros(0, np.int32)
    return off.astype(np.int32), np.ascontiguousarray(ids, dtype=np.int32)


PATH_FLAGS = {"auto": 0, "block": _lib.VXS_FLAG_PATH_BLOCK, "wave": _lib.VXS_FLAG_PATH_WAVE}
RNG_FLAGS = {None: 0, "talker": _lib.VXS_FLAG_RNG_TALKER, "sub": _lib.VXS_FLAG_RNG_SUB}


class Context:
    """Owns one vxs_ctx (one HIP stream). Not thread-safe; use one per thread.

    ``path`` of the sampling calls selects the kernel: "auto" (the library chooses), "block" (one
    workgroup per row) or "wave" (one wave per row first, vocab <= 3072); results are identical."""

    def __init__(self, device: int = 0, max_rows: int = 0, max_vocab: int = 0, max_hist: int = 0):
        self._lib = load_vxs()
        h = ctypes.c_void_p()
        rc = self._lib.vxs_create(ctypes.byref(h), device, max_rows, max_vocab, max_hist)
        if rc != 0:
            raise SamplerError(rc, f"vxs_create(device={device}) failed")
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.vxs_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self):
        return self._h

    def last_error(self) -> str:
        return self._lib.vxs_last_error(self._h).decode()

    def _check(self, rc: int) -> None:
        if rc != 0:
            _raise(rc, self.last_error())

    def set_stream(self, stream_ptr: Optional[int]) -> None:
        self._check(self._lib.vxs_set_stream(self._h, stream_ptr))

    def stream(self) -> int:
        return self._lib.vxs_get_stream(self._h) or 0

    def synchronize(self) -> None:
        self._check(self._lib.vxs_synchronize(self._h))

    # host-memory batched call ----------------------------------------------------------------
    def sample(self, logits: np.ndarray, params: np.ndarray, u: Optional[np.ndarray] = None,
               hist_off: Optional[np.ndarray] = None, hist_ids: Optional[np.ndarray] = None,
               want_logits: bool = False, want_probs: bool = False, raise_on_error: bool = True,
               path: str = "auto", logits_out: Optional[np.ndarray] = None):
        """Sample every row of `logits` [rows, vocab] (host). `params`: one PARAMS_DTYPE record
        (broadcast) or one per row. Returns ids (and the write-back logits / probabilities).
        `logits_out` (float32 [rows, vocab], C-contiguous) receives the write-back instead of a new
        array; a row that fails keeps what it held."""
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        if logits.ndim == 1:
            logits = logits.reshape(1, -1)
        rows, vocab = logits.shape
        params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
        stride = 0 if params.ndim == 0 or params.size == 1 else 1
        if stride and params.shape[0] != rows:
            raise ValueError("params must be one record or one per row")
        if u is not None:
            u = np.ascontiguousarray(u, dtype=np.float64).reshape(-1)
            if u.shape[0] != rows:
                raise ValueError("u must have one value per row")
        if hist_off is not None:
            hist_off = np.ascontiguousarray(hist_off, dtype=np.int32)
            hist_ids = np.ascontiguousarray(hist_ids if hist_ids is not None else np.zeros(0, np.int32), dtype=np.int32)
        ids = np.empty(rows, dtype=np.int32)
        if logits_out is not None:
            if (logits_out.dtype != np.float32 or logits_out.shape != (rows, vocab)
                    or not logits_out.flags.c_contiguous):
                raise ValueError("logits_out must be a C-contiguous float32 [rows, vocab] array")
            want_logits = True
        out_logits = (logits_out if logits_out is not None else np.empty((rows, vocab), dtype=np.float32)) \
            if want_logits else None
        out_probs = np.empty((rows, vocab), dtype=np.float64) if want_probs else None
        rc = self._lib.vxs_sample(self._h, rows, vocab, ptr(logits), vocab, ptr(hist_off), ptr(hist_ids),
                                  ptr(params), stride, ptr(u), ptr(ids), ptr(out_logits), ptr(out_probs),
                                  PATH_FLAGS[path])
        if rc != 0 and (raise_on_error or rc not in (_lib.VXS_ERR_ID_OUT_OF_RANGE, _lib.VXS_ERR_NONFINITE)):
            _raise(rc, self.last_error())
        if want_logits or want_probs:
            return ids, out_logits, out_probs
        return ids

    # device-resident call (torch tensors or raw pointers) -----------------------------------------
    def sample_device(self, rows: int, vocab: int, logits, ld: int, params, params_stride: int, u, out_ids,
                      hist_off=None, hist_ids=None, out_logits=None, out_probs=None, path: str = "auto") -> None:
        rc = self._lib.vxs_sample_device(self._h, rows, vocab, ptr(logits), ld, ptr(hist_off), ptr(hist_ids),
                                         ptr(params), params_stride, ptr(u), ptr(out_ids), ptr(out_logits),
                                         ptr(out_probs), PATH_FLAGS[path])
        self._check(rc)

    def sample_stats_device(self, rows: int, vocab: int, logits, ld: int, params, params_stride: int, u, out_ids,
                            stats, hist_off=None, hist_ids=None, path: str = "auto", probs=None) -> None:
        """vxs_sample_stats_device: ids plus, for rows of the one-wave nucleus regime, [kept fraction,
        smallest kept probability, kept count, 0] in stats[r] (NaN for other rows), and with probs
        ([rows][vocab] fp64) every entry's final probability for those rows (NaN for other rows)."""
        rc = self._lib.vxs_sample_stats_device(self._h, rows, vocab, ptr(logits), ld, ptr(hist_off), ptr(hist_ids),
                                               ptr(params), params_stride, ptr(u), ptr(out_ids), ptr(stats),
                                               ptr(probs), PATH_FLAGS[path])
        self._check(rc)

    def apply_repetition_penalty(self, logits: np.ndarray, hist_off: np.ndarray, hist_ids: np.ndarray,
                                 penalty: float) -> None:
        """In place on a C-contiguous float32 [rows, vocab] host array."""
        if logits.dtype != np.float32 or not logits.flags.c_contiguous:
            raise ValueError("logits must be a C-contiguous float32 array (modified in place)")
        x = logits.reshape(1, -1) if logits.ndim == 1 else logits
        rows, vocab = x.shape
        self._check(self._lib.vxs_apply_repetition_penalty(
            self._h, rows, vocab, ptr(x), vocab, ptr(np.ascontiguousarray(hist_off, dtype=np.int32)),
            ptr(np.ascontiguousarray(hist_ids, dtype=np.int32)), float(np.float32(penalty))))

    def argmax(self, logits: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(logits, dtype=np.float32)
        x = x.reshape(1, -1) if x.ndim == 1 else x
        ids = np.empty(x.shape[0], dtype=np.int32)
        self._check(self._lib.vxs_argmax(self._h, x.shape[0], x.shape[1], ptr(x), x.shape[1], ptr(ids)))
        return ids

    # resident histories ----------------------------------------------------------------------------
    def history(self, slots: int, cap: int) -> "HistoryStore":
        """A resident history store on this context's device (vxs_history_create)."""
        return HistoryStore(self, slots, cap)

    def sample_batch(self, store: "HistoryStore", logits: np.ndarray, slots, params: np.ndarray,
                     u: Optional[np.ndarray] = None, append: bool = True, raise_on_error: bool = True,
                     path: str = "auto", rng: Optional[str] = None) -> np.ndarray:
        """One batched stage over host rows whose histories live in `store`: row r penalises with
        slot slots[r] and, with `append`, its id is added to that slot (vxs_sample_batch). With
        ``rng="talker"`` or ``"sub"`` the uniforms come from the slots' generators on the device
        (``store.seed``) and `u` is ignored."""
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        if logits.ndim == 1:
            logits = logits.reshape(1, -1)
        rows, vocab = logits.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32).reshape(-1)
        if slots.shape[0] != rows:
            raise ValueError("slots must have one entry per row")
        params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
        stride = 0 if params.ndim == 0 or params.size == 1 else 1
        if stride and params.shape[0] != rows:
            raise ValueError("params must be one record or one per row")
        if u is not None:
            u = np.ascontiguousarray(u, dtype=np.float64).reshape(-1)
            if u.shape[0] != rows:
                raise ValueError("u must have one value per row")
        ids = np.empty(rows, dtype=np.int32)
        rc = self._lib.vxs_sample_batch(self._h, store.handle, rows, vocab, ptr(logits), vocab, ptr(slots),
                                        1 if append else 0, ptr(params), stride, ptr(u), ptr(ids),
                                        PATH_FLAGS[path] | RNG_FLAGS[rng])
        if rc != 0 and (raise_on_error or rc not in (_lib.VXS_ERR_ID_OUT_OF_RANGE, _lib.VXS_ERR_NONFINITE,
                                                     _lib.VXS_ERR_HISTORY_FULL)):
            _raise(rc, self.last_error())
        return ids

    def sample_batch_device(self, store: "HistoryStore", rows: int, vocab: int, logits, ld: int, slots, params,
                            params_stride: int, u, out_ids, append: bool = True, path: str = "auto",
                            rng: Optional[str] = None) -> None:
        """vxs_sample_batch_device: device pointers (torch tensors or ints), asynchronous."""
        rc = self._lib.vxs_sample_batch_device(self._h, store.handle, rows, vocab, ptr(logits), ld, ptr(slots),
                                               1 if append else 0, ptr(params), params_stride, ptr(u),
                                               ptr(out_ids), PATH_FLAGS[path] | RNG_FLAGS[rng])
        self._check(rc)

    # logit heads and embedding lookups (device pointers, asynchronous) ------------------------------
    def head_device(self, rows: int, k: int, n: int, x, ldx: int, w, ldw: int, out, ldo: int) -> None:
        """vxs_head_device: out[r][j] = sum_k x[r][k] * W[j][k] (CodecHead / CodePredictorHead)."""
        self._check(self._lib.vxs_head_device(self._h, rows, k, n, ptr(x), ldx, ptr(w), ldw, ptr(out), ldo))

    def head_int8_device(self, rows: int, k: int, n: int, x, ldx: int, q, ldq: int, scale, out, ldo: int) -> None:
        """vxs_head_int8_device: out[r][j] = scale[j] * sum_k x[r][k] * q[j][k] (WeightPrecision.Int8)."""
        self._check(self._lib.vxs_head_int8_device(self._h, rows, k, n, ptr(x), ldx, ptr(q), ldq, ptr(scale), ptr(out), ldo))

    def head_pack_int8_device(self, k: int, n: int, w, ldw: int, q, ldq: int, scale) -> None:
        """vxs_head_pack_int8_device: PackedMatrix.FromBf16LinearInt8 of a bf16 [n][ldw] weight."""
        self._check(self._lib.vxs_head_pack_int8_device(self._h, k, n, ptr(w), ldw, ptr(q), ldq, ptr(scale)))

    def embed_device(self, rows: int, hidden: int, ids, table, vocab: int, out, ld_out: int, add: bool, status) -> None:
        """vxs_embed_device: out[r] = table[ids[r]] or += it (CodecEmbedding / CodePredictorEmbedding)."""
        self._check(self._lib.vxs_embed_device(self._h, rows, hidden, ptr(ids), ptr(table), vocab, ptr(out), ld_out,
                                               1 if add else 0, ptr(status)))

    def frame_embed_device(self, rows: int, groups: int, hidden: int, codes, ld_codes: int, codec_table, vocab: int,
                           cp_tables, cp_vocab: int, out, ld_out: int, status, addend=None, ld_addend: int = 0,
                           group_stride: int = 1) -> None:
        """vxs_frame_embed_device: FrameEmbedding of `rows` frames (+ the text row `addend`); code g of
        frame r at codes[r * ld_codes + g * group_stride]."""
        self._check(self._lib.vxs_frame_embed_device(self._h, rows, groups, hidden, ptr(codes), ld_codes, group_stride,
                                                     ptr(codec_table), vocab, ptr(cp_tables), cp_vocab, ptr(addend),
                                                     ld_addend, ptr(out), ld_out, ptr(status)))


class HistoryStore:
    """Device-resident histories (vxs_history): ``slots`` sequences of at most ``cap`` ids each, all
    empty at creation. One slot stands for one ``Active.History`` list of GenerateBatch
    (TalkerGenerator.cs:304); the sampler appends to it on the device (History.Add, :374)."""

    def __init__(self, context: Context, slots: int, cap: int):
        self._ctx = context
        self._lib = context._lib
        h = ctypes.c_void_p()
        context._check(self._lib.vxs_history_create(context.handle, slots, cap, ctypes.byref(h)))
        self._h = h
        self.slots = slots
        self.cap = cap

    @property
    def handle(self):
        return self._h

    def set(self, slot: int, ids: Iterable[int] = ()) -> None:
        """Replace one slot's history (an empty one for a newly started sequence)."""
        a = np.ascontiguousarray(list(ids), dtype=np.int32)
        self._ctx._check(self._lib.vxs_history_set(self._ctx.handle, self._h, slot, ptr(a) if a.size else None,
                                                   int(a.size)))

    def seed(self, slot: int, seed: int) -> None:
        """Seed the slot's generators: new Random(seed) (talker) and new Random(seed + 1) (code
        predictor), as a sequence's samplers are built (TalkerGenerator.cs:345-346)."""
        s32 = ((int(seed) + 0x80000000) & 0xFFFFFFFF) - 0x80000000
        self._ctx._check(self._lib.vxs_history_seed(self._ctx.handle, self._h, slot, s32))

    def draw(self, slot: int, stream: str, n: int) -> np.ndarray:
        """The next n NextDouble() of the slot's "talker" or "sub" generator, drawn on the device."""
        out = np.empty(n, dtype=np.float64)
        self._ctx._check(self._lib.vxs_history_draw(self._ctx.handle, self._h, slot, {"talker": 0, "sub": 1}[stream],
                                                    n, ptr(out) if n else None))
        return out

    def get(self, slot: int) -> np.ndarray:
        n = ctypes.c_int(0)
        self._ctx._check(self._lib.vxs_history_get(self._ctx.handle, self._h, slot, None, 0, ctypes.byref(n)))
        out = np.empty(n.value, dtype=np.int32)
        if n.value:
            self._ctx._check(self._lib.vxs_history_get(self._ctx.handle, self._h, slot, ptr(out), n.value,
                                                       ctypes.byref(n)))
        return out

    def close(self) -> None:
        """Free the store once the context's queued work is done (freeing waits for the device)."""
        if getattr(self, "_h", None):
            try:
                if self._ctx.handle:
                    self._ctx.synchronize()
            finally:
                self._lib.vxs_history_destroy(self._h)
                self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


_default: dict[int, Context] = {}
_default_lock = threading.Lock()


def default_context(device: int = 0) -> Context:
    with _default_lock:
        ctx = _default.get(device)
        if ctx is None:
            ctx = _default[device] = Context(device)
        return ctx


# ---------------------------------------------------------------------------------------------
# Sampler (Sampler.cs:17-96)
# ---------------------------------------------------------------------------------------------
class Sampler:
    """``Sampler(seed)`` with ``ApplyRepetitionPenalty``, ``Select`` and ``ArgMax``; the GPU does the
    work, the RNG stays on the host (one NextDouble per sampled Select, none per greedy Select)."""

    def __init__(self, seed: Optional[int] = None, context: Optional[Context] = None):
        self._rng = DotNetRandom(seed)
        self._ctx = context

    @property
    def context(self) -> Context:
        return self._ctx or default_context()

    @staticmethod
    def ApplyRepetitionPenalty(logits: np.ndarray, history: Iterable[int], penalty: float,
                               context: Optional[Context] = None) -> None:
        if np.float32(penalty) == np.float32(1.0):
            return
        ctx = context or default_context()
        hist = np.asarray(list(history), dtype=np.int32)
        ctx.apply_repetition_penalty(logits, np.array([0, hist.size], np.int32), hist, penalty)

    def NextUniform(self, opts: SamplingOptions) -> float:
        """The uniform one ``Select(logits, opts)`` would consume (none, returned as 0, when greedy);
        batched callers draw each row's uniform from its own sequence's Sampler with it."""
        return self._rng.NextDouble() if opts.DoSample else 0.0

    def Select(self, logits: np.ndarray, opts: SamplingOptions) -> int:
        """Select one id from a float32 row; the row is updated in place the way the C# span is
        (temperature and top-k mask when sampling)."""
        p = make_params(opts)
        u = np.array([self._rng.NextDouble()]) if opts.DoSample else None
        ids, out, _ = self.context.sample(logits, p, u, want_logits=True)
        if logits.dtype == np.float32 and logits.flags.c_contiguous:
            logits.reshape(-1)[:] = out.reshape(-1)
        return int(ids[0])

    @staticmethod
    def ArgMax(x: np.ndarray, context: Optional[Context] = None) -> int:
        return int((context or default_context()).argmax(np.asarray(x, dtype=np.float32))[0])
