"""Generation loops around the sampler, mirroring the sampling side of voxwerk's TalkerGenerator.

``generate`` follows ``TalkerGenerator.Generate`` (src/Voxwerk/Talker/TalkerGenerator.cs:213-287)
for one sequence; ``generate_batch`` follows ``TalkerGenerator.GenerateBatch`` (:322-455) for many
sequences in lockstep with continuous batching. The sampler work goes through the HIP library: one
``vxs_sample_batch`` call per stage per step over all active rows, each row with its own options and
its own uniform, histories resident on the GPU and appended there. Everything the reference does with
its transformer (prefill, the code predictor, the talker step) is the caller's ``model``, outside this
library: it only has to turn codes into logits.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Any, Callable, List, Optional, Protocol, Sequence

import numpy as np

from .sampler import (CODEC_EOS_ID, CP_VOCAB, TALKER_VOCAB, Context, GenerationOptions, Sampler, default_context,
                      sub_talker_params, talker_params)

NUM_CODE_GROUPS = 16  # Qwen3TtsConfig.NumCodeGroups: codebook 0 from the talker, 1..15 from the code predictor


class OperationCanceledError(Exception):
    """Raised when a generation loop sees its token cancelled (.NET's OperationCanceledException)."""


class CancellationToken:
    """The ``CancellationToken`` the reference's loops take (TalkerGenerator.cs:213, :323): a flag set
    from any thread by ``cancel()``, checked once per step. Cancellation leaves the context and the
    library usable; a batch releases its resident history store on the way out."""

    def __init__(self) -> None:
        self._cancelled = False

    def cancel(self) -> None:
        self._cancelled = True

    @property
    def is_cancellation_requested(self) -> bool:
        return self._cancelled

    def throw_if_cancellation_requested(self) -> None:
        if self._cancelled:
            raise OperationCanceledError("generation cancelled")


class TalkerModel(Protocol):
    """The model side of generation. ``job`` identifies a sequence (its prompt and its caches).

    prefill(job) -> [V] codec-head logits of the prompt's last position (TalkerGenerator.cs:350-357)
    code_predictor(jobs, g, frames) -> [A, CV] logits of codebook g for each job, given the codes
        frames[i, :g] chosen so far in its current frame (:404-426)
    talker_step(jobs, steps, frames) -> [A, V] codec-head logits after feeding each job's finished
        frame at its step (:429-443)
    """

    def prefill(self, job: int) -> np.ndarray: ...

    def code_predictor(self, jobs: Sequence[int], g: int, frames: np.ndarray) -> np.ndarray: ...

    def talker_step(self, jobs: Sequence[int], steps: Sequence[int], frames: np.ndarray) -> np.ndarray: ...


@dataclass(frozen=True)
class BatchJob:
    """One request of ``generate_batch`` (TalkerGenerator.BatchJob, TalkerGenerator.cs:290)."""

    Prompt: Any
    Options: GenerationOptions


@dataclass
class _Active:
    job: int
    options: GenerationOptions
    slot: int
    sampler: Sampler
    sub_sampler: Sampler
    logits: np.ndarray
    frames: List[np.ndarray] = field(default_factory=list)
    step: int = 0


def _sub_seed(opts: GenerationOptions) -> Optional[int]:
    """``Seed + 1`` in C#'s unchecked int arithmetic (TalkerGenerator.cs:218, :346)."""
    if opts.Seed is None:
        return None
    return ((opts.Seed + 1 + 0x80000000) & 0xFFFFFFFF) - 0x80000000


def generate(job: int, opts: GenerationOptions, model: TalkerModel, context: Optional[Context] = None,
             vocab: int = TALKER_VOCAB, groups: int = NUM_CODE_GROUPS, eos_id: int = CODEC_EOS_ID,
             ct: Optional[CancellationToken] = None, on_frame: Optional[Callable[[int], None]] = None) -> List[np.ndarray]:
    """One sequence, step by step as ``Generate`` (TalkerGenerator.cs:213-287): penalty, suppression
    and ``Select`` on the talker row, then ``groups - 1`` code-predictor ``Select`` calls. Returns the
    frames, each ``groups`` codes. ``ct`` is checked at the start of every step (:243) and raises
    ``OperationCanceledError``; ``on_frame(n)`` is called with the frame count after each frame (:277)."""
    ctx = context or default_context()
    sampler = Sampler(opts.Seed, ctx)
    sub_sampler = Sampler(_sub_seed(opts), ctx)
    logits = np.array(model.prefill(job), dtype=np.float32).reshape(-1)
    history: List[int] = []
    frames: List[np.ndarray] = []
    for t in range(opts.MaxNewTokens):
        if ct is not None:
            ct.throw_if_cancellation_requested()                                               # :243
        lg = np.ascontiguousarray(logits[:vocab], dtype=np.float32)
        Sampler.ApplyRepetitionPenalty(lg, history, opts.RepetitionPenalty, context=ctx)      # :246
        keep = lg[eos_id]
        lg[vocab - 1024:] = -np.inf                                                            # :247
        lg[eos_id] = keep
        if t < 2:
            lg[eos_id] = -np.inf                                                               # :248
        code0 = sampler.Select(lg, opts.Talker)                                                # :249
        history.append(code0)
        if code0 == eos_id or t == opts.MaxNewTokens - 1:                                     # :251
            break
        frame = np.zeros(groups, dtype=np.int32)
        frame[0] = code0
        for g in range(1, groups):                                                             # :262-275
            cp = np.array(model.code_predictor([job], g, frame[None, :]), dtype=np.float32).reshape(-1)
            frame[g] = sub_sampler.Select(cp, opts.SubTalker)
        frames.append(frame)
        if on_frame is not None:
            on_frame(len(frames))                                                              # :277
        logits = np.array(model.talker_step([job], [t], frame[None, :]), dtype=np.float32).reshape(-1)
    return frames


def generate_batch(jobs: Sequence[BatchJob], max_batch: int, on_done: Callable[[int, List[np.ndarray]], None],
                   model: TalkerModel, context: Optional[Context] = None, vocab: int = TALKER_VOCAB,
                   cp_vocab: int = CP_VOCAB, groups: int = NUM_CODE_GROUPS, eos_id: int = CODEC_EOS_ID,
                   path: str = "auto", device_rng: bool = False, ct: Optional[CancellationToken] = None) -> None:
    """``GenerateBatch`` (TalkerGenerator.cs:322-455): up to ``max_batch`` sequences advance in
    lockstep; a finished one is reported through ``on_done(job, frames)`` and its slot refilled from the
    queue. Each job keeps its own ``Sampler(Seed)`` / ``Sampler(Seed + 1)``, so its frames do not
    depend on the batch it ran in.

    Per step: one ``vxs_sample_batch`` over the talker rows (penalty from the resident history,
    suppression, select, on-device ``History.Add``), then one per code-predictor group. With
    ``device_rng`` the two generators of each job live in its slot and draw on the GPU (the same
    .NET sequences, so the same frames); otherwise the host draws them. ``ct`` is checked at the
    start of every step (:332) and raises ``OperationCanceledError``; jobs already reported stay
    reported, the rest are dropped, and the resident history store is released."""
    if max_batch <= 0:
        raise ValueError("max_batch must be positive")
    ctx = context or default_context()
    if not jobs:
        return
    cap = max(max(j.Options.MaxNewTokens for j in jobs), 1)  # one history id per step at most
    store = ctx.history(min(max_batch, len(jobs)), cap)
    free = list(range(store.slots))[::-1]
    active: List[_Active] = []
    nxt = 0
    try:
        while nxt < len(jobs) or active:
            if ct is not None:
                ct.throw_if_cancellation_requested()                                           # :332
            while len(active) < max_batch and nxt < len(jobs):                                 # :334-360
                opts = jobs[nxt].Options
                slot = free.pop()
                store.set(slot, ())  # a new sequence starts with an empty history
                if device_rng:
                    store.seed(slot, opts.Seed if opts.Seed is not None else int.from_bytes(os.urandom(4), "little"))
                logits = np.array(model.prefill(nxt), dtype=np.float32).reshape(-1)
                active.append(_Active(nxt, opts, slot, Sampler(opts.Seed, ctx), Sampler(_sub_seed(opts), ctx), logits))
                nxt += 1

            # 1. codebook 0 for every active sequence; retire finished ones             :362-388
            A = len(active)
            x = np.stack([a.logits[:vocab] for a in active])
            params = np.stack([talker_params(a.options, a.step, vocab, eos_id) for a in active])
            slots = [a.slot for a in active]
            if device_rng:
                code0 = ctx.sample_batch(store, x, slots, params, None, append=True, path=path, rng="talker")
            else:
                u = np.array([a.sampler.NextUniform(a.options.Talker) for a in active])
                code0 = ctx.sample_batch(store, x, slots, params, u, append=True, path=path)
            keep: List[_Active] = []
            first: List[int] = []
            for a, c in zip(active, code0.tolist()):
                if c == eos_id or a.step == a.options.MaxNewTokens - 1:
                    on_done(a.job, a.frames)
                    free.append(a.slot)
                    continue
                keep.append(a)
                first.append(c)
            active = keep
            A = len(active)
            if A == 0:
                continue

            # 2. code predictor for all sequences in lockstep                          :404-426
            frames = np.zeros((A, groups), dtype=np.int32)
            frames[:, 0] = first
            job_ids = [a.job for a in active]
            sub = np.stack([sub_talker_params(a.options) for a in active])
            for g in range(1, groups):
                cp = np.ascontiguousarray(model.code_predictor(job_ids, g, frames), dtype=np.float32)
                if cp.shape != (A, cp_vocab):
                    raise ValueError(f"code_predictor returned {cp.shape}, expected {(A, cp_vocab)}")
                if device_rng:  # the code-predictor generators of the slots; no history involved
                    frames[:, g] = ctx.sample_batch(store, cp, [a.slot for a in active], sub, None, append=False,
                                                    path=path, rng="sub")
                else:
                    u = np.array([a.sub_sampler.NextUniform(a.options.SubTalker) for a in active])
                    frames[:, g] = ctx.sample(cp, sub, u, path=path)

            # 3. one talker step for all sequences                                     :429-448
            steps = [a.step for a in active]
            for i, a in enumerate(active):
                a.frames.append(frames[i].copy())
                a.step += 1
            nl = np.ascontiguousarray(model.talker_step(job_ids, steps, frames), dtype=np.float32)
            if nl.shape[0] != A or nl.shape[1] < vocab:
                raise ValueError(f"talker_step returned {nl.shape}, expected ({A}, {vocab})")
            for i, a in enumerate(active):
                a.logits = nl[i]
    finally:
        store.close()
