"""Test helpers for the generation loops: a deterministic stand-in for the talker model, and a context
that runs every sampler call on the CPU oracle (TEST INFRASTRUCTURE: the oracle is the checker here).

The stand-in's logits for a sequence depend only on its job index, its step and the codes it chose,
never on the batch it runs in, which is the property the reference's batched-generation parity test
relies on (tests/Voxwerk.Tests/TalkerParityTests.cs:125-147)."""
from __future__ import annotations

import zlib

import numpy as np

from oracle import ref
from voxwerk_amd.sampler import CODEC_EOS_ID, CP_VOCAB, TALKER_VOCAB


class SyntheticTalker:
    def __init__(self, seed: int = 0, vocab: int = TALKER_VOCAB, cp_vocab: int = CP_VOCAB, eos_id: int = CODEC_EOS_ID):
        self.seed, self.vocab, self.cp_vocab, self.eos_id = seed, vocab, cp_vocab, eos_id
        self.calls = {"prefill": 0, "code_predictor": 0, "talker_step": 0}

    def _rng(self, *key) -> np.random.Generator:
        return np.random.Generator(np.random.PCG64(np.random.SeedSequence([self.seed, *[int(k) & 0xFFFFFFFF for k in key]])))

    def _talker(self, job: int, step: int, h: int) -> np.ndarray:
        x = (self._rng(1, job, step + 1, h).standard_normal(self.vocab) * 2.5).astype(np.float32)
        x[self.eos_id] = np.float32(-2.0 + 1.0 * (step + 1))  # the end becomes likelier as a sequence grows
        fav = (job * 7 + np.arange(4) * 131) % (self.vocab - 1024)
        x[fav] += np.float32(3.0)  # favourite codes, so that the repetition penalty matters
        return x

    def prefill(self, job: int) -> np.ndarray:
        self.calls["prefill"] += 1
        return self._talker(job, -1, 0)

    def code_predictor(self, jobs, g, frames) -> np.ndarray:
        self.calls["code_predictor"] += 1
        out = np.empty((len(jobs), self.cp_vocab), np.float32)
        for i, j in enumerate(jobs):
            h = zlib.crc32(np.ascontiguousarray(frames[i, :g], np.int32).tobytes())
            out[i] = self._rng(2, j, g, h).standard_normal(self.cp_vocab) * 2.0
        return out

    def talker_step(self, jobs, steps, frames) -> np.ndarray:
        self.calls["talker_step"] += 1
        return np.stack([self._talker(j, s, zlib.crc32(np.ascontiguousarray(frames[i], np.int32).tobytes()))
                         for i, (j, s) in enumerate(zip(jobs, steps))])


class OracleStore:
    def __init__(self, slots: int, cap: int):
        self.slots, self.cap = slots, cap
        self.hist = [[] for _ in range(slots)]

    def set(self, slot, ids=()):
        self.hist[slot] = [int(i) for i in ids]

    def get(self, slot):
        return np.array(self.hist[slot], np.int32)

    def close(self):
        pass


def _csr(lists):
    off = np.zeros(len(lists) + 1, np.int32)
    np.cumsum([len(h) for h in lists], out=off[1:])
    ids = np.array([i for h in lists for i in h], np.int32)
    return off, ids


class OracleContext:
    """The subset of ``voxwerk_amd.sampler.Context`` the generation loops use, on the CPU oracle."""

    def history(self, slots, cap):
        return OracleStore(slots, cap)

    def sample(self, logits, params, u=None, hist_off=None, hist_ids=None, want_logits=False, want_probs=False,
               raise_on_error=True, path="auto"):
        r = ref.sample(logits, params, u, hist_off, hist_ids, want_logits=want_logits, want_probs=want_probs)
        assert r["rc"] == 0
        if want_logits or want_probs:
            return r["ids"], r["logits"], r["probs"]
        return r["ids"]

    def apply_repetition_penalty(self, logits, hist_off, hist_ids, penalty):
        assert ref.apply_penalty(logits, hist_off, hist_ids, penalty) == 0

    def sample_batch(self, store, logits, slots, params, u=None, append=True, raise_on_error=True, path="auto"):
        off, ids = _csr([store.hist[s] for s in slots])
        out = self.sample(logits, params, u, off, ids)
        if append:
            for s, c in zip(slots, out.tolist()):
                if c >= 0:
                    store.hist[s].append(c)
        return out


class RecordingContext:
    """Wraps a GPU context: forwards every call, and keeps its inputs, the host copy of each resident
    history and the ids, so that each call can be checked against the oracle afterwards."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.calls = []
        self.mirror = {}

    def history(self, slots, cap):
        store = self.ctx.history(slots, cap)
        mirror = self.mirror
        set_ = store.set

        def tracked_set(slot, ids=()):
            mirror[slot] = [int(i) for i in ids]
            set_(slot, ids)

        store.set = tracked_set
        return store

    def sample(self, logits, params, u=None, path="auto", **kw):
        ids = self.ctx.sample(logits, params, u, path=path, **kw)
        self.calls.append((np.array(logits, np.float32), np.array(params), None if u is None else np.array(u), None,
                           np.array(ids if not isinstance(ids, tuple) else ids[0])))
        return ids

    def sample_batch(self, store, logits, slots, params, u=None, append=True, path="auto", **kw):
        hist = [list(self.mirror[s]) for s in slots]
        ids = self.ctx.sample_batch(store, logits, slots, params, u, append=append, path=path, **kw)
        self.calls.append((np.array(logits, np.float32), np.array(params), None if u is None else np.array(u), hist,
                           ids.copy()))
        if append:
            for s, c in zip(slots, ids.tolist()):
                if c >= 0:
                    self.mirror[s].append(c)
        return ids

    def check_against_oracle(self):
        """Classify every recorded call against the oracle (same inputs): (calls, rows, boundary rows)."""
        rows = boundary = 0
        for i, (x, p, u, hist, ids) in enumerate(self.calls):
            off, hids = _csr(hist) if hist is not None else (None, None)
            ora = ref.sample(x, p, u, off, hids)
            assert ora["rc"] == 0
            c = ref.classify(ids, ora)
            assert c["unexplained"] == 0, f"call {i}: ids differ away from boundaries at rows {c['unexplained_rows']}"
            rows += c["rows"]
            boundary += c["draw_boundary"] + c["topp_boundary"]
        return len(self.calls), rows, boundary
