"""Batched sampling for the engine's step loop, with device-resident histories.

``LLMEngine.step`` (``src/pagellm/engine/llm_engine.py:238-254``) calls
``_append_token`` once per finished sequence, and each call samples one row
with the sequence's full token history (``sample(logits, params, seq.rng,
seq.tokens)``, ``:283``) and then appends the token (``:284``).  The
:class:`BatchSampler` here replaces those per-row calls with one launch per
step:

* the histories live in HBM (:class:`DeviceHistories`), one fixed slot per
  sequence, and grow in place by one id per step on the device
  (``plh_append_ids``, reading the ids the sampler just wrote) instead of
  being re-uploaded every step;
* each sequence keeps its own numpy ``Generator`` on the host: one
  ``rng.random()`` per non-greedy row, none for greedy rows, in row order,
  exactly as the per-row loop consumes them (``sampling.py:98``, ``:102-106``);
* only the token ids come back to the host.

Forked sequences (``SamplingParams.n > 1``, ``llm_engine.py:259-278``) join
with the parent's token list at the time of the fork, so each child samples
against its own copy of the history, as in the reference.
"""

from __future__ import annotations

from typing import Hashable, Sequence

import numpy as np

from . import _native
from .sampling import _draw_uniforms, _expand_params, _history_ids, _is_torch_cuda, _nucleus_hint, _pack_params

__all__ = ["BatchSampler", "DeviceHistories"]


class DeviceHistories:
    """Token histories (prompt + outputs) of live sequences in HBM.

    One slot of ``max_len`` int32 ids per sequence in a single device slab;
    row b of a step reads ``slab[slot * max_len : slot * max_len + length]``
    through the sampler's span form of the history (``PLH_SAMPLE_HIST_SPANS``).
    """

    def __init__(self, vocab_size: int, max_seqs: int, max_len: int, *, ctx: _native.Context | None = None):
        if max_seqs < 1 or max_len < 1:
            raise ValueError("max_seqs and max_len must be >= 1")
        self.ctx = ctx if ctx is not None else _native.default_context()
        self.V = int(vocab_size)
        self.max_seqs = int(max_seqs)
        self.max_len = int(max_len)
        self.slab = self.ctx.empty((self.max_seqs * self.max_len,), np.int32)
        self._free = list(range(self.max_seqs - 1, -1, -1))
        self._slot: dict[Hashable, int] = {}
        self._len: dict[Hashable, int] = {}

    def __contains__(self, key) -> bool:
        return key in self._slot

    def __len__(self) -> int:
        return len(self._slot)

    def length(self, key) -> int:
        return self._len[key]

    def add(self, key, tokens) -> None:
        """A new sequence (or a fork) with its current token list."""
        if key in self._slot:
            raise ValueError(f"sequence {key!r} already has a history")
        ids = _history_ids(tokens, self.V)
        if ids.size > self.max_len:
            raise ValueError(f"history of {ids.size} tokens exceeds max_len {self.max_len}")
        if not self._free:
            raise RuntimeError(f"all {self.max_seqs} history slots are in use")
        slot = self._free.pop()
        if ids.size:
            c = self.ctx
            c._check(c.lib.plh_h2d(c.handle, self.slab.ptr + 4 * slot * self.max_len, ids.ctypes.data, ids.nbytes))
        self._slot[key] = slot
        self._len[key] = int(ids.size)

    def remove(self, key) -> None:
        """A finished or aborted sequence gives its slot back."""
        slot = self._slot.pop(key)
        del self._len[key]
        self._free.append(slot)

    def download(self, key) -> np.ndarray:
        """The sequence's history as the device holds it (for checks)."""
        n = self._len[key]
        out = np.empty(n, dtype=np.int32)
        if n:
            c = self.ctx
            c._check(c.lib.plh_d2h(c.handle, out.ctypes.data, self.slab.ptr + 4 * self._slot[key] * self.max_len,
                                   out.nbytes))
        return out

    def _slots_lengths(self, keys: Sequence) -> tuple[np.ndarray, np.ndarray]:
        B = len(keys)
        slots = np.fromiter(map(self._slot.__getitem__, keys), dtype=np.int64, count=B)
        lens = np.fromiter(map(self._len.__getitem__, keys), dtype=np.int64, count=B)
        return slots, lens

    def spans(self, keys: Sequence, active: Sequence[bool]) -> np.ndarray:
        """int64 [2B] (start, end) per row; inactive rows get an empty span."""
        slots, lens = self._slots_lengths(keys)
        sp = np.empty(2 * len(keys), dtype=np.int64)
        sp[0::2] = slots * self.max_len
        sp[1::2] = sp[0::2] + np.where(np.asarray(active, dtype=bool), lens, 0)
        return sp

    def spans_and_positions(self, keys: Sequence, active) -> tuple[np.ndarray, np.ndarray]:
        """spans(keys, active) and append_positions(keys) in one pass."""
        slots, lens = self._slots_lengths(keys)
        full = lens >= self.max_len
        if full.any():
            key = keys[int(np.argmax(full))]
            raise RuntimeError(f"history of {key!r} is full ({self.max_len} tokens)")
        start = slots * self.max_len
        sp = np.empty(2 * len(keys), dtype=np.int64)
        sp[0::2] = start
        sp[1::2] = start + np.where(np.asarray(active, dtype=bool), lens, 0)
        return sp, start + lens

    def append_positions(self, keys: Sequence) -> np.ndarray:
        """int64 [B]: where each row's next id goes."""
        slots, lens = self._slots_lengths(keys)
        full = lens >= self.max_len
        if full.any():
            key = keys[int(np.argmax(full))]
            raise RuntimeError(f"history of {key!r} is full ({self.max_len} tokens)")
        return slots * self.max_len + lens

    def advance(self, keys: Sequence) -> None:
        for key in keys:
            self._len[key] += 1


class BatchSampler:
    """One sampler launch per engine step over the rows of finished
    sequences (``llm_engine.py:238-254``), histories kept in HBM."""

    def __init__(self, histories: DeviceHistories):
        self.hist = histories
        self.ctx = histories.ctx
        # the last step's packed parameters, with references to its
        # SamplingParams objects (so that equal ids mean the same objects)
        self._packed = None

    def sample(self, logits, params, rngs: Sequence | None, keys: Sequence, *, uniforms=None) -> np.ndarray:
        """Samples one token per row and appends it to the row's history.

        ``logits`` is [B, V] (numpy, or a torch CUDA tensor read in place on
        torch's current stream); ``params`` one SamplingParams or one per
        row; ``rngs[b]`` row b's Generator (None allowed for greedy rows);
        ``keys[b]`` the sequence of row b, which must be in the histories.
        Returns int64 ids [B].
        """
        c = self.ctx
        B = len(keys)
        if B == 0:
            return np.zeros(0, dtype=np.int64)
        if _is_torch_cuda(logits):
            import torch

            if logits.dim() != 2 or logits.stride(1) != 1 or int(logits.shape[0]) != B:
                raise ValueError("logits must be [B, V] with unit stride in the vocabulary dimension")
            if logits.dtype not in (torch.float32, torch.float64):
                raise TypeError("torch logits must be float32 or float64")
            V = int(logits.shape[1])
            ptr, ld = logits.data_ptr(), int(logits.stride(0))
            code = _native.PLH_F64 if logits.dtype == torch.float64 else _native.PLH_F32
            c.set_stream(torch.cuda.current_stream(logits.device).cuda_stream)
        else:
            host = np.asarray(logits)
            if host.dtype != np.float32 and host.dtype != np.float64:
                host = host.astype(np.float64)
            host = np.ascontiguousarray(host)
            if host.ndim != 2 or host.shape[0] != B:
                raise ValueError("logits must be [B, V]")
            V = host.shape[1]
            dev, ld = c.upload_rows("eng_logits", host)
            ptr, code = dev.ptr, _native.dtype_code(host.dtype)
            c.set_stream(None)
        if V != self.hist.V:
            raise ValueError(f"vocabulary {V} does not match the histories' {self.hist.V}")
        params = _expand_params(params, B)
        u = (np.asarray(uniforms, dtype=np.float64).reshape(B) if uniforms is not None
             else _draw_uniforms(params, rngs, B))
        ids = list(map(id, params))
        if self._packed is not None and self._packed[0] == ids:
            t, k, p, r = self._packed[2]  # the same requests in the same rows as the last step
        else:
            t, k, p, r = _pack_params(params)
            self._packed = (ids, list(params), (t, k, p, r))
        # sampling.py:56: only rows whose penalty is active read their history
        spans, pos = self.hist.spans_and_positions(keys, r != 1.0)
        # every per-row array in one page-locked host buffer, one queued copy
        # to the device (the download of the ids below waits for it)
        parts = [t, p, r, u, spans, pos, k]
        offs = np.cumsum([0] + [a.nbytes for a in parts])
        stage = c.pinned("eng_stage", int(offs[-1]))
        for a, o in zip(parts, offs[:-1]):
            stage[o:o + a.nbytes] = np.ascontiguousarray(a).view(np.uint8)
        d = c.scratch("eng_stage", (int(offs[-1]),), np.uint8)
        c.h2d_async(d.ptr, stage[:int(offs[-1])])
        d_t, d_p, d_r, d_u, d_sp, d_pos, d_k = (d.ptr + int(o) for o in offs[:-1])
        out = c.scratch("eng_out", (B,), np.int32)
        c.sample(ptr, code, ld, B, V, self.hist.slab.ptr, d_sp, d_t, d_k, d_p, d_r, d_u,
                 out.ptr, None, _native.PLH_SAMPLE_HIST_SPANS | _nucleus_hint(t, k, p, V))
        # llm_engine.py:284: the token joins the history, on the device
        c.append_ids(self.hist.slab.ptr, d_pos, out.ptr, B)
        ids = out.download().astype(np.int64)
        self.hist.advance(keys)
        return ids

