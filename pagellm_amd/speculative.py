"""Drop-in replacement for the accept/resample step of
``pagellm.engine.speculative`` (``verify``, ``speculative.py:38-60``),
computed on MI355X, plus the batched :func:`verify_batch`.

``verify`` keeps the reference's randomness exactly: the reference calls
``rng.random()`` once per accept test, stopping at the first rejection, then
once for the emitted token (residual or bonus).  The host cannot know the
stop position in advance, so it snapshots the Generator, draws k+1 uniforms,
lets the kernel walk the tests, then restores the snapshot and replays
exactly the number of draws the reference would have made.

:func:`draft_step` and :func:`verify_step` batch the rest of one round of
``SpeculativeDecoder.generate`` (``speculative.py:113-131``) across many
sequences: the draft distributions ``q = probs(...)`` and their draws, and
the target distributions ``p_rows`` with their per-position histories
(``ctx + drafts[:i]``, ``:127``), stay on the device and feed the verify
kernel directly; only tokens and accept counts come back.
"""

from __future__ import annotations

import numpy as np

from . import _native
from .sampling import _as_float_rows, _expand_params, _history_ids, _pack_histories, _pack_params

__all__ = ["draft_buffer", "draft_step", "verify", "verify_batch", "verify_step"]


def _check_draft(draft: np.ndarray, V: int) -> np.ndarray:
    d = np.asarray(draft, dtype=np.int64)
    if d.size:
        lo, hi = int(d.min()), int(d.max())
        if hi >= V or lo < -V:
            raise IndexError(f"index {hi if hi >= V else lo} is out of bounds for axis 0 with size {V}")
        d = np.where(d < 0, d + V, d)  # numpy indexing wraps negative ids
    return d.astype(np.int32)


def _run(c, p, q, draft, accept_u, draw_u, per_stop):
    """p [B,k+1,V], q [B,k,V] (same float dtype), draft int32 [B,k]."""
    B, k1, V = p.shape
    k = k1 - 1
    c.set_stream(None)
    d_p = c.scratch_upload("ver_p", p)
    d_q = c.scratch_upload("ver_q", q) if k else None
    d_d = c.scratch_upload("ver_d", draft) if k else None
    d_a = c.scratch_upload("ver_a", accept_u) if k else None
    d_w = c.scratch_upload("ver_w", draw_u)
    d_t = c.scratch("ver_tok", (B, k + 1), np.int32)
    d_n = c.scratch("ver_n", (B,), np.int32)
    c.verify(
        d_p.ptr, d_q.ptr if d_q else None, _native.dtype_code(p.dtype), B, k, V,
        d_d.ptr if d_d else None, d_a.ptr if d_a else None, d_w.ptr, per_stop, d_t.ptr, d_n.ptr,
    )
    return d_t.download(), d_n.download()


def verify(p_rows: np.ndarray, q_rows: np.ndarray, draft_tokens, rng) -> tuple[list[int], int]:
    """``speculative.py:38-60``.  p_rows: (k+1, V) target distributions;
    q_rows: (k, V) draft distributions.  Returns (emitted tokens, number of
    accepted draft tokens) and leaves ``rng`` exactly where the reference
    would."""
    draft = list(draft_tokens)
    k = len(draft)
    p = _as_float_rows(p_rows)
    if p.ndim != 2 or p.shape[0] < k + 1:
        raise ValueError("p_rows must be (k+1, V)")
    p = p[: k + 1]
    V = p.shape[1]
    q = _as_float_rows(q_rows) if k else np.zeros((0, V), dtype=p.dtype)
    if k and (q.ndim != 2 or q.shape[0] < k or q.shape[1] != V):
        raise ValueError("q_rows must be (k, V)")
    q = q[:k]
    dt = np.result_type(p.dtype, q.dtype)
    p, q = p.astype(dt, copy=False), q.astype(dt, copy=False)
    d = _check_draft(draft, V)

    state = rng.bit_generator.state
    u = np.array([rng.random() for _ in range(k + 1)], dtype=np.float64)
    accept_u = u[:k]
    # stop at s (< k: rejected at s, uniforms u_0..u_s for tests, u_{s+1} for
    # the draw; == k: all accepted, u_k for the bonus draw)
    draw_u = np.array([u[min(s + 1, k)] for s in range(k + 1)], dtype=np.float64)
    c = _native.default_context()
    toks, n = _run(c, p[None], q[None], d[None], accept_u[None], draw_u[None], True)
    s = int(n[0])
    consumed = s + 2 if s < k else k + 1
    rng.bit_generator.state = state
    for _ in range(consumed):
        rng.random()
    out = [int(t) for t in toks[0, : s + 1]]
    # accepted entries are the caller's draft tokens as given
    out[:s] = [draft[i] for i in range(s)]
    return out, s


def verify_batch(p, q, draft, accept_u, resample_u=None, *, ctx: _native.Context | None = None):
    """Batched verify.  p [B,k+1,V], q [B,k,V], draft [B,k].

    Two forms of randomness:

    * ``verify_batch(p, q, draft, rngs)``: ``rngs[b]`` is row b's Generator,
      consumed exactly as the reference's ``verify`` consumes it
      (``speculative.py:50``, ``:57``, ``:59``): one ``random()`` per accept
      test up to the first rejection, then one for the emitted token.  Each
      Generator is left where the reference leaves it.
    * ``verify_batch(p, q, draft, accept_u, resample_u)``: explicit uniforms,
      test i of row b uses ``accept_u[b, i]`` and the emitted (residual or
      bonus) token ``resample_u[b]``.

    Returns (tokens int64 [B,k+1] padded with -1, n_acc int64 [B])."""
    c = ctx if ctx is not None else _native.default_context()
    p = _as_float_rows(p)
    q = _as_float_rows(q)
    dt = np.result_type(p.dtype, q.dtype)
    p, q = p.astype(dt, copy=False), q.astype(dt, copy=False)
    B, k1, V = p.shape
    k = k1 - 1
    if q.shape != (B, k, V):
        raise ValueError(f"q must be {(B, k, V)}, got {q.shape}")
    d = _check_draft(np.asarray(draft).reshape(B, k), V)
    if resample_u is None:
        rngs = list(accept_u)
        if len(rngs) != B:
            raise ValueError(f"expected {B} Generators, got {len(rngs)}")
        # per row: k + 1 uniforms drawn ahead (u_0..u_{k-1} for the tests;
        # the draw at stop s uses u_{s+1}, or u_k after k acceptances), then
        # each Generator replayed to the count the reference consumes
        states = [g.bit_generator.state for g in rngs]
        u = np.array([[g.random() for _ in range(k + 1)] for g in rngs], dtype=np.float64).reshape(B, k + 1)
        a = np.ascontiguousarray(u[:, :k])
        w = np.ascontiguousarray(u[:, np.minimum(np.arange(k + 1) + 1, k)])
        toks, n = _run(c, p, q, d, a, w, True)
        for g, st, s in zip(rngs, states, n):
            g.bit_generator.state = st
            for _ in range(int(s) + 2 if s < k else k + 1):
                g.random()
        return toks.astype(np.int64), n.astype(np.int64)
    a = np.ascontiguousarray(accept_u, dtype=np.float64).reshape(B, k)
    w = np.ascontiguousarray(resample_u, dtype=np.float64).reshape(B)
    toks, n = _run(c, p, q, d, a, w, False)
    return toks.astype(np.int64), n.astype(np.int64)


def _probs_rows(c, x: np.ndarray, dev, hist, tag: str):
    """plh_sample over the rows of x [N, V] with the processed distributions
    exported.  dev: device addresses of the per-row (t, k, p, r, u) arrays;
    hist: (ids, offsets, flags) device addresses of the histories, or None.
    Returns (ids int32 [N] on the device, probs float64 [N, V] on the
    device)."""
    N, V = x.shape
    d_x, ld = c.upload_rows(f"{tag}_x", x)
    out = c.scratch(f"{tag}_out", (N,), np.int32)
    probs = c.scratch(f"{tag}_probs", (N, V), np.float64)
    h_ids, h_off, flags = hist if hist is not None else (None, None, 0)
    c.sample(d_x.ptr, _native.dtype_code(x.dtype), ld, N, V, h_ids, h_off, *dev, out.ptr, probs.ptr, flags)
    return out, probs


def _round_histories(contexts, params, d: np.ndarray, V: int):
    """The histories of one round's B * (k+1) target rows
    (``ctx + drafts[:i]``, ``speculative.py:127``) as spans into one id
    buffer that holds each sequence's context followed by its k drafts once:
    row (b, i) spans the context and the first i drafts.  Sequences whose
    penalty is off get empty spans.  Returns (ids int32, spans int64
    [2 * B * (k+1)]) or (None, None) when no row reads a history."""
    B, k = d.shape
    k1 = k + 1
    parts, spans = [], np.zeros((B, k1, 2), dtype=np.int64)
    start = 0
    for b in range(B):
        if params[b].repetition_penalty == 1.0:
            continue
        ctx = contexts[b]
        ids = _history_ids(ctx if ctx is not None else (), V)
        parts += [ids, d[b]]
        spans[b, :, 0] = start
        spans[b, :, 1] = start + ids.size + np.arange(k1)
        start += ids.size + k
    if not parts or start == 0:
        return None, None
    return np.concatenate(parts).astype(np.int32, copy=False), spans.reshape(-1)


def draft_buffer(B: int, k: int, V: int, *, ctx: _native.Context | None = None):
    """Device buffer [B, k, V] float64 for the draft distributions of one
    round (filled by :func:`draft_step`, read by :func:`verify_step`)."""
    c = ctx if ctx is not None else _native.default_context()
    return c.empty((B, k, V), np.float64)


def draft_step(logits, params, rngs, contexts, q_out, pos: int, *, ctx: _native.Context | None = None):
    """Draft position ``pos`` for B sequences (``speculative.py:117-120``):
    for row b, ``q_b = probs(logits[b], params_b, contexts[b])`` (contexts[b]
    is ``ctx + drafts`` so far) and ``x_b = draw(q_b, rngs[b])``.  Every row
    consumes one uniform, greedy rows included (``draw`` is called on the
    one-hot q, ``:120``).  q_b stays on the device, at ``q_out[b, pos]``
    (a :func:`draft_buffer`).  Returns the tokens, int64 [B]."""
    c = ctx if ctx is not None else _native.default_context()
    c.set_stream(None)
    x = _as_float_rows(logits)
    if x.ndim != 2:
        raise ValueError("logits must be [B, V]")
    B, V = x.shape
    Bq, k, Vq = q_out.shape
    if (Bq, Vq) != (B, V) or not 0 <= pos < k:
        raise ValueError(f"q_out {q_out.shape} does not hold position {pos} of a [{B}, k, {V}] round")
    params = _expand_params(params, B)
    u = np.array([rngs[b].random() for b in range(B)], dtype=np.float64)
    t, kk, p, r = _pack_params(params)
    hist_ids, hist_off = _pack_histories(contexts, params, B, V)
    parts = [t, kk, p, r, u] + ([hist_ids, hist_off] if hist_off is not None else [])
    d = c.stage_upload("dft_in", parts)
    hist = (d[5], d[6], 0) if hist_off is not None else None
    ids, q = _probs_rows(c, x, d[:5], hist, "dft")
    c.copy_rows(q_out.ptr + 8 * pos * V, 8 * k * V, q.ptr, 8 * V, 8 * V, B)
    return ids.download().astype(np.int64)


def verify_step(target_logits, q_rows, drafts, params, rngs, contexts, *, ctx: _native.Context | None = None):
    """The target side of one round for B sequences with k drafts each
    (``speculative.py:124-131``): ``p_rows[b, i] = probs(target_logits[b, i],
    params_b, contexts[b] + drafts[b][:i])`` for i <= k, then
    ``verify(p_rows[b], q_rows[b], drafts[b], rngs[b])`` (or, for k = 0,
    ``draw(p_rows[b, 0], rngs[b])``).  q_rows is [B, k, V] float64: the
    :func:`draft_buffer` the draft steps filled, or a host array.  Each
    Generator ends exactly where the reference leaves it.

    Returns (emitted: list of B token lists, n_acc int64 [B])."""
    c = ctx if ctx is not None else _native.default_context()
    c.set_stream(None)
    x = _as_float_rows(target_logits)
    if x.ndim != 3:
        raise ValueError("target_logits must be [B, k+1, V]")
    B, k1, V = x.shape
    k = k1 - 1
    d = _check_draft(np.asarray(drafts).reshape(B, k), V)
    params = _expand_params(params, B)
    if contexts is None:
        contexts = [()] * B
    if len(contexts) != B:
        raise ValueError(f"expected {B} contexts, got {len(contexts)}")
    # the draft distributions, [B, k, V] float64 on the device
    qd = None
    if k:
        if hasattr(q_rows, "ptr"):
            if tuple(q_rows.shape) != (B, k, V) or q_rows.dtype != np.float64:
                raise ValueError(f"q_rows must be a float64 [{B}, {k}, {V}] device buffer")
            qd = q_rows
        else:
            qd = c.scratch_upload("tgt_q", np.ascontiguousarray(np.asarray(q_rows, dtype=np.float64).reshape(B, k, V)))
    # per row: snapshot the Generator, draw k+1 uniforms (one call draws the
    # same values as k+1 calls of random()), replay what was used
    states = [rngs[b].bit_generator.state for b in range(B)]
    u = np.stack([rngs[b].random(k1) for b in range(B)]) if B else np.zeros((0, k1))
    accept_u = u[:, :k]
    draw_u = u[:, np.minimum(np.arange(k1) + 1, k)]
    # the target rows (b, i) share sequence b's parameters; their histories
    # are spans over each sequence's context and drafts
    t, kk, p, r = (np.repeat(a, k1) for a in _pack_params(params))
    hist_ids, spans = _round_histories(contexts, params, d, V)
    parts = [t, kk, p, r, np.zeros(B * k1), d, accept_u, draw_u]
    parts += [hist_ids, spans] if spans is not None else []
    dv = c.stage_upload("tgt_in", parts)
    hist = (dv[8], dv[9], _native.PLH_SAMPLE_HIST_SPANS) if spans is not None else None
    _, pr = _probs_rows(c, x.reshape(B * k1, V), dv[:5], hist, "tgt")
    d_tok = c.scratch("tgt_tok", (B, k1), np.int32)
    d_n = c.scratch("tgt_n", (B,), np.int32)
    c.verify(pr.ptr, qd.ptr if k else None, _native.PLH_F64, B, k, V, dv[5] if k else None,
             dv[6] if k else None, dv[7], True, d_tok.ptr, d_n.ptr)
    toks, n = d_tok.download(), d_n.download()
    emitted = []
    for b in range(B):
        s = int(n[b])
        rngs[b].bit_generator.state = states[b]
        rngs[b].random(s + 2 if s < k else k + 1)
        emitted.append([int(t) for t in toks[b, : s + 1]])
    return emitted, n.astype(np.int64)
