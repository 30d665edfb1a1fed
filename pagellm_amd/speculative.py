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
from .sampling import _as_float_rows, _expand_params, _pack_histories, _pack_params

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


def verify_batch(p, q, draft, accept_u, resample_u, *, ctx: _native.Context | None = None):
    """Batched verify with explicit uniforms: test i of row b uses
    ``accept_u[b, i]``; the emitted (residual or bonus) token of row b uses
    ``resample_u[b]``.  p [B,k+1,V], q [B,k,V], draft [B,k].
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
    a = np.ascontiguousarray(accept_u, dtype=np.float64).reshape(B, k)
    w = np.ascontiguousarray(resample_u, dtype=np.float64).reshape(B)
    toks, n = _run(c, p, q, d, a, w, False)
    return toks.astype(np.int64), n.astype(np.int64)


def _probs_rows(c, x: np.ndarray, params, contexts, uniforms, tag: str):
    """plh_sample over the rows of x [N, V] with the processed distributions
    exported: returns (ids int32 [N] on the host, probs float64 [N, V] on the
    device)."""
    N, V = x.shape
    t, k, p, r = _pack_params(params)
    hist_ids, hist_off = _pack_histories(contexts, params, N, V)
    d_x = c.scratch_upload(f"{tag}_x", x)
    d_t = c.scratch_upload(f"{tag}_t", t)
    d_k = c.scratch_upload(f"{tag}_k", k)
    d_p = c.scratch_upload(f"{tag}_p", p)
    d_r = c.scratch_upload(f"{tag}_r", r)
    d_u = c.scratch_upload(f"{tag}_u", np.ascontiguousarray(uniforms, dtype=np.float64))
    d_ids = d_off = None
    if hist_off is not None:
        d_ids = c.scratch_upload(f"{tag}_hid", hist_ids)
        d_off = c.scratch_upload(f"{tag}_hoff", hist_off)
    out = c.scratch(f"{tag}_out", (N,), np.int32)
    probs = c.scratch(f"{tag}_probs", (N, V), np.float64)
    c.sample(d_x.ptr, _native.dtype_code(x.dtype), V, N, V, d_ids.ptr if d_ids is not None else None,
             d_off.ptr if d_off is not None else None, d_t.ptr, d_k.ptr, d_p.ptr, d_r.ptr, d_u.ptr, out.ptr,
             probs.ptr, 0)
    return out.download(), probs


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
    ids, q = _probs_rows(c, x, params, contexts, u, "dft")
    c.copy_rows(q_out.ptr + 8 * pos * V, 8 * k * V, q.ptr, 8 * V, 8 * V, B)
    return ids.astype(np.int64)


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
    rows_params = [params[b] for b in range(B) for _ in range(k1)]
    rows_ctx = [list(contexts[b]) + [int(t) for t in d[b, :i]] for b in range(B) for i in range(k1)]
    _, p = _probs_rows(c, x.reshape(B * k1, V), rows_params, rows_ctx, np.zeros(B * k1), "tgt")
    # the draft distributions, [B, k, V] float64 on the device
    qd = None
    if k:
        if hasattr(q_rows, "ptr"):
            if tuple(q_rows.shape) != (B, k, V) or q_rows.dtype != np.float64:
                raise ValueError(f"q_rows must be a float64 [{B}, {k}, {V}] device buffer")
            qd = q_rows
        else:
            qd = c.scratch_upload("tgt_q", np.ascontiguousarray(np.asarray(q_rows, dtype=np.float64).reshape(B, k, V)))
    # per row: snapshot the Generator, draw k+1 uniforms, replay what was used
    states = [rngs[b].bit_generator.state for b in range(B)]
    u = np.array([[rngs[b].random() for _ in range(k1)] for b in range(B)], dtype=np.float64)
    accept_u = np.ascontiguousarray(u[:, :k])
    draw_u = np.ascontiguousarray(np.stack([u[:, min(s + 1, k)] for s in range(k1)], axis=1))
    d_d = c.scratch_upload("tgt_d", d) if k else None
    d_a = c.scratch_upload("tgt_a", accept_u) if k else None
    d_w = c.scratch_upload("tgt_w", draw_u)
    d_tok = c.scratch("tgt_tok", (B, k1), np.int32)
    d_n = c.scratch("tgt_n", (B,), np.int32)
    c.verify(p.ptr, qd.ptr if k else None, _native.PLH_F64, B, k, V, d_d.ptr if k else None,
             d_a.ptr if k else None, d_w.ptr, True, d_tok.ptr, d_n.ptr)
    toks, n = d_tok.download(), d_n.download()
    emitted = []
    for b in range(B):
        s = int(n[b])
        rngs[b].bit_generator.state = states[b]
        for _ in range(s + 2 if s < k else k + 1):
            rngs[b].random()
        emitted.append([int(t) for t in toks[b, : s + 1]])
    return emitted, n.astype(np.int64)
