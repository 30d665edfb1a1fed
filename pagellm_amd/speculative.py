"""Drop-in replacement for the accept/resample step of
``pagellm.engine.speculative`` (``verify``, ``speculative.py:38-60``),
computed on MI355X, plus the batched :func:`verify_batch`.

``verify`` keeps the reference's randomness exactly: the reference calls
``rng.random()`` once per accept test, stopping at the first rejection, then
once for the emitted token (residual or bonus).  The host cannot know the
stop position in advance, so it snapshots the Generator, draws k+1 uniforms,
lets the kernel walk the tests, then restores the snapshot and replays
exactly the number of draws the reference would have made.
"""

from __future__ import annotations

import numpy as np

from . import _native
from .sampling import _as_float_rows

__all__ = ["verify", "verify_batch"]


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
