"""CPU oracle: a numpy restatement of pagellm's sampler and speculative verify.

TEST INFRASTRUCTURE ONLY.  This module gives the expected results for the HIP sampler in
``pagellm_amd`` and the timed CPU baseline in ``bench.py``; the product never
imports it.

It follows ``src/pagellm/engine/sampling.py:52-111`` and
``src/pagellm/engine/speculative.py:38-60`` of the reference operation by
operation (float64 promotion, strict ``>``/``<``/``>=``, stable descending
order, exclusive-mass top-p rule, ``searchsorted(side="right")``, the
``min(i, V-1)`` clamp), with one deliberate change of interface: randomness
is passed in as explicit uniforms (or any object with a ``random()`` method)
instead of a ``numpy.random.Generator``, so the GPU path and the oracle can be
fed the very same draws.  ``ScriptedRNG`` replays a list of uniforms through
the reference's ``rng.random()`` call sites, which is how the tests show that
the explicit-uniform form consumes randomness exactly as the reference does.

The arithmetic of the path lives in numpy (``np.unique``, ``np.partition``,
``np.exp``, ``ndarray.sum`` (pairwise), ``np.argsort(kind="stable")``,
``np.cumsum``, ``np.searchsorted``): the reference pins ``numpy>=1.24``
(``pyproject.toml:24``) without a lockfile; this oracle runs on numpy 2.2.x.
Every function here is pinned by ``tests/test_oracle.py`` against the
reference's own known-answer tests (``tests/unit/test_sampling.py``,
``tests/unit/test_speculative.py``, transcribed as data into
``tests/golden/reference_kats.json``), against a pure-Python brute force
written with different primitives (sorting, ``math.exp``, ``math.fsum``,
linear scans), and against closed forms and invariants chosen so that a
dropped term, a flipped comparison or a wrong index fails one of them.

The ``*_boundary_gap`` helpers measure how close a decision came to flipping;
parity tests use them to tell genuine mismatches from counted boundary cases.
"""

from __future__ import annotations

from typing import Iterable, Sequence

import numpy as np

# ------------------------------------------------------------------ helpers


class ScriptedRNG:
    """Stand-in for ``numpy.random.Generator`` whose ``random()`` returns
    pre-drawn values in order; ``consumed`` counts the calls."""

    def __init__(self, values: Iterable[float]):
        self._values = [float(v) for v in values]
        self.consumed = 0

    def random(self) -> float:
        if self.consumed >= len(self._values):
            raise IndexError("ScriptedRNG exhausted")
        v = self._values[self.consumed]
        self.consumed += 1
        return v


def _uniform(u) -> float:
    """Accept either a float or an object with ``random()``."""
    if hasattr(u, "random"):
        return u.random()
    return float(u)


# ------------------------------------------------------------- sampling.py


def apply_repetition_penalty(logits: np.ndarray, context, penalty: float) -> np.ndarray:
    """sampling.py:52-62.  Returns the input object itself when the penalty
    is disabled (``penalty == 1.0``) or the context is empty (``:56-57``),
    else a copy (``:58``) in which every *distinct* id of the context has
    ``x > 0 ? x / penalty : x * penalty`` applied once (``:59-61``)."""
    if penalty == 1.0 or len(context) == 0:
        return logits
    logits = logits.copy()
    seen = np.unique(np.asarray(context, dtype=np.int64))
    x = logits[seen]
    logits[seen] = np.where(x > 0, x / penalty, x * penalty)
    return logits


def _processed_logits(logits, params, context):
    """sampling.py:67-70: float64 promotion then the penalty."""
    return apply_repetition_penalty(
        np.asarray(logits, dtype=np.float64), context, params.repetition_penalty
    )


def probs(logits: np.ndarray, params, context=()) -> np.ndarray:
    """sampling.py:65-91, the processed next-token distribution (float64)."""
    x = _processed_logits(logits, params, context)
    V = x.shape[-1]
    if params.temperature == 0:  # sampling.py:71-74 (SamplingParams.greedy, :47-49)
        p = np.zeros(V)
        p[int(np.argmax(x))] = 1.0
        return p
    x = x / params.temperature  # :75
    if 0 < params.top_k < V:  # :76-78, ties with the k-th value are kept
        kth = np.partition(x, V - params.top_k)[V - params.top_k]
        x = np.where(x >= kth, x, -np.inf)
    x = x - x.max()  # :79-81
    p = np.exp(x)
    p /= p.sum()
    if params.top_p < 1.0:  # :82-90
        p = _top_p_filter(p, params.top_p)
    return p


def _top_p_filter(p: np.ndarray, top_p: float) -> np.ndarray:
    """sampling.py:83-90: stable descending order, keep while the mass
    *before* a token is below top_p, renormalise."""
    order = np.argsort(-p, kind="stable")
    cum = np.cumsum(p[order])
    keep = cum - p[order] < top_p
    mask = np.zeros(p.shape[-1], dtype=bool)
    mask[order[keep]] = True
    p = np.where(mask, p, 0.0)
    p /= p.sum()
    return p


def draw(p: np.ndarray, u) -> int:
    """sampling.py:94-98 with the uniform passed in (a float, or an object
    with ``random()``): inverse CDF in vocabulary order, ``side="right"``,
    clamped to ``V-1``."""
    c = np.cumsum(p)
    return int(min(np.searchsorted(c, _uniform(u) * c[-1], side="right"), len(p) - 1))


def sample(logits: np.ndarray, params, u, context=()) -> int:
    """sampling.py:101-107.  Greedy rows take no uniform (``u`` may be None)."""
    if params.temperature == 0:
        x = _processed_logits(logits, params, context)
        return int(np.argmax(x))
    return draw(probs(logits, params, context), u)


def sample_batch(logits: np.ndarray, params: Sequence, uniforms, contexts=None) -> np.ndarray:
    """Row-by-row loop over :func:`sample`, as ``llm_engine.py:238-254`` does.
    ``uniforms[b]`` is used only for non-greedy rows."""
    B = logits.shape[0]
    out = np.empty(B, dtype=np.int64)
    for b in range(B):
        ctx = () if contexts is None else contexts[b]
        out[b] = sample(logits[b], params[b], uniforms[b], ctx)
    return out


# ---------------------------------------------------------- speculative.py


def _verify_core(p_rows, q_rows, draft_tokens, next_accept, next_draw):
    out = []
    for i, x in enumerate(draft_tokens):
        p, q = p_rows[i], q_rows[i]
        if next_accept(i) < min(1.0, p[x] / q[x]):  # speculative.py:50
            out.append(x)
            continue
        resid = np.maximum(p - q, 0.0)  # :53-57
        s = resid.sum()
        out.append(draw(resid / s if s > 0 else p, next_draw(i)))
        return out, i
    k = len(draft_tokens)
    out.append(draw(p_rows[k], next_draw(k)))  # :59-60
    return out, k


def verify(p_rows, q_rows, draft_tokens, rng):
    """speculative.py:38-60.  ``rng`` is anything with ``random()``; it is
    called once per accept test and once for the final draw, in the
    reference's order."""
    with np.errstate(divide="ignore", invalid="ignore"):
        return _verify_core(
            p_rows, q_rows, draft_tokens, lambda i: rng.random(), lambda i: rng.random()
        )


def verify_explicit(p_rows, q_rows, draft_tokens, accept_u, draw_u):
    """verify with explicit uniforms: test i uses ``accept_u[i]``; the final
    draw (stop position s = first rejected index, or k) uses ``draw_u`` if it
    is a scalar, else ``draw_u[s]``."""
    scalar = np.ndim(draw_u) == 0
    with np.errstate(divide="ignore", invalid="ignore"):
        return _verify_core(
            p_rows,
            q_rows,
            draft_tokens,
            lambda i: float(accept_u[i]),
            lambda s: float(draw_u) if scalar else float(draw_u[s]),
        )


def verify_batch(p, q, draft, accept_u, resample_u):
    """Batched verify in the layout of the speculative benchmark workload:
    p [B,k+1,V], q [B,k,V], draft [B,k], accept_u [B,k], resample_u [B].
    Returns tokens [B,k+1] (padded with -1) and n_acc [B]."""
    B, k = draft.shape
    tokens = np.full((B, k + 1), -1, dtype=np.int64)
    n_acc = np.empty(B, dtype=np.int64)
    for b in range(B):
        out, n = verify_explicit(p[b], q[b], [int(t) for t in draft[b]], accept_u[b], resample_u[b])
        tokens[b, : len(out)] = out
        n_acc[b] = n
    return tokens, n_acc


# --------------------------------------------------------- boundary gauges


def top_p_boundary_gap(logits, params, context=()) -> float:
    """How far the top-p cut of ``probs`` is from flipping: the smaller of
    ``top_p - excl(last kept)`` and ``excl(first dropped) - top_p``, where
    ``excl`` is the reference's ``cum - p``.  Returns 0.0 when the last kept
    and first dropped tokens tie in probability without tying in logit (a
    tie created by ``exp`` rounding), and ``inf`` when top-p is inactive."""
    if params.temperature == 0 or params.top_p >= 1.0:
        return float("inf")
    x = _processed_logits(logits, params, context)
    V = x.shape[-1]
    x = x / params.temperature
    if 0 < params.top_k < V:
        kth = np.partition(x, V - params.top_k)[V - params.top_k]
        x = np.where(x >= kth, x, -np.inf)
    y = x
    x = x - x.max()
    p = np.exp(x)
    p /= p.sum()
    order = np.argsort(-p, kind="stable")
    cum = np.cumsum(p[order])
    excl = cum - p[order]
    keep = excl < params.top_p
    n = int(keep.sum())
    gap = float(params.top_p - excl[n - 1])
    if n < V:
        gap = min(gap, float(excl[n] - params.top_p))
        a, b = order[n - 1], order[n]
        if p[a] == p[b] and y[a] != y[b]:
            return 0.0
    return gap


def draw_boundary_gap(p: np.ndarray, u: float) -> float:
    """Distance, in units of the uniform, from ``u`` to the nearest CDF
    boundary of the draw ``draw(p, u)`` (``c_i / c[-1]``)."""
    c = np.cumsum(p)
    t = u * c[-1]
    i = int(np.searchsorted(c, t, side="right"))
    lo = c[i - 1] if i > 0 else 0.0
    hi = c[i] if i < len(c) else c[-1]
    return float(min(t - lo, hi - t) / c[-1])


def sample_boundary_gaps(logits, params, u, context=()):
    """(top-p gap, draw gap) for one row of :func:`sample`."""
    if params.temperature == 0:
        return float("inf"), float("inf")
    p = probs(logits, params, context)
    return top_p_boundary_gap(logits, params, context), draw_boundary_gap(p, u)


def verify_boundary_gap(p_rows, q_rows, draft_tokens, accept_u, draw_u) -> float:
    """Smallest distance of any accept uniform used to its threshold
    ``min(1, p/q)``, and of the final draw's uniform to a CDF boundary."""
    gap = float("inf")
    scalar = np.ndim(draw_u) == 0
    with np.errstate(divide="ignore", invalid="ignore"):
        for i, x in enumerate(draft_tokens):
            p, q = p_rows[i], q_rows[i]
            thr = min(1.0, p[x] / q[x])
            u = float(accept_u[i])
            gap = min(gap, abs(u - thr))
            if u < thr:
                continue
            resid = np.maximum(p - q, 0.0)
            s = resid.sum()
            dist = resid / s if s > 0 else p
            du = float(draw_u) if scalar else float(draw_u[i])
            return min(gap, draw_boundary_gap(dist, du))
        k = len(draft_tokens)
        du = float(draw_u) if scalar else float(draw_u[k])
        return min(gap, draw_boundary_gap(p_rows[k], du))
