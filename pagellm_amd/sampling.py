"""Drop-in replacement for ``pagellm.engine.sampling`` computed on MI355X.

Same names, signatures, argument meaning and error behaviour as
``src/pagellm/engine/sampling.py`` (``SamplingParams``,
``apply_repetition_penalty``, ``probs``, ``draw``, ``sample``, ``make_rng``),
plus :func:`sample_batch`, the batched form the engine's per-sequence loop
(``llm_engine.py:238-254``) maps onto.

Randomness stays on the host: each non-greedy sample consumes exactly one
``rng.random()`` from the sequence's own Generator, in row order, exactly as
the reference does (``sampling.py:98``); greedy rows consume nothing
(``:102-106``).  The uniforms, logits, histories and per-row parameters go to
HBM; only token ids (and, for :func:`probs`, the distribution) come back.
There is no CPU fallback: without the HIP library or a GPU every function
here raises.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np

from . import _native
from .params import SamplingParams, make_rng

__all__ = [
    "SamplingParams",
    "abi_params",
    "apply_repetition_penalty",
    "draw",
    "draw_batch",
    "make_rng",
    "probs",
    "sample",
    "sample_batch",
]


def _ctx(ctx):
    return ctx if ctx is not None else _native.default_context()


def _as_float_rows(x) -> np.ndarray:
    """float32 stays float32 (widened exactly on the device); any other type
    is promoted to float64 on the host, as ``np.asarray(logits, float64)``."""
    a = np.asarray(x)
    if a.dtype != np.float32 and a.dtype != np.float64:
        a = a.astype(np.float64)
    return np.ascontiguousarray(a)


def _history_ids(context, V: int) -> np.ndarray:
    """Token ids of one history as int32 in [0, V): numpy indexing semantics
    (negative ids wrap, ids outside [-V, V) raise IndexError)."""
    ids = np.asarray(context, dtype=np.int64).reshape(-1)
    if ids.size:
        lo, hi = int(ids.min()), int(ids.max())
        if hi >= V or lo < -V:
            bad = hi if hi >= V else lo
            raise IndexError(f"index {bad} is out of bounds for axis 0 with size {V}")
        if lo < 0:
            ids = np.where(ids < 0, ids + V, ids)
    return ids.astype(np.int32)


MAX_PENALTY_VOCAB = 262144  # vocabulary size up to which penalised rows are supported


def _pack_histories(contexts, params: Sequence[SamplingParams], B: int, V: int):
    """CSR (ids, offsets) of the histories of rows whose penalty is active,
    or (None, None) when no row needs one (nothing is uploaded)."""
    if contexts is None:
        return None, None
    if len(contexts) != B:
        raise ValueError(f"expected {B} contexts, got {len(contexts)}")
    parts, off = [], np.zeros(B + 1, dtype=np.int64)
    for b in range(B):
        ctx = contexts[b]
        n = 0
        if ctx is not None and params[b].repetition_penalty != 1.0 and len(ctx) > 0:
            ids = _history_ids(ctx, V)
            parts.append(ids)
            n = ids.size
        off[b + 1] = off[b] + n
    if off[-1] == 0:
        return None, None
    if V > MAX_PENALTY_VOCAB:
        raise NotImplementedError(
            f"repetition penalty over a token history needs V <= {MAX_PENALTY_VOCAB} here (got V = {V}): "
            "the kernels mark a row's penalised tokens in an on-chip bitmap of that many bits; "
            "the reference (sampling.py:52-62) has no such limit"
        )
    return np.concatenate(parts), off


def _pack_params(params: Sequence[SamplingParams]):
    """The per-row parameter arrays (float64 T, int32 top_k clamped to
    2^31 - 1, float64 top_p and penalty).  A batch usually holds few
    distinct SamplingParams objects (one per request); each distinct object
    is then read once and the rows index into its values."""
    B = len(params)
    ids = list(map(id, params))
    first = dict.fromkeys(ids)
    if 4 * len(first) <= B:
        by_id = dict(zip(ids, params))
        objs = [by_id[key] for key in first]
        pos = {key: i for i, key in enumerate(first)}
        idx = np.fromiter(map(pos.__getitem__, ids), dtype=np.intp, count=B)
    else:
        objs, idx = params, None
    t = np.array([sp.temperature for sp in objs], dtype=np.float64)
    k = np.array([min(int(sp.top_k), 2**31 - 1) for sp in objs], dtype=np.int32)
    p = np.array([sp.top_p for sp in objs], dtype=np.float64)
    r = np.array([sp.repetition_penalty for sp in objs], dtype=np.float64)
    if idx is None:
        return t, k, p, r
    return t[idx], k[idx], p[idx], r[idx]


def abi_params(params: Sequence) -> dict[str, np.ndarray]:
    """The per-row parameter arrays ``plh_sample`` reads for one batch:
    ``temperature``, ``top_p``, ``repetition_penalty`` float64 [B] and
    ``top_k`` int32 [B] (clamped to 2^31 - 1, which disables the mask as any
    top_k >= V does).

    Each entry is a ``SamplingParams``, or a parsed request that carries one
    in ``.params`` (the reference's ``CompletionRequest``,
    ``src/pagellm/serving/protocol.py:75-79``, as its
    ``parse_completion_request`` returns it, ``:82-108``).  A JSON number
    parses to a Python float, an IEEE double, so every value reaches the
    kernels bit for bit.  This is the packing every sampler entry point uses.
    """
    rows = [r if hasattr(r, "temperature") else r.params for r in params]
    t, k, p, r = _pack_params(rows)
    return {"temperature": t, "top_k": k, "top_p": p, "repetition_penalty": r}


def _expand_params(params, B: int) -> list[SamplingParams]:
    if isinstance(params, SamplingParams) or hasattr(params, "temperature"):
        return [params] * B
    params = list(params)
    if len(params) != B:
        raise ValueError(f"expected {B} SamplingParams, got {len(params)}")
    return params


NUCLEUS_TOP_P = 0.98  # rows with no top-k from this top_p up may take the nucleus path


def _nucleus_hint(t: np.ndarray, k: np.ndarray, p: np.ndarray, V: int) -> int:
    """``PLH_SAMPLE_NUCLEUS`` when some row is non-greedy with no top-k and
    ``NUCLEUS_TOP_P <= top_p < 1``: such nuclei hold most of the vocabulary,
    which the multi-pass nucleus kernels handle faster than the per-row general
    pipeline.  The sampled ids do not depend on the hint."""
    rows = (t != 0) & ((k <= 0) | (k >= V)) & (p >= NUCLEUS_TOP_P) & (p < 1.0)
    if not bool(rows.any()):
        return 0
    # every row one of them: no merge launch (PLH_SAMPLE_NUCLEUS_ONLY)
    return _native.PLH_SAMPLE_NUCLEUS | (_native.PLH_SAMPLE_NUCLEUS_ONLY if bool(rows.all()) else 0)


def _draw_uniforms(params, rngs, B: int) -> np.ndarray:
    """One ``rng.random()`` per non-greedy row, in row order."""
    u = np.zeros(B, dtype=np.float64)
    for b in range(B):
        if not params[b].temperature == 0:
            rng = rngs[b] if rngs is not None else None
            if rng is None:
                raise ValueError(f"row {b} is not greedy and needs an rng")
            u[b] = rng.random()
    return u


def _is_torch_cuda(x) -> bool:
    t = type(x)
    return t.__module__.startswith("torch") and getattr(x, "is_cuda", False)


def sample_batch(
    logits,
    params,
    rngs: Sequence | None = None,
    contexts: Sequence | None = None,
    *,
    uniforms=None,
    ctx: _native.Context | None = None,
    rowwise: bool = False,
) -> np.ndarray:
    """Batched :func:`sample`: one token id per row of ``logits [B, V]``.

    ``params`` is one SamplingParams or one per row; ``rngs[b]`` is row b's
    Generator (unused, may be None, for greedy rows); ``contexts[b]`` is row
    b's token history (prompt + outputs).  ``uniforms`` may replace ``rngs``
    (pre-drawn, one per row).  ``logits`` may be a numpy array or a torch
    CUDA tensor (then read in place on torch's current stream).
    Returns int64 ids [B].
    """
    c = _ctx(ctx)
    keep = []
    if _is_torch_cuda(logits):
        import torch

        if logits.dim() != 2 or logits.stride(1) != 1:
            raise ValueError("logits must be a 2-D tensor with unit stride in the vocabulary dimension")
        if logits.dtype not in (torch.float32, torch.float64):
            raise TypeError("torch logits must be float32 or float64")
        B, V = int(logits.shape[0]), int(logits.shape[1])
        ptr, ld = logits.data_ptr(), int(logits.stride(0))
        code = _native.PLH_F64 if logits.dtype == torch.float64 else _native.PLH_F32
        c.set_stream(torch.cuda.current_stream(logits.device).cuda_stream)
    else:
        host = _as_float_rows(logits)
        if host.ndim != 2:
            raise ValueError("logits must be [B, V]")
        B, V = host.shape
        if B and V == 0:
            raise ValueError("empty vocabulary")
        dev, ld = c.upload_rows("logits", host)
        ptr, code = dev.ptr, _native.dtype_code(host.dtype)
        c.set_stream(None)
    if B == 0:
        return np.zeros(0, dtype=np.int64)
    params = _expand_params(params, B)
    u = np.asarray(uniforms, dtype=np.float64).reshape(B) if uniforms is not None else _draw_uniforms(params, rngs, B)
    t, k, p, r = _pack_params(params)
    hist_ids, hist_off = _pack_histories(contexts, params, B, V)
    # the per-row arrays go over in one queued copy, on the stream the
    # kernels run on (the download below waits for both)
    parts = [t, p, r, u, k] + ([hist_off, hist_ids] if hist_off is not None else [])
    d = c.stage_upload("sample_in", parts)
    d_off, d_ids = (d[5], d[6]) if hist_off is not None else (None, None)
    out = c.scratch("out_ids", (B,), np.int32)
    c.sample(
        ptr, code, ld, B, V, d_ids, d_off, d[0], d[4], d[1], d[2], d[3], out.ptr, None,
        _native.PLH_SAMPLE_ROWWISE if rowwise else _nucleus_hint(t, k, p, V),
    )
    del keep
    return out.download().astype(np.int64)


def apply_repetition_penalty(logits: np.ndarray, context, penalty: float) -> np.ndarray:
    """``sampling.py:52-62``: returns ``logits`` itself when the penalty is
    disabled or the context is empty, else a penalised copy (same dtype)."""
    if penalty == 1.0 or len(context) == 0:
        return logits
    x = _as_float_rows(logits)
    if x.ndim != 1:
        raise ValueError("logits must be 1-D")
    V = x.shape[0]
    ids = _history_ids(context, V)
    c = _ctx(None)
    c.set_stream(None)
    d_x = c.scratch_upload("pen_x", x[None, :])
    d_o = c.scratch("pen_out", (1, V), x.dtype)
    d_ids = c.scratch_upload("pen_ids", ids)
    d_off = c.scratch_upload("pen_off", np.array([0, ids.size], dtype=np.int64))
    d_r = c.scratch_upload("pen_r", np.array([penalty], dtype=np.float64))
    c.penalize(d_x.ptr, _native.dtype_code(x.dtype), V, 1, V, d_ids.ptr, d_off.ptr, d_r.ptr, d_o.ptr, V)
    return d_o.download()[0]


def probs(logits: np.ndarray, params: SamplingParams, context=()) -> np.ndarray:
    """``sampling.py:65-91``: the processed next-token distribution (float64)."""
    x = _as_float_rows(logits)
    if x.ndim != 1 or x.shape[0] == 0:
        raise ValueError("logits must be a non-empty 1-D array")
    V = x.shape[0]
    c = _ctx(None)
    c.set_stream(None)
    hist_ids, hist_off = _pack_histories([context], [params], 1, V)
    t, k, p, r = _pack_params([params])
    d_x = c.scratch_upload("probs_x", x[None, :])
    d_t = c.scratch_upload("probs_t", t)
    d_k = c.scratch_upload("probs_k", k)
    d_p = c.scratch_upload("probs_p", p)
    d_r = c.scratch_upload("probs_r", r)
    d_u = c.scratch_upload("probs_u", np.zeros(1))
    d_ids = d_off = None
    if hist_off is not None:
        d_ids = c.scratch_upload("probs_ids", hist_ids)
        d_off = c.scratch_upload("probs_off", hist_off)
    d_out = c.scratch("probs_id", (1,), np.int32)
    d_pr = c.scratch("probs_out", (1, V), np.float64)
    c.sample(
        d_x.ptr, _native.dtype_code(x.dtype), V, 1, V,
        d_ids.ptr if d_ids is not None else None,
        d_off.ptr if d_off is not None else None,
        d_t.ptr, d_k.ptr, d_p.ptr, d_r.ptr, d_u.ptr, d_out.ptr, d_pr.ptr, _native.PLH_SAMPLE_ROWWISE,
    )
    return d_pr.download()[0]


def draw(p: np.ndarray, rng: np.random.Generator) -> int:
    """``sampling.py:94-98``: inverse-CDF draw, one ``rng.random()``."""
    x = _as_float_rows(p)
    if x.ndim != 1 or x.shape[0] == 0:
        raise ValueError("p must be a non-empty 1-D array")
    u = rng.random()
    c = _ctx(None)
    c.set_stream(None)
    V = x.shape[0]
    d_p = c.scratch_upload("draw_p", x[None, :])
    d_u = c.scratch_upload("draw_u", np.array([u], dtype=np.float64))
    d_o = c.scratch("draw_out", (1,), np.int32)
    c.draw(d_p.ptr, _native.dtype_code(x.dtype), V, 1, V, d_u.ptr, d_o.ptr)
    return int(d_o.download()[0])


def draw_batch(p, uniforms, *, ctx: _native.Context | None = None) -> np.ndarray:
    """Batched :func:`draw` with explicit uniforms: row b of ``p [B, V]`` is
    drawn at ``uniforms[b]`` (``sampling.py:94-98``: the first index whose
    running mass exceeds ``u * total``, clamped to V - 1).  A float32 ``p`` is
    widened exactly and drawn in float64 arithmetic (the reference's
    ``probs()`` always hands ``draw`` float64 rows).  Returns int64 ids [B]."""
    x = _as_float_rows(p)
    if x.ndim != 2 or x.shape[1] == 0:
        raise ValueError("p must be a 2-D array with at least one column")
    u = np.ascontiguousarray(uniforms, dtype=np.float64).reshape(-1)
    B, V = x.shape
    if u.shape[0] != B:
        raise ValueError(f"expected {B} uniforms, got {u.shape[0]}")
    if B == 0:
        return np.zeros(0, dtype=np.int64)
    c = _ctx(ctx)
    c.set_stream(None)
    d_p = c.scratch_upload("drawb_p", x)
    d_u = c.scratch_upload("drawb_u", u)
    d_o = c.scratch("drawb_out", (B,), np.int32)
    c.draw(d_p.ptr, _native.dtype_code(x.dtype), V, B, V, d_u.ptr, d_o.ptr)
    return d_o.download().astype(np.int64)


def sample(logits: np.ndarray, params: SamplingParams, rng: np.random.Generator, context=()) -> int:
    """``sampling.py:101-107``: greedy consumes no randomness (``rng`` may be
    None); otherwise exactly one ``rng.random()``."""
    x = _as_float_rows(logits)
    if x.ndim != 1 or x.shape[0] == 0:
        raise ValueError("logits must be a non-empty 1-D array")
    return int(sample_batch(x[None, :], [params], [rng], [context])[0])
