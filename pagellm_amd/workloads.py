"""Seeded synthetic workloads for the sampler and speculative verify.

Five workloads, each reproducible from fixed numpy seeds:

  char65    16 x 65 fp32 logits ~ N(0, 2^2), 64-token histories; rows 0-3
            greedy, rows 4-15 T=0.8, top_k=10, top_p=0.9, penalty 1.1
  zipf32k   64 x 32000 Zipf-shaped rows (logit = -1.1 ln rank + N(0, .5^2),
            ranks permuted per row), T=0.7, top_p=0.95, penalty 1.2 over
            512-token Zipf histories
  mixed128k 256 x 128256 fp32 ~ N(0, 3^2) plus 8 spikes of +10 per row; four
            groups of 64 rows: greedy | top_k 50 | top_p 0.9 |
            top_k 40 + top_p 0.95 + T 0.6 + penalty 1.1 (2048-token
            uniform histories)
  spec32k   speculative verify, 64 rows, k=4, V=32000
  zipf152k  1024 x 152064 Zipf (exponent 1.0, N(0, .3^2) noise), top_p 0.99,
            penalty 1.05 over 4096-token Zipf histories

Row r's uniform is the first draw of ``make_rng(r, 0)`` (the engine's
per-request Generator, seed = row index), taken only for non-greedy rows.
"""

from __future__ import annotations

import hashlib

import numpy as np

from .params import SamplingParams, make_rng


def _uniforms(params, seeds):
    u = np.zeros(len(params))
    for r, (p, s) in enumerate(zip(params, seeds)):
        if not p.greedy:
            u[r] = make_rng(s, 0).random()
    return u


def _zipf_rows(g, B, V, s, noise):
    """Per row: ranks 1..V in random order; logit = -s ln(rank) + N(0, noise^2).
    Also returns each row's inverse permutation (token id of rank r+1)."""
    logits = np.empty((B, V), dtype=np.float32)
    inv = np.empty((B, V), dtype=np.int64)
    for b in range(B):
        perm = g.permutation(V)
        rank = 1 + perm
        logits[b] = (-s * np.log(rank) + g.normal(0.0, noise, V)).astype(np.float32)
        inv[b, perm] = np.arange(V)
    return logits, inv


def _zipf_histories(g, inv, H, s):
    """H ids per row drawn with P(token) proportional to rank(token)^-s."""
    B, V = inv.shape
    w = np.arange(1, V + 1, dtype=np.float64) ** -s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    out = []
    for b in range(B):
        r = np.minimum(np.searchsorted(cdf, g.random(H), side="right"), V - 1)
        out.append(inv[b, r].astype(np.int64))
    return out


def char65():
    g = np.random.default_rng(1001)
    logits = g.normal(0.0, 2.0, (16, 65)).astype(np.float32)
    hist = g.integers(0, 65, (16, 64))
    params = [SamplingParams(temperature=0.0)] * 4 + [
        SamplingParams(temperature=0.8, top_k=10, top_p=0.9, repetition_penalty=1.1)
    ] * 12
    seeds = list(range(16))
    return dict(name="char65", logits=logits, params=params, contexts=[h for h in hist],
                seeds=seeds, uniforms=_uniforms(params, seeds))


def zipf32k(rows: int = 64):
    g = np.random.default_rng(1002)
    V = 32000
    logits, inv = _zipf_rows(g, rows, V, 1.1, 0.5)
    hist = _zipf_histories(g, inv, 512, 1.1)
    params = [SamplingParams(temperature=0.7, top_k=0, top_p=0.95, repetition_penalty=1.2)] * rows
    seeds = list(range(rows))
    return dict(name="zipf32k", logits=logits, params=params, contexts=hist, seeds=seeds,
                uniforms=_uniforms(params, seeds))


MIXED_GROUPS = (
    SamplingParams(temperature=0.0),
    SamplingParams(top_k=50),
    SamplingParams(top_p=0.9),
    SamplingParams(temperature=0.6, top_k=40, top_p=0.95, repetition_penalty=1.1),
)


def mixed128k(rows: int = 256, V: int = 128256):
    """The mixed-parameter batch (N(0, 3^2) logits plus 8 spikes of +10 a
    row, four parameter groups); V other than 128 256 gives the same recipe
    at another vocabulary size."""
    g = np.random.default_rng(1003)
    logits = g.normal(0.0, 3.0, (rows, V)).astype(np.float32)
    for b in range(rows):
        logits[b, g.choice(V, 8, replace=False)] += np.float32(10.0)
    hist = g.integers(0, V, (rows, 2048))
    q = rows // 4
    params = [MIXED_GROUPS[min(b // q, 3)] for b in range(rows)]
    seeds = list(range(rows))
    return dict(name="mixed128k", logits=logits, params=params, contexts=[h for h in hist],
                seeds=seeds, uniforms=_uniforms(params, seeds))


def zipf152k(rows: int = 1024):
    g = np.random.default_rng(1005)
    V = 152064
    logits, inv = _zipf_rows(g, rows, V, 1.0, 0.3)
    hist = _zipf_histories(g, inv, 4096, 1.0)
    params = [SamplingParams(temperature=1.0, top_k=0, top_p=0.99, repetition_penalty=1.05)] * rows
    seeds = list(range(rows))
    return dict(name="zipf152k", logits=logits, params=params, contexts=hist, seeds=seeds,
                uniforms=_uniforms(params, seeds))


def _softmax(x):
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def spec32k(rows: int = 64, k: int = 4, V: int = 32000):
    """Target logits ~ N(0, 2^2) [rows, k+1, V]; draft logits = target[:, :k]
    + N(0, .5^2); p and q their temperature-1 softmax (float64).  With
    default_rng(0): draft_u [rows,k] picks each draft token by inverse CDF of
    q, then accept_u [rows,k] and resample_u [rows]."""
    g = np.random.default_rng(1004)
    target = g.normal(0.0, 2.0, (rows, k + 1, V))
    draft = target[:, :k] + g.normal(0.0, 0.5, (rows, k, V))
    p = _softmax(target)
    q = _softmax(draft)
    g0 = np.random.default_rng(0)
    draft_u = g0.random((rows, k))
    accept_u = g0.random((rows, k))
    resample_u = g0.random(rows)
    c = np.cumsum(q, axis=-1)
    tokens = np.empty((rows, k), dtype=np.int64)
    for b in range(rows):
        for i in range(k):
            tokens[b, i] = min(np.searchsorted(c[b, i], draft_u[b, i] * c[b, i, -1], side="right"), V - 1)
    return dict(name="spec32k", p=p, q=q, draft=tokens, accept_u=accept_u, resample_u=resample_u)


WORKLOADS = {"char65": char65, "zipf32k": zipf32k, "mixed128k": mixed128k, "zipf152k": zipf152k}


def algorithmic_bytes(w) -> int:
    """HBM bytes one sampling pass must move: 4V per fp32 logit row, 4H per
    history id of rows whose penalty is active, and 48 B of per-row
    parameters, uniform, CSR offset and output id."""
    B, V = w["logits"].shape
    esize = w["logits"].dtype.itemsize
    h = sum(len(c) for c, p in zip(w["contexts"], w["params"]) if p.repetition_penalty != 1.0)
    return B * V * esize + 4 * h + 48 * B


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
