"""Batched speculative rounds (draft_step + verify_step) against the
reference's single-sequence loop restated with the oracle
(SpeculativeDecoder.generate, speculative.py:113-131): draft q = probs(...)
and x = draw(q, rng) per position with history ctx + drafts (:117-120); the
target p_rows with per-position histories ctx + drafts[:i] (:127); verify
(:129) or, for k = 0, draw(p_rows[0], rng) (:131).  Same logits, same
Generators: the emitted tokens, accept counts and Generator states match."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from pagellm_amd.params import SamplingParams, make_rng
from pagellm_amd.speculative import draft_buffer, draft_step, verify_step

pytestmark = pytest.mark.gpu

V = 2000
PARAMS = [
    SamplingParams(temperature=0.0, seed=1),
    SamplingParams(temperature=1.0, seed=2),
    SamplingParams(temperature=0.8, top_k=30, seed=3),
    SamplingParams(temperature=1.0, top_p=0.9, repetition_penalty=1.2, seed=4),
    SamplingParams(temperature=0.7, top_k=50, top_p=0.95, repetition_penalty=1.1, seed=5),
]


def _target(b, ctx):
    g = np.random.default_rng([101, b, len(ctx), int(sum(ctx)) % 100003])
    x = g.normal(0.0, 1.5, V)
    x[g.integers(0, V, 3)] += 4.0
    return x.astype(np.float32)


def _draft(b, ctx):
    g = np.random.default_rng([202, b, len(ctx), int(sum(ctx)) % 100003])
    return (_target(b, ctx) + g.normal(0.0, 0.4, V)).astype(np.float32)


def _reference_round(b, ctx, prm, rng, k):
    drafts, q_rows = [], []
    for _ in range(k):
        full = ctx + drafts
        q = oracle.probs(_draft(b, full), prm, full)
        drafts.append(int(oracle.draw(q, rng.random())))
        q_rows.append(q)
    p_rows = np.stack([oracle.probs(_target(b, ctx + drafts[:i]), prm, ctx + drafts[:i]) for i in range(k + 1)])
    if k:
        emitted, acc = oracle.verify(p_rows, np.stack(q_rows), drafts, rng)
    else:
        emitted, acc = [int(oracle.draw(p_rows[0], rng.random()))], 0
    return [int(t) for t in emitted], int(acc)


@pytest.mark.parametrize("k", [3, 0])
def test_batched_rounds_match_the_reference_loop(k):
    B = len(PARAMS)
    g = np.random.default_rng(5)
    prompts = [[int(t) for t in g.integers(0, V, 4 + b)] for b in range(B)]
    ref_ctx = [list(p) for p in prompts]
    got_ctx = [list(p) for p in prompts]
    ref_rng = [make_rng(p.seed, 0) for p in PARAMS]
    got_rng = [make_rng(p.seed, 0) for p in PARAMS]
    for rnd in range(3):
        ref = [_reference_round(b, ref_ctx[b], PARAMS[b], ref_rng[b], k) for b in range(B)]
        drafts = [[] for _ in range(B)]
        q_buf = draft_buffer(B, k, V) if k else None
        for i in range(k):
            full = [got_ctx[b] + drafts[b] for b in range(B)]
            ids = draft_step(np.stack([_draft(b, full[b]) for b in range(B)]), PARAMS, got_rng, full, q_buf, i)
            for b in range(B):
                drafts[b].append(int(ids[b]))
        tl = np.stack([np.stack([_target(b, got_ctx[b] + drafts[b][:i]) for i in range(k + 1)]) for b in range(B)])
        emitted, n_acc = verify_step(tl, q_buf, np.asarray(drafts, dtype=np.int64).reshape(B, k), PARAMS, got_rng,
                                     got_ctx)
        for b in range(B):
            assert (emitted[b], int(n_acc[b])) == ref[b], (rnd, b, emitted[b], int(n_acc[b]), ref[b])
            ref_ctx[b] += ref[b][0]
            got_ctx[b] += emitted[b]
    for b in range(B):
        assert got_rng[b].random() == ref_rng[b].random(), b
