"""The engine adapter (BatchSampler over DeviceHistories) against the
reference's per-sequence loop, restated with the oracle: llm_engine.py:238-254
calls sample(logits, params, seq.rng, seq.tokens) per finished sequence and
appends the token (:283-284); forks (n > 1, :259-278) copy the parent's tokens
and get Generators make_rng(seed, i).  Same logits, same Generators: the token
streams and the device-resident histories must match."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from pagellm_amd.engine import BatchSampler, DeviceHistories
from pagellm_amd.params import SamplingParams, make_rng

pytestmark = pytest.mark.gpu

V = 3000
REQUESTS = [  # (params, prompt length)
    (SamplingParams(temperature=0.0, seed=1), 5),
    (SamplingParams(temperature=0.0, repetition_penalty=1.3, seed=2), 9),
    (SamplingParams(temperature=0.8, top_k=20, seed=3, n=3), 7),
    (SamplingParams(temperature=1.0, top_p=0.9, repetition_penalty=1.2, seed=4, n=2), 12),
    (SamplingParams(temperature=0.6, top_k=40, top_p=0.95, repetition_penalty=1.1, seed=5), 3),
    (SamplingParams(temperature=1.0, seed=6), 1),
]


def _row(key, step):
    g = np.random.default_rng([7919, key[0], key[1], step])
    x = g.normal(0.0, 2.0, V).astype(np.float32)
    x[g.integers(0, V, 4)] += 6.0
    return x


def _run(steps, sampler=None, hist=None):
    """Reference-style loop; with `sampler`, every step is one batched call."""
    g = np.random.default_rng(11)
    seqs = {}  # key -> dict(tokens, rng, params)
    order = []
    for r, (prm, plen) in enumerate(REQUESTS):
        key = (r, 0)
        seqs[key] = dict(tokens=[int(t) for t in g.integers(0, V, plen)], rng=make_rng(prm.seed, 0), params=prm,
                         parent_row=None)
        order.append(key)
        if hist is not None:
            hist.add(key, seqs[key]["tokens"])
    streams = {}
    for step in range(steps):
        keys, rows = [], []
        for key in list(order):
            group = [key]
            prm = seqs[key]["params"]
            if step == 0 and prm.n > 1:  # the fork, before the parent's token is appended
                for i in range(1, prm.n):
                    kid = (key[0], i)
                    seqs[kid] = dict(tokens=list(seqs[key]["tokens"]), rng=make_rng(prm.seed, i), params=prm)
                    order.append(kid)
                    if hist is not None:
                        hist.add(kid, seqs[kid]["tokens"])
                    group.append(kid)
            row = _row(key, step)  # children share the parent's row this step
            for k in group:
                keys.append(k)
                rows.append(row if step == 0 else _row(k, step))
        if sampler is None:
            for k, x in zip(keys, rows):
                s = seqs[k]
                u = None if s["params"].greedy else s["rng"].random()
                tok = oracle.sample(x, s["params"], u, s["tokens"])
                s["tokens"].append(int(tok))
                streams.setdefault(k, []).append(int(tok))
        else:
            ids = sampler.sample(np.stack(rows), [seqs[k]["params"] for k in keys], [seqs[k]["rng"] for k in keys],
                                 keys)
            for k, tok in zip(keys, ids):
                seqs[k]["tokens"].append(int(tok))
                streams.setdefault(k, []).append(int(tok))
    return streams, seqs


def test_engine_loop_matches_per_sequence_sampling():
    ref, ref_seqs = _run(6)
    hist = DeviceHistories(V, max_seqs=16, max_len=64)
    got, got_seqs = _run(6, BatchSampler(hist), hist)
    assert got.keys() == ref.keys()
    for k in ref:
        assert got[k] == ref[k], (k, got[k], ref[k])
        # the device history is the host token list, grown one id per step
        assert np.array_equal(hist.download(k), np.asarray(got_seqs[k]["tokens"], dtype=np.int32)), k
        # every Generator advanced exactly as in the per-sequence loop
        assert got_seqs[k]["rng"].random() == ref_seqs[k]["rng"].random(), k


def test_history_slots_are_reused_and_bounded():
    hist = DeviceHistories(V, max_seqs=2, max_len=4)
    hist.add("a", [1, 2, 3])
    hist.add("b", [])
    with pytest.raises(RuntimeError):
        hist.add("c", [5])
    hist.remove("a")
    hist.add("c", [7, 8])
    assert list(hist.download("c")) == [7, 8]
    sampler = BatchSampler(hist)
    x = np.zeros((2, V), dtype=np.float32)
    x[0, 11] = 5.0
    x[1, 22] = 5.0
    ids = sampler.sample(x, SamplingParams(temperature=0.0), None, ["c", "b"])
    assert list(ids) == [11, 22]
    assert list(hist.download("c")) == [7, 8, 11] and list(hist.download("b")) == [22]
    hist.remove("b")
    hist.add("d", [1, 2, 3, 4])
    with pytest.raises(RuntimeError):  # a full history has no room for the next id
        sampler.sample(x[:1], SamplingParams(temperature=0.0), None, ["d"])
