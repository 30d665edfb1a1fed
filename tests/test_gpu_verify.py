"""GPU parity of speculative verify against the CPU oracle (needs an MI355X):
the reference's statistical law tests, exact replay of the Generator
consumption, and the spec32k workload."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle.sampler import verify_boundary_gap
from pagellm_amd import workloads
from parity import BAND, DRAW_GAP
from pagellm_amd.speculative import verify, verify_batch

pytestmark = pytest.mark.gpu


def _dist(rng, V, sharp=1.0):
    x = np.exp(rng.standard_normal(V) * sharp)
    return x / x.sum()


@pytest.mark.parametrize("k", [1, 2, 3])
def test_kat_verify_law(kats, k):
    """The reference's law test (``test_speculative.py:14-39``) at its full
    40 000 trials, all trials in one batched verify: the first emitted token
    follows p[0] and, after an acceptance, the second follows p[1]."""
    c = kats["verify_law"]
    rng = np.random.default_rng(k)
    V = c["V"]
    p = np.stack([_dist(rng, V, c["sharp"]) for _ in range(k + 1)])
    q = np.stack([_dist(rng, V, c["sharp"]) for _ in range(k)])
    trials = c["trials"]
    cq = np.cumsum(q, axis=1)
    xs = np.stack([np.minimum(np.searchsorted(cq[i], rng.random(trials) * cq[i, -1], side="right"), V - 1)
                   for i in range(k)], axis=1)
    au = rng.random((trials, k))
    ru = rng.random(trials)
    toks, n = verify_batch(np.broadcast_to(p, (trials, k + 1, V)), np.broadcast_to(q, (trials, k, V)), xs, au, ru)
    first = np.bincount(toks[:, 0], minlength=V)
    assert 0.5 * np.abs(first / trials - p[0]).sum() < c["tv_first"]
    if k >= 2:
        two = n >= 1
        second = np.bincount(toks[two, 1], minlength=V)
        assert 0.5 * np.abs(second / two.sum() - p[1]).sum() < c["tv_conditional"]
    rt, rn = oracle.verify_batch(p[None].repeat(256, 0), q[None].repeat(256, 0), xs[:256], au[:256], ru[:256])
    assert np.array_equal(rn, n[:256]) and np.array_equal(rt, toks[:256])


def test_kat_verify_identical(kats):
    c = kats["verify_identical"]
    rng = np.random.default_rng(c["rng_seed"])
    p = np.stack([_dist(rng, c["V"]) for _ in range(c["rows"])])
    for _ in range(c["trials"]):
        xs = [oracle.draw(p[i], rng) for i in range(c["k"])]
        out, acc = verify(p, p[: c["k"]], xs, rng)
        assert acc == c["k"] and out[: c["k"]] == xs and len(out) == c["k"] + 1


def test_verify_replays_generator_exactly():
    """Same outputs as the oracle fed by an identical Generator, and both
    Generators end in the same state (same number of draws)."""
    g = np.random.default_rng(11)
    for trial in range(300):
        V = int(g.integers(2, 50))
        k = int(g.integers(0, 6))
        p = np.stack([_dist(g, V, 1.5) for _ in range(k + 1)])
        q = np.stack([_dist(g, V, 1.5) for _ in range(k)]) if k else np.zeros((0, V))
        draft = [int(g.integers(0, V)) for _ in range(k)]
        a, b = np.random.default_rng([5, trial]), np.random.default_rng([5, trial])
        got = verify(p, q, draft, a)
        ref = oracle.verify(p, q, draft, b)
        assert got == ref, trial
        assert a.random() == b.random()


def test_verify_batch_generator_form_matches_the_reference_loop():
    """verify_batch(p, q, draft, rngs): each row's Generator is consumed as
    the reference's verify consumes it (one draw per accept test up to the
    first rejection, one for the emitted token), so the outputs equal the
    oracle's per-row loop on identical Generators and every Generator ends in
    the same state; k = 0 included."""
    g = np.random.default_rng(12)
    for trial, (B, k, V) in enumerate([(16, 4, 40), (9, 0, 17), (33, 2, 5), (8, 6, 3000)]):
        p = np.stack([[_dist(g, V, 1.5) for _ in range(k + 1)] for _ in range(B)])
        q = np.array([[_dist(g, V, 1.5) for _ in range(k)] for _ in range(B)]).reshape(B, k, V)
        draft = np.array([[int(g.choice(V, p=q[b, i])) for i in range(k)] for b in range(B)]).reshape(B, k)
        mine = [np.random.default_rng([trial, b]) for b in range(B)]
        ref = [np.random.default_rng([trial, b]) for b in range(B)]
        toks, n = verify_batch(p, q, draft, mine)
        for b in range(B):
            out, acc = oracle.verify(p[b], q[b], [int(t) for t in draft[b]], ref[b])
            assert int(n[b]) == acc and [int(t) for t in toks[b, : acc + 1]] == out, (trial, b)
            assert (toks[b, acc + 1 :] == -1).all()
            assert mine[b].random() == ref[b].random(), (trial, b)


def test_spec32k_parity():
    w = workloads.spec32k()
    toks, n = verify_batch(w["p"], w["q"], w["draft"], w["accept_u"], w["resample_u"])
    rt, rn = oracle.verify_batch(w["p"], w["q"], w["draft"], w["accept_u"], w["resample_u"])
    mism = band = 0
    for b in range(len(n)):
        gap = verify_boundary_gap(w["p"][b], w["q"][b], list(w["draft"][b]), w["accept_u"][b], w["resample_u"][b])
        band += gap < BAND
        if n[b] != rn[b] or not np.array_equal(toks[b], rt[b]):
            assert gap < DRAW_GAP, (b, gap)
            mism += 1
    print(f"spec32k rows {len(n)}, accepted mean {n.mean():.3f}, mismatches {mism}, "
          f"rows within 1e-6 of a decision boundary {band}")


def test_spec32k_float32_inputs():
    w = workloads.spec32k(rows=8)
    p32, q32 = w["p"].astype(np.float32), w["q"].astype(np.float32)
    toks, n = verify_batch(p32, q32, w["draft"], w["accept_u"], w["resample_u"])
    rt, rn = oracle.verify_batch(p32.astype(np.float64), q32.astype(np.float64), w["draft"], w["accept_u"],
                                 w["resample_u"])
    assert np.array_equal(n, rn) and np.array_equal(toks, rt)


def test_verify_edge_cases():
    p = np.array([[0.5, 0.5], [0.1, 0.9], [0.2, 0.8]])
    q = np.array([[0.25, 0.75], [0.5, 0.5]])
    # k = 0: a single draw from p[0]
    toks, n = verify_batch(p[None, :1], np.zeros((1, 0, 2)), np.zeros((1, 0), np.int64), np.zeros((1, 0)), [0.7])
    assert list(toks[0]) == [1] and n[0] == 0
    # zero residual: p <= q everywhere at the rejected position -> draw from p
    toks, n = verify_batch(np.array([[[0.1, 0.0], [0.5, 0.5]]]), np.array([[[0.2, 0.5]]]), [[0]], [[0.6]], [0.99])
    assert list(toks[0]) == [0, -1] and n[0] == 0
    # strict '<': u equal to the ratio rejects
    toks, n = verify_batch(np.array([[[0.5, 0.5], [1.0, 0.0]]]), np.array([[[1.0, 0.0]]]), [[0]], [[0.5]], [0.0])
    assert n[0] == 0
    with pytest.raises(IndexError):
        verify_batch(p[None], q[None], [[0, 2]], [[0.1, 0.1]], [0.5])


def test_verify_draw_across_chunks():
    """Rows longer than one 4096-token chunk, with the draw's mass placed in
    chosen chunks (the rest zero), a ragged last chunk, uniforms swept to
    both ends, and more draft tokens than one wave tests at once."""
    g = np.random.default_rng(21)
    V = 3 * 4096 + 17
    rows_p, rows_q, drafts, aus, dus = [], [], [], [], []
    k = 70
    for b in range(12):
        p = np.zeros((k + 1, V))
        q = np.zeros((k, V))
        for i in range(k + 1):
            # mass in one chunk, two chunks, or spread, by row
            lo, hi = [(0, V), (4096, 8192), (3 * 4096, V), (4095, 4097)][b % 4]
            p[i, lo:hi] = _dist(g, hi - lo, 2.0)
        for i in range(k):
            q[i] = p[i]
            # a rejection at b % k: q moves mass off the draft token's chunk
            if i == b % 5:
                q[i] = _dist(g, V, 0.5)
        draft = [int(np.argmax(q[i])) for i in range(k)]
        rows_p.append(p)
        rows_q.append(q)
        drafts.append(draft)
        aus.append(np.full(k, 0.5) if b % 3 else np.full(k, 1e-300))
        dus.append([0.0, 0.999999999, 0.5, 0.25][b % 4])
    P, Q = np.stack(rows_p), np.stack(rows_q)
    for dt in (np.float64, np.float32):
        toks, n = verify_batch(P.astype(dt), Q.astype(dt), drafts, np.stack(aus), dus)
        Pc, Qc = P.astype(dt).astype(np.float64), Q.astype(dt).astype(np.float64)
        rt, rn = oracle.verify_batch(Pc, Qc, np.array(drafts), np.stack(aus), np.array(dus))
        for b in range(len(n)):
            if n[b] != rn[b] or not np.array_equal(toks[b], rt[b]):
                gap = verify_boundary_gap(Pc[b], Qc[b], drafts[b], aus[b], dus[b])
                assert gap < DRAW_GAP, (dt, b, n[b], rn[b], gap)


def test_verify_draw_ends_of_the_cdf():
    """Uniforms at 0 and at the largest double below 1, mass confined to
    one chunk (zero weight after it, so the last chunks carry nothing), in
    the bonus draw (k = 0) and the residual draw: the first and the last
    token of positive weight, as numpy's searchsorted gives them."""
    V = 3 * 4096 + 5
    g = np.random.default_rng(4)
    u_top = float(np.nextafter(1.0, 0.0))
    for lo, hi in [(0, 100), (4100, 4200), (4095, 4097)]:
        p = np.zeros((1, 1, V))
        p[0, 0, lo:hi] = _dist(g, hi - lo)
        for u in (0.0, u_top):
            toks, n = verify_batch(p, np.zeros((1, 0, V)), np.zeros((1, 0), np.int64), np.zeros((1, 0)), [u])
            rt, rn = oracle.verify_batch(p, np.zeros((1, 0, V)), np.zeros((1, 0), np.int64), np.zeros((1, 0)),
                                         np.array([u]))
            assert n[0] == rn[0] == 0
            assert toks[0][0] == rt[0][0] == (lo if u == 0.0 else hi - 1), (lo, hi, u, toks, rt)
        # residual draw: q puts its mass elsewhere, so the residual is p's
        q = np.zeros((1, 1, V))
        q[0, 0, V - 1] = 1.0
        pp = np.concatenate([p, p], axis=1)
        for u in (0.0, u_top):
            toks, n = verify_batch(pp, q, [[V - 1]], [[0.999]], [u])
            rt, rn = oracle.verify_batch(pp, q, np.array([[V - 1]]), np.array([[0.999]]), np.array([u]))
            assert n[0] == rn[0] == 0
            assert toks[0][0] == rt[0][0] == (lo if u == 0.0 else hi - 1), (lo, hi, u, toks, rt)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_verify_batches(seed):
    """Random batches: k from 0 to 6, V from 2 to 70000 (chunk edges
    included), smooth, peaky and one-hot distributions, identical draft and
    target rows, drafts at the argmax or anywhere q is positive, in float64
    and float32.  float32 inputs are widened exactly and processed in
    float64, so they are compared with the oracle on the same values as
    float64 arrays."""
    for it in range(10):
        g = np.random.default_rng(77 + seed * 1000 + it)
        B, k = int(g.integers(1, 40)), int(g.integers(0, 7))
        V = int(g.choice([2, 50, 4096, 4097, 32000, 70000]))

        def dist(shape):
            m = int(g.integers(0, 3))
            if m == 2:  # one-hot rows (greedy drafts and targets)
                z = np.full(shape, -np.inf)
                np.put_along_axis(z, g.integers(0, V, shape[:-1])[..., None], 0.0, -1)
            else:
                z = g.normal(0, [2.0, 20.0][m], shape)
            e = np.exp(z - z.max(-1, keepdims=True))
            return e / e.sum(-1, keepdims=True)

        p, q = dist((B, k + 1, V)), dist((B, k, V))
        if k and g.random() < 0.3:
            q = p[:, :k].copy()
        draft = np.zeros((B, k), dtype=np.int64)
        for b in range(B):
            for i in range(k):
                t = int(np.argmax(q[b, i])) if g.random() < 0.5 else int(g.integers(0, V))
                draft[b, i] = t if q[b, i, t] > 0 else int(np.argmax(q[b, i]))
        au, ru = g.random((B, k)), g.random(B)
        if g.random() < 0.5:
            p, q = p.astype(np.float32), q.astype(np.float32)
        toks, n = verify_batch(p, q, draft, au, ru)
        p64, q64 = p.astype(np.float64), q.astype(np.float64)
        rt, rn = oracle.verify_batch(p64, q64, draft, au, ru)
        for b in np.nonzero((n != rn) | (toks != rt).any(1))[0]:
            gap = verify_boundary_gap(p64[b], q64[b], list(draft[b]), au[b], float(ru[b]))
            assert gap < DRAW_GAP, (it, int(b), toks[b].tolist(), rt[b].tolist(), gap)
