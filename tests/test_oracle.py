"""Pins the CPU oracle (CPU only, no GPU).

Three independent anchors:
  * the reference's own known-answer tests, transcribed as data in
    ``golden/reference_kats.json`` (``test_sampling.py``, ``test_speculative.py``);
  * a pure-Python brute force (``brute.py``) on many small random inputs,
    with ties forced on purpose;
  * targeted cases chosen so that a plausible slip in the oracle (``>``
    instead of ``>=`` for top-k, inclusive instead of exclusive mass for
    top-p, ``side="left"``, a missing clamp, a penalty applied per occurrence
    instead of per distinct id, a wrong RNG order in verify) fails.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import brute
import oracle
from oracle.sampler import _top_p_filter, verify_explicit
from pagellm_amd.params import SamplingParams, make_rng

# ------------------------------------------------------------------ KATs


def test_kat_greedy(kats):
    L = np.array(kats["logits"])
    g = kats["greedy"]
    assert oracle.sample(L, SamplingParams(temperature=0), None) == g["expected_id"]
    assert oracle.probs(L, SamplingParams(temperature=0))[g["expected_id"]] == 1.0


def test_kat_softmax(kats):
    L = np.array(kats["logits"])
    e = np.exp(L - L.max())
    np.testing.assert_allclose(oracle.probs(L, SamplingParams()), e / e.sum())


def test_kat_top_k(kats):
    L = np.array(kats["logits"])
    p = oracle.probs(L, SamplingParams(top_k=kats["top_k"]["top_k"]))
    assert set(np.nonzero(p)[0]) == set(kats["top_k"]["expected_support"])
    assert p.sum() == pytest.approx(1)


def test_kat_top_p(kats):
    L = np.array(kats["logits"])
    for case in kats["top_p"]:
        p = oracle.probs(L, SamplingParams(top_p=case["top_p"]))
        assert set(np.nonzero(p)[0]) == set(case["expected_support"])


def test_kat_penalty(kats):
    L = np.array(kats["logits"])
    c = kats["penalty"]
    out = oracle.apply_repetition_penalty(L, c["context"], c["penalty"])
    for i, v in c["expected"].items():
        assert out[int(i)] == v
    g = kats["penalty_greedy"]
    got = oracle.sample(L, SamplingParams(temperature=0, repetition_penalty=g["penalty"]), None, g["context"])
    assert got == g["expected_id"]


def test_kat_seeded(kats):
    L = np.array(kats["logits"])
    s = kats["seeded"]
    p = SamplingParams(temperature=s["temperature"], seed=s["seed"])
    a, b = make_rng(s["seed"], 0), make_rng(s["seed"], 0)
    xs = [oracle.sample(L, p, a) for _ in range(s["n_samples"])]
    ys = [oracle.sample(L, p, b) for _ in range(s["n_samples"])]
    assert xs == ys
    assert make_rng(42, 0).random() != make_rng(42, 1).random()


def test_kat_draw_stats(kats):
    d = kats["draw_stats"]
    p = np.array(d["p"])
    rng = np.random.default_rng(d["rng_seed"])
    counts = np.bincount([oracle.draw(p, rng) for _ in range(d["n_draws"])], minlength=len(p))
    counts = counts / d["n_draws"]
    assert counts[d["never_drawn"]] == 0
    np.testing.assert_allclose(counts, p, atol=d["atol"])


def test_kat_param_validation(kats):
    for bad in kats["param_validation"]["bad"]:
        with pytest.raises(ValueError):
            SamplingParams(**bad)


def _dist(rng, V, sharp=1.0):
    x = np.exp(rng.standard_normal(V) * sharp)
    return x / x.sum()


@pytest.mark.parametrize("k", [1, 2, 3])
def test_kat_verify_law(kats, k):
    c = kats["verify_law"]
    rng = np.random.default_rng(k)
    V = c["V"]
    p = np.stack([_dist(rng, V, c["sharp"]) for _ in range(k + 1)])
    q = np.stack([_dist(rng, V, c["sharp"]) for _ in range(k)])
    trials = c["trials"]  # the reference's own trial count and bounds
    first = np.zeros(V)
    joint = np.zeros((V, V))
    n_joint = 0
    for _ in range(trials):
        xs = [oracle.draw(q[i], rng) for i in range(k)]
        out, _ = oracle.verify(p, q, xs, rng)
        first[out[0]] += 1
        if len(out) >= 2:
            joint[out[0], out[1]] += 1
            n_joint += 1
    assert 0.5 * np.abs(first / trials - p[0]).sum() < c["tv_first"]
    if k >= 2:
        cond = joint.sum(0) / n_joint
        assert 0.5 * np.abs(cond - p[1]).sum() < c["tv_conditional"]


def test_kat_verify_naive_biased(kats):
    c = kats["verify_naive_biased"]
    rng = np.random.default_rng(c["rng_seed"])
    p, q = np.array(c["p"]), np.array(c["q"])
    wrong = np.bincount([int(np.argmax(p)) for _ in range(1000)], minlength=3) / 1000
    assert 0.5 * np.abs(wrong - p).sum() > c["tv_wrong_min"]
    good = np.bincount(
        [oracle.verify(p[None].repeat(2, 0), q[None], [oracle.draw(q, rng)], rng)[0][0] for _ in range(c["trials"])],
        minlength=3,
    ) / c["trials"]
    assert 0.5 * np.abs(good - p).sum() < c["tv_good_max"]


def test_kat_verify_identical(kats):
    c = kats["verify_identical"]
    rng = np.random.default_rng(c["rng_seed"])
    p = np.stack([_dist(rng, c["V"]) for _ in range(c["rows"])])
    for _ in range(c["trials"]):
        xs = [oracle.draw(p[i], rng) for i in range(c["k"])]
        out, acc = oracle.verify(p, p[: c["k"]], xs, rng)
        assert acc == c["k"] and out[: c["k"]] == xs and len(out) == c["k"] + 1


# ------------------------------------------------------- brute force pins


def _random_case(g, V):
    kind = g.integers(0, 3)
    if kind == 0:
        x = g.normal(0, 2, V)
    elif kind == 1:  # integer-valued logits: many exact ties
        x = g.integers(-3, 4, V).astype(np.float64)
    else:
        x = g.normal(0, 2, V).astype(np.float32).astype(np.float64)
        x[g.integers(0, V, 3)] = x.max()  # ties at the max
    T = [0.0, 1.0, 0.7, 1.3][g.integers(0, 4)]
    top_k = int(g.integers(0, V + 2))
    top_p = [1.0, 0.9, 0.5, 0.2, 0.999][g.integers(0, 5)]
    pen = [1.0, 1.2, 0.8][g.integers(0, 3)]
    ctx = list(g.integers(0, V, g.integers(0, 2 * V)))
    return x, T, top_k, top_p, pen, ctx


@pytest.mark.parametrize("seed", range(12))
def test_oracle_matches_brute_force(seed):
    g = np.random.default_rng(seed)
    for _ in range(40):
        V = int(g.integers(1, 40))
        x, T, top_k, top_p, pen, ctx = _random_case(g, V)
        params = SamplingParams(temperature=T, top_k=top_k, top_p=top_p, repetition_penalty=pen)
        po = oracle.probs(x, params, ctx)
        pb = np.array(brute.probs(x, T, top_k, top_p, pen, ctx))
        gap = oracle.top_p_boundary_gap(x, params, ctx)
        if gap > 1e-12:
            assert np.array_equal(po > 0, pb > 0), (V, T, top_k, top_p, pen)
        np.testing.assert_allclose(po, pb, rtol=1e-12, atol=1e-15)
        u = float(g.random())
        so = oracle.sample(x, params, u, ctx)
        if T == 0:
            assert so == brute.argmax_lowest(brute.penalize(x, ctx, pen))
        elif oracle.draw_boundary_gap(po, u) > 1e-12 and gap > 1e-12:
            assert so == brute.draw(list(pb), u)


@pytest.mark.parametrize("seed", range(6))
def test_oracle_verify_matches_brute_force(seed):
    g = np.random.default_rng(100 + seed)
    for _ in range(60):
        V = int(g.integers(2, 12))
        k = int(g.integers(0, 5))
        p = np.stack([_dist(g, V, 1.5) for _ in range(k + 1)])
        q = np.stack([_dist(g, V, 1.5) for _ in range(k)]) if k else np.zeros((0, V))
        if k and g.random() < 0.3:
            q[0] = p[0]  # a rejection here draws from p (zero residual)
        draft = [int(g.integers(0, V)) for _ in range(k)]
        us = list(g.random(k + 1))
        ob = oracle.verify(p, q, draft, oracle.ScriptedRNG(us))
        bb = brute.verify([list(r) for r in p], [list(r) for r in q], draft, us)
        assert ob == bb


# ------------------------------------------------------ targeted semantics


def test_top_k_keeps_all_ties_at_kth_value():
    # k=2, second-largest value 1.0 appears three times: support 4, not 2
    x = np.array([3.0, 1.0, 1.0, 0.0, 1.0])
    p = oracle.probs(x, SamplingParams(top_k=2))
    assert set(np.nonzero(p)[0]) == {0, 1, 2, 4}


def test_top_k_disabled_at_or_above_vocab():
    x = np.array([0.5, 0.1, 0.3])
    full = oracle.probs(x, SamplingParams())
    for k in (0, 3, 7):
        np.testing.assert_array_equal(oracle.probs(x, SamplingParams(top_k=k)), full)


def test_top_p_exclusive_mass_rule():
    # masses are exact binary fractions, so the comparisons are exact
    p = np.array([0.25, 0.5, 0.125, 0.125])
    # excl in order (1,0,2,3) = 0, .5, .75, .875
    for top_p, support in [(0.5, {1}), (0.5000001, {1, 0}), (0.75, {1, 0}), (0.875, {1, 0, 2}), (0.9, {0, 1, 2, 3})]:
        q = _top_p_filter(p.copy(), top_p)
        assert set(np.nonzero(q)[0]) == support, top_p
        assert q.sum() == pytest.approx(1.0)


def test_top_p_ties_broken_by_lowest_index():
    p = np.array([0.125, 0.25, 0.25, 0.25, 0.125])
    # order 1,2,3,0,4 ; excl 0,.25,.5,.75,.875 ; top_p .5 keeps {1,2}
    q = _top_p_filter(p.copy(), 0.5)
    assert set(np.nonzero(q)[0]) == {1, 2}


def test_draw_side_right_and_clamp():
    p = np.array([0.25, 0.25, 0.5])
    assert oracle.draw(p, 0.0) == 0
    assert oracle.draw(p, 0.25) == 1  # t == c_0 exactly: first c_i > t is i=1
    assert oracle.draw(p, 0.5) == 2
    assert oracle.draw(np.array([0.0, 0.0, 1.0]), 0.0) == 2  # zero-mass prefix skipped
    # a zero-mass tail can never be drawn, the clamp keeps the result < V
    assert oracle.draw(np.array([1.0, 0.0]), 0.999999) == 0
    assert oracle.draw(np.array([0.0, 0.0]), 0.5) == 1  # empty mass -> V-1


def test_penalty_once_per_distinct_id_and_sign_rule():
    x = np.array([2.0, -2.0, 0.0, 4.0])
    out = oracle.apply_repetition_penalty(x, [0, 0, 0, 1, 2], 2.0)
    assert list(out) == [1.0, -4.0, 0.0, 4.0]
    out = oracle.apply_repetition_penalty(x, [3], 0.5)  # penalty < 1 raises
    assert out[3] == 8.0
    assert oracle.apply_repetition_penalty(x, [0], 1.0) is x
    assert oracle.apply_repetition_penalty(x, [], 2.0) is x


def test_greedy_ignores_temperature_and_consumes_no_uniform():
    x = np.array([0.1, 0.9, 0.9, -1.0])
    r = oracle.ScriptedRNG([])
    assert oracle.sample(x, SamplingParams(temperature=0, top_k=1, top_p=0.1), r) == 1
    assert r.consumed == 0


def test_nongreedy_sample_consumes_exactly_one_uniform():
    x = np.array([0.1, 0.9, 0.3])
    r = oracle.ScriptedRNG([0.5, 0.7])
    oracle.sample(x, SamplingParams(temperature=0.5, top_k=2), r)
    assert r.consumed == 1


def test_verify_rng_order_and_counts():
    p = np.array([[0.5, 0.5], [0.5, 0.5], [0.1, 0.9]])
    q = np.array([[0.25, 0.75], [0.5, 0.5]])
    # test 0: x=1, ratio .5/.75 = 2/3 -> u=.9 rejects; residual = [.25,0] -> draw 0
    r = oracle.ScriptedRNG([0.9, 0.99, 123.0])
    out, n = oracle.verify(p, q, [1, 0], r)
    assert (out, n, r.consumed) == ([0], 0, 2)
    # accept both (ratio 2/3 then 1): bonus from p[2] with u=.05 -> token 0
    r = oracle.ScriptedRNG([0.1, 0.999, 0.05])
    out, n = oracle.verify(p, q, [1, 0], r)
    assert (out, n, r.consumed) == ([1, 0, 0], 2, 3)
    # strict '<': u exactly equal to the ratio rejects
    r = oracle.ScriptedRNG([0.5, 0.0])
    out, n = oracle.verify(np.array([[0.5, 0.5], [1.0, 0.0]]), np.array([[1.0, 0.0]]), [0], r)
    assert n == 0


def test_verify_identical_rows_always_accept():
    p = np.array([[0.2, 0.8], [0.5, 0.5]])
    out, n = verify_explicit(p, p[:1], [0], [0.9999999], 0.1)  # ratio 1: any u < 1 accepts
    assert (out, n) == ([0, 0], 1)


def test_verify_residual_and_zero_residual_branches():
    # ratio .1/.2 = .5, u = .6 rejects; residual max(p-q,0) = [0, .1] -> token 1
    out, n = verify_explicit(np.array([[0.1, 0.9], [0.5, 0.5]]), np.array([[0.2, 0.8]]), [0], [0.6], 0.95)
    assert (out, n) == ([1], 0)
    # p <= q everywhere (unnormalised on purpose): residual sums to 0, so the
    # draw falls back to p itself (speculative.py:55-57)
    out, n = verify_explicit(np.array([[0.1, 0.0], [0.5, 0.5]]), np.array([[0.2, 0.5]]), [0], [0.6], 0.99)
    assert (out, n) == ([0], 0)


def test_boundary_gauges():
    p = np.array([0.25, 0.25, 0.5])
    assert oracle.draw_boundary_gap(p, 0.25) == 0.0
    assert oracle.draw_boundary_gap(p, 0.3) == pytest.approx(0.05)
    x = np.log(np.array([0.5, 0.25, 0.125, 0.125]))
    gap = oracle.top_p_boundary_gap(x, SamplingParams(top_p=0.7), ())
    assert gap == pytest.approx(0.05, abs=1e-12)
    assert math.isinf(oracle.top_p_boundary_gap(x, SamplingParams(), ()))


def test_sample_batch_uses_row_uniforms():
    g = np.random.default_rng(5)
    L = g.normal(0, 1, (4, 9))
    params = [SamplingParams(temperature=0), SamplingParams(), SamplingParams(top_k=3), SamplingParams(top_p=0.5)]
    u = g.random(4)
    ids = oracle.sample_batch(L, params, u)
    for b in range(4):
        assert ids[b] == oracle.sample(L[b], params[b], u[b])


# ------------------------------------------------- verify_batch, verify gauge


def _brute_uniforms(p_rows, q_rows, draft, accept_u, draw_u):
    """The uniforms the brute force consumes, left to right: the accept
    uniforms up to and including the first rejection (found here with the
    brute force's own ratio rule), then the draw's."""
    used = []
    for i, x in enumerate(draft):
        used.append(float(accept_u[i]))
        r = float(p_rows[i][x]) / float(q_rows[i][x])
        if not float(accept_u[i]) < (r if r < 1.0 else 1.0):
            break
    return used + [float(draw_u)]


@pytest.mark.parametrize("seed", range(6))
def test_verify_batch_matches_brute_force_row_by_row(seed):
    """oracle.verify_batch against brute.verify on random small batches:
    k from 0 to 5, smooth and peaked rows, drafts drawn from q (so q[x] > 0),
    with uniforms spread so that both the accept and the reject branches
    occur; the tokens past the stop position stay -1."""
    g = np.random.default_rng(900 + seed)
    seen_accept_all = seen_reject = 0
    for k in range(6):
        B, V = 7, int(g.integers(2, 40))
        sharp = [0.3, 1.0, 3.0][seed % 3]
        p = np.stack([[_dist(g, V, sharp) for _ in range(k + 1)] for _ in range(B)])
        q = np.array([[_dist(g, V, sharp) for _ in range(k)] for _ in range(B)]).reshape(B, k, V)
        draft = np.array([[int(g.choice(V, p=q[b, i])) for i in range(k)] for b in range(B)], dtype=np.int64).reshape(B, k)
        accept_u = g.random((B, k)) ** 0.5
        resample_u = g.random(B)
        tokens, n_acc = oracle.verify_batch(p, q, draft, accept_u, resample_u)
        assert tokens.shape == (B, k + 1) and n_acc.shape == (B,)
        for b in range(B):
            d = [int(t) for t in draft[b]]
            want_out, want_n = brute.verify(
                [list(r) for r in p[b]], [list(r) for r in q[b]], d,
                _brute_uniforms(p[b], q[b], d, accept_u[b], resample_u[b]),
            )
            assert int(n_acc[b]) == want_n
            assert [int(t) for t in tokens[b, : want_n + 1]] == want_out
            assert (tokens[b, want_n + 1 :] == -1).all()
            seen_accept_all += want_n == k
            seen_reject += want_n < k
    assert seen_accept_all > 0 and seen_reject > 0


def test_verify_batch_k0_is_one_draw_per_row():
    g = np.random.default_rng(31)
    B, V = 9, 11
    p = np.stack([[_dist(g, V)] for _ in range(B)])
    u = g.random(B)
    tokens, n_acc = oracle.verify_batch(p, np.zeros((B, 0, V)), np.zeros((B, 0), np.int64), np.zeros((B, 0)), u)
    assert (n_acc == 0).all() and tokens.shape == (B, 1)
    for b in range(B):
        assert int(tokens[b, 0]) == brute.draw(list(p[b, 0]), float(u[b]))


def test_verify_boundary_gap_hand_built():
    """Cases whose gap is fixed by hand: a uniform exactly at min(1, p/q),
    a final draw exactly on a CDF boundary, known positive gaps on both the
    accept and the residual branch, and the per-stop draw uniforms."""
    p = np.array([[0.5, 0.5], [0.25, 0.75]])
    q = np.array([[0.25, 0.75]])
    thr = 0.5 / 0.75
    # u exactly at the threshold: gap 0 (u < thr is false: a rejection)
    assert oracle.verify_boundary_gap(p, q, [1], [thr], 0.3) == 0.0
    # accepted (u = 0.2 < 2/3): accept gap 2/3 - 0.2; final draw over p[1] =
    # [.25, .75] at u = 0.25 sits on the boundary c_0 = 0.25: gap 0
    assert oracle.verify_boundary_gap(p, q, [1], [0.2], 0.25) == 0.0
    # same, draw at u = 0.5: distance 0.25 to c_0 and 0.5 to c_1 = 1
    assert oracle.verify_boundary_gap(p, q, [1], [0.2], 0.5) == pytest.approx(0.25)
    # accept gap smaller than the draw gap: u = 0.6, thr - u = 0.0667
    assert oracle.verify_boundary_gap(p, q, [1], [0.6], 0.5) == pytest.approx(thr - 0.6)
    # q[x] = 0 makes the ratio inf: threshold 1, gap 1 - u
    assert oracle.verify_boundary_gap(p, np.array([[0.0, 1.0]]), [0], [0.9], 0.5) == pytest.approx(0.1)
    # rejection with a zero ratio (p[x] = 0): gap u, then the residual
    # max(p - q, 0) = [.3, .3, 0] normalised to [.5, .5, 0] drawn at u = 0.25
    # (distance 0.25 to both c_-1 = 0 and c_0 = 0.5)
    p3 = np.array([[0.5, 0.5, 0.0], [1 / 3, 1 / 3, 1 / 3]])
    q3 = np.array([[0.2, 0.2, 0.6]])
    assert oracle.verify_boundary_gap(p3, q3, [2], [0.4], 0.25) == pytest.approx(0.25)
    assert oracle.verify_boundary_gap(p3, q3, [2], [0.1], 0.25) == pytest.approx(0.1)
    assert oracle.verify_boundary_gap(p3, q3, [2], [0.4], 0.5) == 0.0  # on c_0 of the residual
    # identical rows with u = 1 (outside [0, 1) on purpose): rejected at the
    # threshold itself, gap 0, and the zero residual falls back to p
    assert oracle.verify_boundary_gap(p[:1], p[:1], [0], [1.0], 0.3) == 0.0
    # per-stop draw uniforms: a rejection at position 0 uses draw_u[0], the
    # accept-all path draw_u[k]
    assert oracle.verify_boundary_gap(p3, q3, [2], [0.4], np.array([0.25, 0.9])) == pytest.approx(0.25)
    assert oracle.verify_boundary_gap(p, q, [1], [0.2], np.array([0.9, 0.25])) == 0.0
    # k = 0: only the draw over p_rows[0]
    assert oracle.verify_boundary_gap(p[1:], q[:0], [], [], 0.625) == pytest.approx(0.375)


def test_verify_boundary_gap_bounds_every_flip():
    """On random rows, moving every uniform by half the reported gap changes
    neither n_acc nor the emitted tokens (checked with the brute force)."""
    g = np.random.default_rng(77)
    for trial in range(40):
        k, V = int(g.integers(0, 4)), int(g.integers(2, 12))
        p = np.stack([_dist(g, V) for _ in range(k + 1)])
        q = np.array([_dist(g, V) for _ in range(k)]).reshape(k, V)
        draft = [int(g.choice(V, p=q[i])) for i in range(k)]
        au = g.random(k)
        du = float(g.random())
        gap = oracle.verify_boundary_gap(p, q, draft, au, du)
        assert gap >= 0.0
        base = brute.verify([list(r) for r in p], [list(r) for r in q], draft, _brute_uniforms(p, q, draft, au, du))
        eps = gap * 0.5
        for shift in (-eps, eps):
            au2 = np.clip(au + shift, 0.0, np.nextafter(1.0, 0.0))
            du2 = float(np.clip(du + shift, 0.0, np.nextafter(1.0, 0.0)))
            got = brute.verify([list(r) for r in p], [list(r) for r in q], draft, _brute_uniforms(p, q, draft, au2, du2))
            assert got == base, (trial, gap, shift)
