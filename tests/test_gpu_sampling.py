"""GPU parity of the sampler against the CPU oracle (needs an MI355X).

Bar (per the numerics contract of this path):
  * greedy ids: bit-exact;
  * top-k / top-p support sets: exact, except rows whose top-p cut sits
    within 1e-12 of flipping in the oracle (counted and reported);
  * probabilities on the support: within 1e-5 relative;
  * sampled ids: equal, except where the uniform lies within 1e-12 of a CDF
    boundary; rows within 1e-6 of one are counted and reported.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle.sampler import sample_boundary_gaps
from parity import DRAW_GAP, TOPP_GAP
from parity import compare_rows as _compare_rows
from pagellm_amd import _native, workloads
from pagellm_amd.params import SamplingParams, make_rng
from pagellm_amd.sampling import apply_repetition_penalty, draw, probs, sample, sample_batch

pytestmark = pytest.mark.gpu

PROB_RTOL = 1e-5


def _compare_probs(x, prm, ctx, label):
    pg = probs(x, prm, ctx)
    pr = oracle.probs(x, prm, ctx)
    gap = oracle.top_p_boundary_gap(x, prm, ctx)
    if gap >= TOPP_GAP:
        assert np.array_equal(pg > 0, pr > 0), (label, np.flatnonzero((pg > 0) != (pr > 0))[:10])
    both = (pg > 0) & (pr > 0)
    if both.any():
        rel = np.max(np.abs(pg[both] - pr[both]) / pr[both])
        assert rel < PROB_RTOL, (label, rel)
        return rel
    return 0.0


# ------------------------------------------------------------- reference KATs


def test_kat_greedy(kats):
    L = np.array(kats["logits"])
    assert sample(L, SamplingParams(temperature=0), make_rng(0, 0)) == kats["greedy"]["expected_id"]
    assert probs(L, SamplingParams(temperature=0))[kats["greedy"]["expected_id"]] == 1.0


def test_kat_softmax(kats):
    L = np.array(kats["logits"])
    e = np.exp(L - L.max())
    np.testing.assert_allclose(probs(L, SamplingParams()), e / e.sum(), rtol=1e-12)


def test_kat_top_k_and_top_p(kats):
    L = np.array(kats["logits"])
    p = probs(L, SamplingParams(top_k=kats["top_k"]["top_k"]))
    assert set(np.nonzero(p)[0]) == set(kats["top_k"]["expected_support"]) and p.sum() == pytest.approx(1)
    for case in kats["top_p"]:
        p = probs(L, SamplingParams(top_p=case["top_p"]))
        assert set(np.nonzero(p)[0]) == set(case["expected_support"])


def test_kat_penalty(kats):
    L = np.array(kats["logits"])
    c = kats["penalty"]
    out = apply_repetition_penalty(L, c["context"], c["penalty"])
    for i, v in c["expected"].items():
        assert out[int(i)] == v
    assert apply_repetition_penalty(L, c["context"], 1.0) is L
    g = kats["penalty_greedy"]
    assert sample(L, SamplingParams(temperature=0, repetition_penalty=g["penalty"]), None, g["context"]) == g["expected_id"]


def test_kat_seeded(kats):
    L = np.array(kats["logits"])
    p = SamplingParams(temperature=1.0, seed=42)
    a, b = make_rng(42, 0), make_rng(42, 0)
    xs = [sample(L, p, a) for _ in range(20)]
    ys = [sample(L, p, b) for _ in range(20)]
    assert xs == ys
    # and they are the oracle's draws from the same stream
    c = make_rng(42, 0)
    assert xs == [oracle.sample(L, p, c) for _ in range(20)]


def test_kat_draw_stats(kats):
    d = kats["draw_stats"]
    p = np.array(d["p"])
    rng = np.random.default_rng(d["rng_seed"])
    counts = np.bincount([draw(p, rng) for _ in range(d["n_draws"])], minlength=len(p)) / d["n_draws"]
    assert counts[d["never_drawn"]] == 0
    np.testing.assert_allclose(counts, p, atol=d["atol"])


def test_sample_consumes_like_reference():
    L = np.array([0.3, -0.2, 1.5, 0.0])
    for prm in [SamplingParams(temperature=0), SamplingParams(), SamplingParams(top_k=2, top_p=0.7)]:
        a, b = make_rng(9, 1), make_rng(9, 1)
        for _ in range(5):
            assert sample(L, prm, a) == oracle.sample(L, prm, b)
        assert a.random() == b.random()


# ------------------------------------------------------------ workloads


def test_char65_full_parity():
    w = workloads.char65()
    for rowwise in (False, True):
        ids = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"], rowwise=rowwise)
        _compare_rows(w, range(16), ids, f"char65 rowwise={rowwise}")
    rels = [_compare_probs(w["logits"][r], w["params"][r], w["contexts"][r], "char65") for r in range(16)]
    print("char65 max prob rel err", max(rels))


def test_char65_through_engine_rngs():
    """Same ids whether uniforms come pre-drawn or from each row's Generator."""
    w = workloads.char65()
    rngs = [make_rng(s, 0) for s in w["seeds"]]
    ids = sample_batch(w["logits"], w["params"], rngs, w["contexts"])
    ref = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    assert np.array_equal(ids, ref)


@pytest.fixture(scope="module")
def mixed():
    return workloads.mixed128k()


def test_mixed128k_parity(mixed):
    w = mixed
    before = _native.default_context().fallback_rows()
    ids = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    fb = _native.default_context().fallback_rows() - before
    print(f"mixed128k: rows finished by the general path: {fb}")
    rows = [g * 64 + i for g in range(4) for i in range(0, 64, 8)]
    _compare_rows(w, rows, ids, "mixed128k split")
    assert np.all((ids >= 0) & (ids < w["logits"].shape[1]))
    # greedy group: every row bit-exact against numpy argmax
    assert np.array_equal(ids[:64], np.argmax(w["logits"][:64], axis=1))


def test_mixed128k_rowwise_matches_split(mixed):
    w = mixed
    a = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    b = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"], rowwise=True)
    diff = np.flatnonzero(a != b)
    for r in diff:  # only boundary cases may differ between two exact paths
        g_topp, g_draw = sample_boundary_gaps(w["logits"][r], w["params"][r], w["uniforms"][r], w["contexts"][r])
        assert g_topp < TOPP_GAP or g_draw < DRAW_GAP, r
    print(f"mixed128k split vs rowwise differing rows: {len(diff)}")


def test_mixed128k_probs(mixed):
    w = mixed
    rels = []
    for r in (1, 70, 130, 200, 255):
        rels.append(_compare_probs(w["logits"][r], w["params"][r], w["contexts"][r], f"mixed128k row {r}"))
    print("mixed128k max prob rel err", max(rels))


def test_mixed128k_deterministic(mixed):
    w = mixed
    a = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    b = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    assert np.array_equal(a, b)


def test_zipf32k_parity():
    w = workloads.zipf32k()
    ids = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    _compare_rows(w, range(64), ids, "zipf32k split")
    for r in (0, 31, 63):
        _compare_probs(w["logits"][r], w["params"][r], w["contexts"][r], f"zipf32k row {r}")


def test_zipf152k_parity():
    w = workloads.zipf152k(rows=128)
    ids = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    _compare_rows(w, range(0, 128, 8), ids, "zipf152k")
    _compare_probs(w["logits"][3], w["params"][3], w["contexts"][3], "zipf152k row 3")


def test_general_path_inside_fast_kernel():
    """Rows whose kept set outgrows the LDS candidate store (top-p over a
    near-flat distribution, or a huge top-k) are finished by the general
    pipeline inside the same kernel; results must match the oracle and the
    row-wise kernel."""
    g = np.random.default_rng(21)
    V = 50000
    x = g.normal(0, 0.05, (4, V)).astype(np.float32)
    params = [SamplingParams(top_p=0.9), SamplingParams(top_k=30000), SamplingParams(top_k=30000, top_p=0.5),
              SamplingParams(top_p=0.97, temperature=2.0)]
    u = g.random(4)
    c = _native.default_context()
    before = c.fallback_rows()
    ids = sample_batch(x, params, uniforms=u)
    assert c.fallback_rows() - before == 4
    w = dict(logits=x, params=params, contexts=[[]] * 4, uniforms=u)
    _compare_rows(w, range(4), ids, "general-in-fast")
    assert np.array_equal(ids, sample_batch(x, params, uniforms=u, rowwise=True))


def test_penalize_matches_reference_rule():
    g = np.random.default_rng(3)
    for dt in (np.float32, np.float64):
        x = g.normal(0, 2, 1000).astype(dt)
        x[:5] = 0
        ctx = list(g.integers(0, 1000, 300)) + [0, 1, 2, -1]
        got = apply_repetition_penalty(x, ctx, 1.7)
        ref = oracle.apply_repetition_penalty(x, ctx, 1.7)
        assert got.dtype == ref.dtype == dt
        assert np.array_equal(got, ref)


def _nucleus_batch(g, V, B, kind, dtype):
    if kind == "zipf":
        x = -np.log(1 + g.permuted(np.tile(np.arange(V), (B, 1)), axis=1)) + g.normal(0, 0.3, (B, V))
    elif kind == "flat":
        x = g.normal(0, 0.05, (B, V))
    elif kind == "masked":
        x = g.normal(0, 2, (B, V))
        x[:, g.integers(0, V, V // 2)] = -np.inf
    elif kind == "ties":
        x = np.round(g.normal(0, 1, (B, V)) * 2) / 2
    else:
        x = g.normal(0, 3, (B, V))
    return x.astype(dtype)


@pytest.mark.parametrize("kind", ["zipf", "flat", "masked", "ties", "normal"])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_nucleus_path_matches_oracle(kind, dtype):
    """Rows with no top-k and top_p >= 0.98 take the three-pass nucleus path
    (sample_batch sets the hint): against the oracle and the row-wise
    kernel, with penalties on both sides of 1, temperatures, vocabularies
    at and off the chunk size, and rows mixed with other modes."""
    g = np.random.default_rng(2 * ["zipf", "flat", "masked", "ties", "normal"].index(kind) + (dtype == np.float64))
    for V in (16384, 50257, 152064):
        B = 12
        x = _nucleus_batch(g, V, B, kind, dtype)
        params = [SamplingParams(top_p=float(g.choice([0.98, 0.99, 0.995, 0.999999])),
                                 temperature=float(g.choice([1.0, 0.7, 1.6])),
                                 repetition_penalty=float(g.choice([1.0, 1.05, 0.9])))
                  for _ in range(B - 2)]
        params += [SamplingParams(temperature=0.0), SamplingParams(top_k=40, top_p=0.99)]
        # histories short enough that no chunk sets aside more penalised
        # tokens than its pools hold (which would send the row to the
        # general pipeline in every mode)
        ctx = [list(g.integers(-V, V, int(g.integers(0, min(3000, V // 32))))) for _ in range(B)]
        u = g.random(B)
        c = _native.default_context()
        before = c.fallback_rows()
        ids = sample_batch(x, params, uniforms=u, contexts=ctx)
        if kind in ("zipf", "normal"):  # no row needs the general pipeline
            assert c.fallback_rows() == before, (kind, V)
        w = dict(logits=x, params=params, contexts=ctx, uniforms=u)
        _compare_rows(w, range(B), ids, f"nucleus-{kind}-{V}")
        assert np.array_equal(ids, sample_batch(x, params, uniforms=u, contexts=ctx, rowwise=True))


def test_nucleus_path_hands_rows_to_the_general_pipeline():
    """A row with a single distinct finite value, and a row whose cut window
    outgrows the candidate slots (a wide flat band at the cut), are finished
    by the general pipeline inside the nucleus kernels."""
    V = 40000
    x = np.zeros((3, V), dtype=np.float32)
    x[1, : V // 2] = 1.0  # two values: half the vocabulary ties at the cut
    x[2] = np.random.default_rng(3).normal(0, 1, V)
    params = [SamplingParams(top_p=0.99)] * 3
    u = np.array([0.3, 0.6, 0.9])
    c = _native.default_context()
    before = c.fallback_rows()
    ids = sample_batch(x, params, uniforms=u)
    assert c.fallback_rows() - before == 2
    w = dict(logits=x, params=params, contexts=[[]] * 3, uniforms=u)
    _compare_rows(w, range(3), ids, "nucleus-general")
    assert np.array_equal(ids, sample_batch(x, params, uniforms=u, rowwise=True))
