"""GPU edge cases and cross-path agreement (needs an MI355X): tiny and odd
vocabularies, float64 inputs, strided rows, ties, masked (-inf) logits,
extreme parameters; the split kernel against the row-wise kernel and the
oracle on many random configurations."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle.sampler import sample_boundary_gaps
from parity import DRAW_GAP, TOPP_GAP
from pagellm_amd.params import SamplingParams
from pagellm_amd.sampling import probs, sample, sample_batch

pytestmark = pytest.mark.gpu


def _check(x, params, u, ctx, ids):
    for r in range(len(ids)):
        ref = oracle.sample(x[r], params[r], u[r], ctx[r])
        if ids[r] != ref:
            g_topp, g_draw = sample_boundary_gaps(x[r], params[r], u[r], ctx[r])
            assert g_topp < TOPP_GAP or g_draw < DRAW_GAP, (r, params[r], int(ids[r]), ref)


def _random_params(g, V):
    T = [0.0, 1.0, 0.7, 1.7, 0.05][g.integers(0, 5)]
    k = [0, 1, 2, 5, 50, V - 1, V, V + 3][g.integers(0, 8)]
    p = [1.0, 0.9, 0.5, 1e-9, 0.999999][g.integers(0, 5)]
    r = [1.0, 1.3, 0.7][g.integers(0, 3)]
    return SamplingParams(temperature=T, top_k=max(int(k), 0), top_p=p, repetition_penalty=r)


@pytest.mark.parametrize("V", [1, 2, 5, 65, 2047, 2048, 2049, 8191, 8192, 8193, 20000, 40000])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_random_rows_all_paths(V, dtype):
    g = np.random.default_rng(V * 7 + (dtype == np.float64))
    B = 24
    x = g.normal(0, 2, (B, V))
    x[::3] = np.round(x[::3])  # rows with many exact ties
    x = x.astype(dtype)
    params = [_random_params(g, V) for _ in range(B)]
    ctx = [list(g.integers(0, V, g.integers(0, 300))) for _ in range(B)]
    u = g.random(B)
    a = sample_batch(x, params, uniforms=u, contexts=ctx)
    b = sample_batch(x, params, uniforms=u, contexts=ctx, rowwise=True)
    _check(x, params, u, ctx, a)
    _check(x, params, u, ctx, b)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("V", [8192, 50000])
def test_tiny_top_p_keeps_the_row_max(V, dtype):
    """top_p far below the largest probability keeps exactly the row's
    maximum (sampling.py:82-90), whatever the temperature and penalty.  The
    row max's exp argument, y(z) - y(zmax), can round to a residual just
    above 0 when T != 1, which puts its probability an ulp above 1/S; the
    merge's top-p key range must still hold it."""
    g = np.random.default_rng(V + 11 * (dtype == np.float64))
    B = 48
    x = g.normal(0, 2, (B, V)).astype(dtype)
    temps = [0.7, 0.9, 1.3, 0.35, 1.0, 2.5]
    params = [SamplingParams(temperature=temps[b % len(temps)], top_p=1e-9,
                             repetition_penalty=(1.3, 1.0, 0.8)[b % 3]) for b in range(B)]
    ctx = [list(g.integers(0, V, 200)) for _ in range(B)]
    u = g.random(B)
    ids = sample_batch(x, params, uniforms=u, contexts=ctx)
    _check(x, params, u, ctx, ids)
    for b in range(B):
        assert ids[b] == oracle.sample(x[b], params[b], u[b], ctx[b]), b


def test_masked_logits_and_all_ties():
    V = 10000
    x = np.full((4, V), -np.inf, dtype=np.float32)
    x[0, 17] = 1.0
    x[1, [3, 9000]] = 2.0
    x[2] = 0.5  # all equal
    x[3, ::7] = np.arange(len(x[3, ::7]), dtype=np.float32) % 5
    params = [SamplingParams(), SamplingParams(top_k=1), SamplingParams(top_p=0.3), SamplingParams(top_k=3, top_p=0.5)]
    u = np.array([0.3, 0.9, 0.77, 0.51])
    ctx = [[], [], [], []]
    ids = sample_batch(x, params, uniforms=u, contexts=ctx)
    _check(x, params, u, ctx, ids)
    assert ids[0] == 17
    assert ids[1] in (3, 9000)
    gre = sample_batch(x, SamplingParams(temperature=0), contexts=ctx)
    assert list(gre) == [17, 3, 0, int(np.argmax(x[3]))]


def test_strided_torch_rows():
    torch = pytest.importorskip("torch")
    g = np.random.default_rng(5)
    base = g.normal(0, 3, (16, 40000)).astype(np.float32)
    t = torch.from_numpy(base).cuda()[:, :33333]  # ld 40000, V 33333
    params = [SamplingParams(top_k=20, top_p=0.8)] * 16
    u = g.random(16)
    ids = sample_batch(t, params, uniforms=u)
    ref = sample_batch(np.ascontiguousarray(base[:, :33333]), params, uniforms=u)
    assert np.array_equal(ids, ref)


def test_single_row_api_float64():
    x = np.array([2.0, 1.0, 0.5, -1.0, 3.0, 3.0])
    assert sample(x, SamplingParams(temperature=0), None) == 4  # lowest index among ties
    p = probs(x, SamplingParams(top_k=1))
    assert set(np.nonzero(p)[0]) == {4, 5}  # both tied tokens kept
    p = probs(x, SamplingParams(top_p=1e-9))
    assert set(np.nonzero(p)[0]) == {4}  # the index tie-break keeps the lower one


def test_large_history_duplicates():
    V = 50000
    g = np.random.default_rng(8)
    x = g.normal(0, 1, (2, V)).astype(np.float32)
    ctx = [np.tile(np.arange(1000), 30), np.concatenate([np.arange(V), np.arange(V)])]
    params = [SamplingParams(temperature=0, repetition_penalty=1.5), SamplingParams(repetition_penalty=3.0, top_k=7)]
    u = np.array([0.0, 0.42])
    ids = sample_batch(x, params, uniforms=u, contexts=ctx)
    _check(x, params, u, ctx, ids)


def _shaped_logits(g, kind, B, V):
    if kind == 0:
        return g.normal(0, 3, (B, V))
    if kind == 1:
        return g.normal(0, 30, (B, V))  # peaky: a handful of tokens hold the mass
    if kind == 2:
        return g.normal(0, 0.05, (B, V))  # nearly flat: nuclei of most of the vocabulary
    if kind == 3:
        return np.round(g.normal(0, 2, (B, V)) * 4) / 4  # a few hundred distinct values
    if kind == 4:  # Zipf over a random token order
        return -np.log(1 + g.permuted(np.tile(np.arange(V), (B, 1)), axis=1)) + g.normal(0, 0.3, (B, V))
    x = g.normal(0, 2, (B, V))
    x[:, g.integers(0, V, max(1, V // 3))] = -np.inf  # a third of the vocabulary masked
    return x


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_batches_across_shapes(seed):
    """Random batches over vocabularies from 3 to 152064 (chunk edges
    included), six logit shapes, both input precisions, mixed per-row
    parameters (greedy, extreme temperatures, top-k above V, tiny and
    near-one top_p, penalties on both sides of 1) and histories with
    negative ids and duplicates, against the oracle row by row."""
    for it in range(12):
        g = np.random.default_rng(seed * 1000 + it)
        V = int(g.choice([3, 100, 4097, 16383, 16384, 16385, 32000, 50257, 128256, 152064]))
        B = int(g.integers(1, 40))
        kind = int(g.integers(0, 6))
        dtype = np.float64 if g.random() < 0.25 else np.float32
        x = _shaped_logits(g, kind, B, V).astype(dtype)
        params = [SamplingParams(temperature=float(g.choice([0.0, 1.0, 0.6, 1.5, 1e-3, 5.0])),
                                 top_k=int(g.choice([0, 0, 1, 7, 40, 400, 600, 5000, V, V + 1])),
                                 top_p=float(g.choice([1.0, 1.0, 0.9, 0.95, 0.99, 0.5, 1e-6, 0.999999])),
                                 repetition_penalty=float(g.choice([1.0, 1.0, 1.1, 1.3, 0.8, 2.0])))
                  for _ in range(B)]
        H = int(g.choice([0, 10, 500, 2048, 6000]))
        ctx = [list(g.integers(-V, V, int(g.integers(0, H + 1)))) for _ in range(B)]
        u = g.random(B)
        _check(x, params, u, ctx, sample_batch(x, params, uniforms=u, contexts=ctx))


@pytest.mark.parametrize("offset", [1e4, -1e4])
def test_logits_far_from_zero(offset):
    """Logits near +-1e4 over a narrow range: the float histogram's bin
    edges move by up to |lo * scale| * 2^-24 bins there, and the threshold's
    margin grows with it.  Ids match the oracle, and the chunks keep enough
    candidates that the rows stay on the fast path as often as the same
    rows near zero do."""
    from pagellm_amd import _native, workloads

    w = workloads.mixed128k(rows=64, V=32768)
    c = _native.default_context()
    f0 = c.fallback_rows()
    ids0 = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    f1 = c.fallback_rows()
    w["logits"] = (w["logits"].astype(np.float64) + offset).astype(np.float32)
    ids = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    f2 = c.fallback_rows()
    _check(w["logits"], w["params"], w["uniforms"], w["contexts"], ids)
    print(f"offset {offset}: general-path rows {f2 - f1} (near zero: {f1 - f0})", flush=True)
    assert f2 - f1 <= f1 - f0 + 4
    assert ids0.shape == ids.shape


def test_clustered_top_p_rows():
    """Top-p rows whose large values cluster inside the threads' register
    slots (values repeated in blocks of 4, 16 or 256 tokens, sorted rows),
    where a threshold taken from a few values per thread would keep far too
    many candidates.  Ids match the oracle, and the block rows stay on the
    fast path: the chunk's value histogram keeps ~965-995 candidates of the
    1024 slots on them, as on unclustered rows.  The sorted rows hold their
    whole nucleus in one chunk and go to the general pipeline."""
    from pagellm_amd import _native

    g = np.random.default_rng(77)
    V, B = 65536, 12
    rows = []
    for b in range(B):
        kind = b % 6
        if kind == 0:
            r = np.repeat(g.normal(0, 3, V // 4), 4)
        elif kind == 1:
            r = np.repeat(g.normal(0, 3, V // 16), 16)
        elif kind == 2:
            r = np.repeat(g.normal(0, 3, V // 256), 256) + g.normal(0, 0.01, V)
        elif kind == 3:
            r = g.normal(0, 3, V)  # control: no clustering
        elif kind == 4:
            r = np.sort(g.normal(0, 3, V))
        else:
            r = np.sort(g.normal(0, 3, V))[::-1].copy()
        rows.append(r)
    x = np.stack(rows).astype(np.float32)
    # nuclei that fit the slots (top_p 0.95 over N(0, 3^2) rows would need
    # ~1440 candidates a chunk: the general pipeline with either threshold)
    params = [SamplingParams(top_p=[0.9, 0.8, 0.5][b % 3], repetition_penalty=1.0 if b < 6 else 1.2) for b in range(B)]
    ctx = [list(g.integers(0, V, 200)) for _ in range(B)]
    u = g.random(B)
    c = _native.default_context()
    block_rows = [b for b in range(B) if b % 6 in (0, 1, 2, 3)]
    f0 = c.fallback_rows()
    ids_blocks = sample_batch(x[block_rows], [params[b] for b in block_rows], uniforms=u[block_rows],
                              contexts=[ctx[b] for b in block_rows])
    f1 = c.fallback_rows()
    ids = sample_batch(x, params, uniforms=u, contexts=ctx)
    f2 = c.fallback_rows()
    _check(x, params, u, ctx, ids)
    assert list(ids_blocks) == [int(ids[b]) for b in block_rows]
    print(f"clustered rows: general-path rows {f1 - f0} of {len(block_rows)} block rows, {f2 - f1} of {B} in all",
          flush=True)
    assert f1 - f0 == 0
