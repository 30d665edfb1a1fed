"""GPU parity at the configurations' real sizes, and draw() id for id.

* ``draw`` (``sampling.py:94-98``): the draw kernel against the oracle's
  ``searchsorted(cumsum(p), u * c[-1], side="right")`` clamped to V - 1, on
  the same uniforms, at vocabulary sizes from 65 to 152 064, float64 and
  float32 rows (a float32 row is compared with the oracle on its exact
  float64 widening, the arithmetic the kernel uses), plus the edges: u * c[-1]
  exactly on a boundary c_i, zero-mass prefixes and tails, all-zero rows,
  u = 0 and u = nextafter(1, 0).
* mixed128k: every one of the 256 rows against the oracle.
* zipf152k at its stated batch of 1024 rows: 256 rows spread over the batch
  against the oracle, every row in range, the fallback count reported.

Ids may differ only where the oracle's boundary gauges put the uniform
within 1e-12 of a CDF boundary or the top-p cut within 1e-12 of flipping;
each such row is counted and printed, and so is every row whose uniform lies
within 1e-6 of a boundary.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from parity import DRAW_GAP, BAND
from parity import compare_rows as _compare_rows
from pagellm_amd import _native, workloads
from pagellm_amd.sampling import draw_batch, sample_batch

pytestmark = pytest.mark.gpu


def _check_draws(p, u, label):
    ids = draw_batch(p, u)
    p64 = p.astype(np.float64)
    mism = band = 0
    for b in range(p.shape[0]):
        ref = oracle.draw(p64[b], float(u[b]))
        gap = oracle.draw_boundary_gap(p64[b], float(u[b]))
        band += gap < BAND
        if ids[b] != ref:
            assert gap < DRAW_GAP, (label, b, int(ids[b]), ref, gap)
            mism += 1
    print(f"[{label}] draws {p.shape[0]}, mismatches {mism}, within 1e-6 of a boundary {band}", flush=True)
    return ids


def _rows(g, B, V, kind):
    if kind == "softmax":
        x = g.normal(0, 2, (B, V))
        e = np.exp(x - x.max(axis=1, keepdims=True))
        return e / e.sum(axis=1, keepdims=True)
    if kind == "unnormalised":  # draw() normalises by c[-1] itself
        return g.gamma(0.3, 5.0, (B, V))
    if kind == "sparse":
        p = g.random((B, V)) * (g.random((B, V)) < 0.01)
        p[:, g.integers(0, V)] += 0.5
        return p
    raise ValueError(kind)


@pytest.mark.parametrize("V", [65, 4097, 32000, 128256, 152064])
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_draw_matches_oracle_id_for_id(V, dtype):
    g = np.random.default_rng(V + (dtype == np.float32))
    for kind in ("softmax", "unnormalised", "sparse"):
        B = 24
        p = _rows(g, B, V, kind).astype(dtype)
        u = g.random(B)
        u[:3] = [0.0, np.nextafter(1.0, 0.0), 0.5]
        _check_draws(p, u, f"draw {kind} V={V} {np.dtype(dtype).name}")


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_draw_edges_exact(dtype):
    """Cases whose answer the arithmetic fixes exactly (dyadic weights, so
    every running sum and u * c[-1] are exact): the kernel must return the
    oracle's id with no boundary excuse."""
    g = np.random.default_rng(5)
    rows, us = [], []
    V = 4096
    # u * c[-1] exactly equal to c_i: side="right" skips past token i (and
    # past the zero-weight tokens after it)
    w = g.integers(0, 5, V).astype(np.float64)  # zeros included
    w[[0, 17, 2000]] = [3, 0, 0]
    total = 2.0 ** int(np.ceil(np.log2(w.sum() + 1)))
    w[V - 1] += total - w.sum()  # the total is a power of two: p = w / total is exact
    c = np.cumsum(w)
    for i in (0, 16, 17, 1999, 2000, V // 2, V - 2):
        rows.append(w / total)
        us.append(c[i] / total)  # exact, and u * c[-1] = c_i exactly
    # zero-mass prefix and tail (eight tokens of weight 1, total 8), u at
    # both ends, on a boundary and between boundaries
    z = np.zeros(V)
    z[1000:1008] = 1.0
    for u in (0.0, np.nextafter(1.0, 0.0), 0.5, 0.1, 0.9):
        rows.append(z)
        us.append(u)
    # all-zero rows: c[-1] = 0, searchsorted(..., 0, right) = V, clamped to V - 1
    for u in (0.0, 0.5, np.nextafter(1.0, 0.0)):
        rows.append(np.zeros(V))
        us.append(u)
    # one positive token at either end
    for pos in (0, V - 1):
        one = np.zeros(V)
        one[pos] = 0.25
        for u in (0.0, 0.75, np.nextafter(1.0, 0.0)):
            rows.append(one)
            us.append(u)
    p = np.stack(rows).astype(dtype)
    u = np.array(us)
    ids = draw_batch(p, u)
    for b in range(len(rows)):
        assert ids[b] == oracle.draw(p[b].astype(np.float64), float(u[b])), (b, int(ids[b]))


def test_mixed128k_every_row():
    w = workloads.mixed128k()
    c = _native.default_context()
    before = c.fallback_rows()
    ids = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    print(f"mixed128k rows finished by the general path: {c.fallback_rows() - before}", flush=True)
    _compare_rows(w, range(256), ids, "mixed128k all rows")


def test_zipf152k_at_its_batch_of_1024():
    w = workloads.zipf152k(rows=1024)
    assert w["logits"].shape == (1024, 152064)
    c = _native.default_context()
    before = c.fallback_rows()
    ids = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    print(f"zipf152k x1024 rows finished by the general path: {c.fallback_rows() - before}", flush=True)
    assert ids.shape == (1024,) and np.all((ids >= 0) & (ids < 152064))
    _compare_rows(w, range(0, 1024, 4), ids, "zipf152k x1024")


def test_unaligned_vocabulary_50257():
    """V = 50 257, an odd vocabulary: host rows go over with their stride
    padded to 16 bytes and take the 128-bit load path; a device tensor with
    stride V takes the element-wise path.  Both against the oracle on every
    row, and against each other."""
    import torch

    w = workloads.mixed128k(rows=64, V=50257)
    ids = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    _compare_rows(w, range(64), ids, "mixed V=50257 padded")
    dev = torch.from_numpy(w["logits"]).to("cuda:0")
    assert dev.stride(0) == 50257
    ids_dev = sample_batch(dev, w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    assert np.array_equal(ids, ids_dev)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_small_batch_at_a_large_vocabulary(dtype):
    """16 rows of the mixed batch (V = 128 256): 128 chunk workgroups (float32)
    or 256 (float64), fewer than the chip holds at once.  Every row against
    the oracle."""
    w = workloads.mixed128k(rows=16)
    w["logits"] = w["logits"].astype(dtype)
    ids = sample_batch(w["logits"], w["params"], uniforms=w["uniforms"], contexts=w["contexts"])
    _compare_rows(w, range(16), ids, f"mixed128k x16 {np.dtype(dtype).name}")
