"""Shared parity bars for the GPU tests.

The kernels build each row's CDF in 2^-62 fixed point from float64
exponentials, so their draw position differs from numpy's float64
``cumsum`` by less than V * 2^-62 + V * 1e-16 of the row mass, about 3e-14 at
V = 152 064. The tests therefore hold ids to a 1e-12 band:

* a sampled id may differ from the oracle's only if the uniform lies within
  ``DRAW_GAP`` = 1e-12 of a CDF boundary, or the row's top-p cut lies within
  ``TOPP_GAP`` = 1e-12 of flipping (both measured by the oracle's gauges,
  ``sampling.py:94-98`` and ``:84-92``);
* speculative accept/resample decisions are held to the same 1e-12 band;
* rows whose uniform lies within ``BAND`` = 1e-6 of a CDF boundary are
  counted and printed (the count the 1e-6 boundary rule reports), whether or
  not the ids agree.
"""

from __future__ import annotations

import oracle
from oracle.sampler import sample_boundary_gaps

TOPP_GAP = 1e-12
DRAW_GAP = 1e-12
BAND = 1e-6


def compare_rows(w, rows, ids, label):
    """Checks GPU ids against the oracle on the given rows of a workload
    dict. Returns (mismatches, rows in the 1e-6 band)."""
    mism = band = 0
    for r in rows:
        prm, x, ctx, u = w["params"][r], w["logits"][r], w["contexts"][r], w["uniforms"][r]
        ref = oracle.sample(x, prm, u, ctx)
        if prm.greedy:
            assert ids[r] == ref, (label, r)
            continue
        g_topp, g_draw = sample_boundary_gaps(x, prm, u, ctx)
        if g_draw < BAND:
            band += 1
        if ids[r] != ref:
            assert g_topp < TOPP_GAP or g_draw < DRAW_GAP, (label, r, int(ids[r]), ref, g_topp, g_draw)
            mism += 1
    print(f"[{label}] rows checked {len(rows)}, mismatches {mism} (all within 1e-12), "
          f"rows within 1e-6 of a CDF boundary {band}", flush=True)
    return mism, band
