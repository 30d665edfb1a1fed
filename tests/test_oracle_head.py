"""Pins the logits-producer oracle (``oracle/head.py``) on the CPU."""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle


def _brute(h, norm, W, eps):
    """float64 loops with math.fsum / math.sqrt: rms_norm then the product."""
    N, D = len(h), len(h[0])
    V = len(W[0])
    out = []
    for n in range(N):
        ms = math.fsum(float(x) * float(x) for x in h[n]) / D
        r = 1.0 / math.sqrt(ms + eps)
        a = [float(h[n][d]) * r * float(norm[d]) for d in range(D)]
        out.append([math.fsum(a[d] * float(W[d][v]) for d in range(D)) for v in range(V)])
    return np.array(out)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_matches_float64_brute_force(seed):
    g = np.random.default_rng(seed)
    N, D, V = 3, 24, 7
    h = g.standard_normal((N, D)).astype(np.float32)
    norm = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
    W = (0.05 * g.standard_normal((D, V))).astype(np.float32)
    got = oracle.lm_head_logits(h, norm, W, 1e-5)
    ref = _brute(h, norm, W, 1e-5)
    bound = oracle.head_error_bound(h, norm, W, 1e-5)
    assert got.dtype == np.float32
    assert np.all(np.abs(got - ref) <= 1e-6 * bound + 1e-12)


def test_constant_rows_closed_form():
    """h[n] = c everywhere, norm = 1, W = I: logits = c / sqrt(c^2 + eps)."""
    D = 16
    cs = np.array([1.0, -3.0, 0.01, 1e-3], dtype=np.float32)
    h = np.repeat(cs[:, None], D, axis=1)
    got = oracle.lm_head_logits(h, np.ones(D), np.eye(D), 1e-5)
    want = cs.astype(np.float64) / np.sqrt(cs.astype(np.float64) ** 2 + 1e-5)
    assert np.allclose(got, want[:, None], rtol=1e-6, atol=0)


def test_eps_is_added_inside_the_root():
    """Rows of norm ~1e-3 are visibly shrunk by eps = 1e-5 (and not by eps = 0)."""
    g = np.random.default_rng(5)
    D = 32
    h = (1e-3 * g.standard_normal((2, D))).astype(np.float32)
    a0 = oracle.rms_norm(h, np.ones(D, np.float32), 0.0)
    a1 = oracle.rms_norm(h, np.ones(D, np.float32), 1e-5)
    assert np.allclose(np.mean(a0.astype(np.float64) ** 2, axis=1), 1.0, rtol=1e-5)
    ms = np.mean(h.astype(np.float64) ** 2, axis=1)
    assert np.allclose(np.mean(a1.astype(np.float64) ** 2, axis=1), ms / (ms + 1e-5), rtol=1e-5)


def test_power_of_two_row_scaling_is_exact():
    """Scaling one row by 4 leaves every logit bit-identical (eps = 0), and
    leaves the other rows alone: the mean is over each row's own entries."""
    g = np.random.default_rng(9)
    N, D, V = 4, 64, 33
    h = g.standard_normal((N, D)).astype(np.float32)
    norm = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
    W = g.standard_normal((D, V)).astype(np.float32)
    base = oracle.lm_head_logits(h, norm, W, 0.0)
    h2 = h.copy()
    h2[1] *= 4
    assert np.array_equal(oracle.lm_head_logits(h2, norm, W, 0.0), base)
    assert np.array_equal(oracle.rms_norm(h2, norm, 0.0)[0], oracle.rms_norm(h, norm, 0.0)[0])
