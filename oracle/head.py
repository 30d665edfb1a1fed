"""CPU oracle for the logits producer: test infrastructure only.

TEST INFRASTRUCTURE ONLY: the expected results for ``plh_rmsnorm_lm_head``; the
product never imports it.

A numpy restatement of the model's last two operations,
``rms_norm(h, norm, eps) @ lm_head`` (``src/pagellm/model/transformer.py:271``)
with ``rms_norm`` as at ``:79-82``: ``r = 1 / sqrt(mean(x * x) + eps)``,
``x * r * weight``, all in the arrays' float32 (numpy 2 treats the Python
floats ``eps`` and ``1.0`` as weak scalars, so nothing promotes to float64),
then a float32 matrix product.  ``head_error_bound`` is the scale parity
tests measure float32 rounding against: ``|rms_norm(h)| @ |lm_head|``
computed in float64.

Pinned by ``tests/test_oracle_head.py`` against a pure-Python float64 brute
force (``math.fsum``, ``math.sqrt``, explicit loops), the closed form for
constant rows, exact invariance under power-of-two scaling of one row, and
the eps term's effect on rows of tiny norm.
"""

from __future__ import annotations

import numpy as np


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """transformer.py:79-82."""
    x = np.asarray(x)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r * weight


def lm_head_logits(h: np.ndarray, norm: np.ndarray, lm_head: np.ndarray, eps: float) -> np.ndarray:
    """transformer.py:271, float32 in and out."""
    h = np.asarray(h, dtype=np.float32)
    return rms_norm(h, np.asarray(norm, dtype=np.float32), eps) @ np.asarray(lm_head, dtype=np.float32)


def head_error_bound(h: np.ndarray, norm: np.ndarray, lm_head: np.ndarray, eps: float) -> np.ndarray:
    """sum_d |a[n, d]| |W[d, v]| in float64, a = rms_norm(h): the magnitude a
    float32 dot product's rounding error scales with."""
    a = np.abs(rms_norm(np.asarray(h, dtype=np.float64), np.asarray(norm, dtype=np.float64), eps))
    return a @ np.abs(np.asarray(lm_head, dtype=np.float64))
