"""The normaliser exp of the fast path (plh_fast.h exp_neg_term): its
constants are the ones pagellm_amd/csrc/exp_poly.py derives, and its
reduction + polynomial + table, evaluated in long double with those double
constants, stay within 6e-15 relative of exp on d in [-40, 0] (the kernel's
own double roundings add about 2 ulp)."""

from __future__ import annotations

import importlib.util
import re
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
HDR = (ROOT / "pagellm_amd" / "csrc" / "plh_fast.h").read_text()
_spec = importlib.util.spec_from_file_location("exp_poly", ROOT / "pagellm_amd" / "csrc" / "exp_poly.py")
exp_poly = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(exp_poly)
LD = np.longdouble


def _hexes(block: str) -> list[float]:
    return [float.fromhex(h) for h in re.findall(r"0x1\.[0-9a-f]+p[+-]\d+", block)]


def _consts():
    cheb = _hexes(HDR[HDR.index("kExpCheb4[4] = {"):HDR.index("};", HDR.index("kExpCheb4[4] = {"))])
    ln2 = _hexes(HDR[HDR.index("kLn2Over64 ="):HDR.index(";", HDR.index("kLn2Over64 ="))])[0]
    tab = _hexes(HDR[HDR.index("kExp2Frac64[64] = {"):HDR.index("};", HDR.index("kExp2Frac64[64] = {"))])
    return cheb, ln2, tab


def test_constants_match_their_derivation():
    cheb, ln2, tab = _consts()
    want = exp_poly.cheb4()
    assert want[0] == 1.0
    assert cheb == want[1:]
    assert ln2 == exp_poly.ln2_over_64()
    assert len(tab) == 64 and tab == exp_poly.exp2_table()


def _exp_neg_term_ld(d: np.ndarray) -> np.ndarray:
    cheb, ln2, tab = _consts()
    d = np.maximum(d.astype(LD), LD(-708.0))
    k = np.rint(d * LD(64.0 / 0.6931471805599453)).astype(np.int64)
    r = d - k.astype(LD) * LD(ln2)
    q = LD(cheb[3])
    for c in (cheb[2], cheb[1], cheb[0], 1.0):
        q = q * r + LD(c)
    return np.ldexp(np.asarray(tab, dtype=LD)[k & 63] * q, (k >> 6).astype(np.int32))


def test_relative_error_on_the_terms_a_normaliser_notices():
    d = np.concatenate([np.linspace(-40.0, 0.0, 400001), -np.logspace(-12, np.log10(40.0), 20001)])
    got = _exp_neg_term_ld(d)
    want = np.exp(d.astype(LD))
    rel = np.max(np.abs(got / want - 1))
    assert rel < 6e-15, float(rel)


def test_deep_terms_and_minus_inf():
    d = np.array([-100.0, -500.0, -707.9, -708.0, -1e4, -np.inf])
    got = _exp_neg_term_ld(d)
    assert np.all(got > 0) and np.all(np.isfinite(got))
    assert np.all(got[3:] == got[3])  # clamped at -708
    assert abs(float(got[0] / np.exp(LD(-100.0))) - 1) < 2e-14
