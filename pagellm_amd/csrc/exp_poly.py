"""Derives the constants of the normaliser exp in plh_fast.h.

* kExpCheb4: the degree-4 polynomial interpolating exp at the five
  Chebyshev nodes of [-ln2/128, ln2/128] (near-minimax: relative error
  2.4e-15 there, against 3.9e-14 for the degree-4 Taylor polynomial),
  solved in 80-bit long double and rounded to double.  Its constant term
  rounds to exactly 1.
* kLn2Over64: ln2 / 64 rounded to double.
* the 2^(j/64) table, each entry correctly rounded.

Run it to print the constants: python pagellm_amd/csrc/exp_poly.py
"""

from __future__ import annotations

import numpy as np

LD = np.longdouble


def cheb4() -> list[float]:
    a = LD(np.log(LD(2))) / 128
    n = 5
    nodes = [a * np.cos((2 * LD(i) + 1) * LD(np.pi) / (2 * n)) for i in range(n)]
    A = [[x ** j for j in range(n)] for x in nodes]
    b = [np.exp(x) for x in nodes]
    for i in range(n):  # Gaussian elimination with partial pivoting, in long double
        p = max(range(i, n), key=lambda r: abs(A[r][i]))
        A[i], A[p], b[i], b[p] = A[p], A[i], b[p], b[i]
        for r in range(i + 1, n):
            m = A[r][i] / A[i][i]
            A[r] = [A[r][k] - m * A[i][k] for k in range(n)]
            b[r] -= m * b[i]
    c = [LD(0)] * n
    for i in reversed(range(n)):
        c[i] = (b[i] - sum(A[i][k] * c[k] for k in range(i + 1, n))) / A[i][i]
    return [float(x) for x in c]


def ln2_over_64() -> float:
    return float(np.log(LD(2)) / 64)


def exp2_table() -> list[float]:
    return [float(np.exp2(LD(j) / 64)) for j in range(64)]


if __name__ == "__main__":
    c = cheb4()
    print("constant term:", c[0].hex())
    print("kExpCheb4 (r^1..r^4):", ", ".join(x.hex() for x in c[1:]))
    print("kLn2Over64:", ln2_over_64().hex())
