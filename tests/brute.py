"""Pure-Python brute force of the sampler and verify rules, used to pin the
numpy oracle on small inputs.

Written from the reference's rules (``sampling.py:52-111``,
``speculative.py:38-60``) with different primitives from the oracle: Python
lists, full ``sorted`` orders instead of ``np.partition``/``np.argsort``,
``math.exp``, ``math.fsum`` (exactly rounded sums) and explicit linear scans
for the inverse CDF.  Only the running sums that the reference defines as a
left-to-right ``cumsum`` are kept sequential.
"""

from __future__ import annotations

import math


def penalize(x, context, penalty):
    x = [float(v) for v in x]
    if penalty == 1.0 or len(context) == 0:
        return x
    V = len(x)
    for i in sorted(set(int(c) for c in context)):
        j = i + V if i < 0 else i  # numpy fancy-index wrap for negatives
        v = x[j]
        x[j] = v / penalty if v > 0 else v * penalty
    return x


def argmax_lowest(x):
    best = 0
    for i in range(1, len(x)):
        if x[i] > x[best]:
            best = i
    return best


def probs(logits, T, top_k=0, top_p=1.0, penalty=1.0, context=()):
    x = penalize(logits, context, penalty)
    V = len(x)
    if T == 0:
        p = [0.0] * V
        p[argmax_lowest(x)] = 1.0
        return p
    y = [v / T for v in x]
    if 0 < top_k < V:
        kth = sorted(y, reverse=True)[top_k - 1]
        y = [v if v >= kth else -math.inf for v in y]
    m = max(y)
    e = [math.exp(v - m) for v in y]
    s = math.fsum(e)
    p = [v / s for v in e]
    if top_p < 1.0:
        order = sorted(range(V), key=lambda i: (-p[i], i))
        run = 0.0
        kept = [False] * V
        for i in order:
            run = run + p[i]
            if run - p[i] < top_p:
                kept[i] = True
        p = [p[i] if kept[i] else 0.0 for i in range(V)]
        s2 = math.fsum(p)
        p = [v / s2 for v in p]
    return p


def draw(p, u):
    c = []
    run = 0.0
    for v in p:
        run = run + v
        c.append(run)
    t = u * c[-1]
    for i, ci in enumerate(c):
        if ci > t:
            return i
    return len(p) - 1


def verify(p_rows, q_rows, draft, uniforms):
    """``uniforms`` is consumed left to right: one per accept test, then one
    for the final draw."""
    it = iter(uniforms)
    out = []
    for i, x in enumerate(draft):
        p, q = p_rows[i], q_rows[i]
        r = p[x] / q[x]
        thr = r if r < 1.0 else 1.0
        if next(it) < thr:
            out.append(x)
            continue
        resid = [max(a - b, 0.0) for a, b in zip(p, q)]
        s = math.fsum(resid)
        dist = [v / s for v in resid] if s > 0 else list(p)
        out.append(draw(dist, next(it)))
        return out, i
    out.append(draw(p_rows[len(draft)], next(it)))
    return out, len(draft)
