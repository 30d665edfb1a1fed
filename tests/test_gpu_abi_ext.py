"""The history-span form of plh_sample, plh_append_ids and plh_copy_rows
(needs an MI355X): spans give the same ids as CSR offsets over the same
histories (overlapping and empty spans included); the append skips negative
positions; the strided copy places [B, V] blocks."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from pagellm_amd import _native
from parity import DRAW_GAP, TOPP_GAP
from pagellm_amd.params import SamplingParams
from pagellm_amd.sampling import _pack_params

pytestmark = pytest.mark.gpu


def _sample(c, x, params, u, hist_ids, hist_off, flags):
    B, V = x.shape
    t, k, p, r = _pack_params(params)
    d = {n: c.to_device(a) for n, a in dict(x=x, t=t, k=k, p=p, r=r, u=u).items()}
    hi = c.to_device(hist_ids)
    ho = c.to_device(hist_off)
    out = c.empty((B,), np.int32)
    c.sample(d["x"].ptr, _native.dtype_code(x.dtype), V, B, V, hi.ptr, ho.ptr, d["t"].ptr, d["k"].ptr, d["p"].ptr,
             d["r"].ptr, d["u"].ptr, out.ptr, None, flags)
    return out.download()


@pytest.mark.parametrize("rowwise", [False, True])
def test_spans_match_csr(rowwise):
    g = np.random.default_rng(3)
    B, V = 12, 30000
    x = g.normal(0, 2, (B, V)).astype(np.float32)
    hists = [list(g.integers(0, V, g.integers(0, 400))) for _ in range(B)]
    hists[3] = []
    hists[5] = list(hists[4])  # same ids as row 4
    params = [SamplingParams(temperature=[0.0, 1.0, 0.8][b % 3], top_k=[0, 40][b % 2], top_p=[1.0, 0.9][b % 2],
                             repetition_penalty=1.3) for b in range(B)]
    u = g.random(B)
    off = np.zeros(B + 1, dtype=np.int64)
    for b in range(B):
        off[b + 1] = off[b] + len(hists[b])
    ids = np.concatenate([np.asarray(h, dtype=np.int32) for h in hists])
    # spans: rows 4 and 5 share one stored copy; the slab has gaps
    slab, spans = [], np.zeros(2 * B, dtype=np.int64)
    for b in range(B):
        if b == 5:
            spans[10], spans[11] = spans[8], spans[9]
            continue
        slab.extend([0] * 7)  # unused ids between histories
        spans[2 * b] = len(slab)
        slab.extend(hists[b])
        spans[2 * b + 1] = len(slab)
    slab = np.asarray(slab, dtype=np.int32)
    c = _native.Context(0)
    flags = _native.PLH_SAMPLE_ROWWISE if rowwise else 0
    a = _sample(c, x, params, u, ids, off, flags)
    s = _sample(c, x, params, u, slab, spans, flags | _native.PLH_SAMPLE_HIST_SPANS)
    assert np.array_equal(a, s)
    for b in range(B):
        assert s[b] == oracle.sample(x[b], params[b], u[b], hists[b]), b
    c.close()


def test_append_ids_and_copy_rows():
    c = _native.Context(0)
    slab = c.to_device(np.full(16, -7, dtype=np.int32))
    pos = c.to_device(np.array([3, -1, 0, 15], dtype=np.int64))
    ids = c.to_device(np.array([30, 31, 32, 33], dtype=np.int32))
    c.append_ids(slab.ptr, pos.ptr, ids.ptr, 4)
    got = slab.download()
    want = np.full(16, -7, dtype=np.int32)
    want[[3, 0, 15]] = [30, 32, 33]
    assert np.array_equal(got, want)
    B, k, V = 3, 4, 5
    src = np.arange(B * V, dtype=np.float64).reshape(B, V)
    d_src = c.to_device(src)
    dst = c.to_device(np.zeros((B, k, V)))
    c.copy_rows(dst.ptr + 8 * 2 * V, 8 * k * V, d_src.ptr, 8 * V, 8 * V, B)
    out = dst.download()
    assert np.array_equal(out[:, 2], src)
    assert not out[:, [0, 1, 3]].any()
    c.close()


def test_quantized_logits_general_path():
    """bf16-like logits (8 mantissa bits): long runs of equal values at the
    top-k and top-p cuts, through the row-wise general pipeline."""
    g = np.random.default_rng(9)
    B, V = 16, 50000
    x = g.normal(0, 2, (B, V))
    m, e = np.frexp(x)
    x = np.ldexp(np.round(m * 256) / 256, e).astype(np.float32)
    params = [SamplingParams(temperature=1.0, top_p=[0.5, 0.9, 0.99, 0.999][b % 4], top_k=[0, 0, 1000, 0][b % 4])
              for b in range(B)]
    u = g.random(B)
    c = _native.Context(0)
    t, k, p, r = _pack_params(params)
    d = {n: c.to_device(a) for n, a in dict(x=x, t=t, k=k, p=p, r=r, u=u).items()}
    out = c.empty((B,), np.int32)
    c.sample(d["x"].ptr, _native.PLH_F32, V, B, V, None, None, d["t"].ptr, d["k"].ptr, d["p"].ptr, d["r"].ptr,
             d["u"].ptr, out.ptr, None, _native.PLH_SAMPLE_ROWWISE)
    ids = out.download()
    from oracle.sampler import sample_boundary_gaps
    for b in range(B):
        ref = oracle.sample(x[b], params[b], u[b], ())
        if ids[b] != ref:
            gt, gd = sample_boundary_gaps(x[b], params[b], u[b], ())
            assert gt < TOPP_GAP or gd < DRAW_GAP, (b, int(ids[b]), ref)
    c.close()


def test_pinned_staging_and_queued_copy():
    """plh_host_alloc / plh_h2d_async: bytes staged in page-locked memory
    arrive intact once the stream has passed the copy (the next download),
    at an offset inside a larger device buffer, and a grown staging buffer
    keeps working."""
    c = _native.Context(0)
    try:
        g = np.random.default_rng(3)
        for n in (16, 5000, 70000):
            src = g.integers(0, 256, n, dtype=np.uint8)
            stage = c.pinned("t", n)
            stage[:n] = src
            dev = c.empty((n + 64,), np.uint8)
            c.h2d_async(dev.ptr + 64, stage[:n])
            got = np.empty(n, dtype=np.uint8)
            c._check(c.lib.plh_d2h(c.handle, got.ctypes.data, dev.ptr + 64, n))
            assert np.array_equal(got, src), n
            dev.free()
    finally:
        c.close()


def test_nucleus_hint_changes_the_path_not_the_ids():
    """PLH_SAMPLE_NUCLEUS only moves rows with no top-k and top_p >= 0.98
    from the general pipeline to the nucleus kernels: the same batch (a
    Zipf-like row set mixed with greedy, top-k and plain top-p rows, CSR and
    span histories) gives the same ids with and without it, and only
    without it do the high-top_p rows fall back.  PLH_SAMPLE_NUCLEUS_ONLY
    (no merge launch) gives them too, right or wrong."""
    g = np.random.default_rng(8)
    B, V = 10, 60000
    ranks = 1 + np.stack([g.permutation(V) for _ in range(B)])
    x = (-np.log(ranks) + g.normal(0, 0.3, (B, V))).astype(np.float32)
    params = [SamplingParams(top_p=0.99, repetition_penalty=1.05)] * 6 + [
        SamplingParams(temperature=0.0), SamplingParams(top_k=50), SamplingParams(top_p=0.9),
        SamplingParams(top_p=0.995, temperature=0.8)]
    u = g.random(B)
    hists = [g.integers(0, V, 700).astype(np.int32) for _ in range(B)]
    ids = np.concatenate(hists)
    off = np.concatenate([[0], np.cumsum([h.size for h in hists])]).astype(np.int64)
    c = _native.Context(0)
    f0 = c.fallback_rows()
    plain = _sample(c, x, params, u, ids, off, 0)
    f1 = c.fallback_rows()
    hinted = _sample(c, x, params, u, ids, off, _native.PLH_SAMPLE_NUCLEUS)
    f2 = c.fallback_rows()
    assert np.array_equal(plain, hinted)
    # the seven top_p >= 0.98 rows leave the general pipeline; the top_p 0.9
    # row (a nucleus too wide for the candidate slots) falls back either way
    assert (f1 - f0) - (f2 - f1) == 7, (f1 - f0, f2 - f1)
    spans = np.stack([off[:-1], off[1:]], axis=1).reshape(-1)
    assert np.array_equal(hinted, _sample(c, x, params, u, ids, spans,
                                          _native.PLH_SAMPLE_NUCLEUS | _native.PLH_SAMPLE_HIST_SPANS))
    for b in range(B):
        ref = oracle.sample(x[b], params[b], u[b], hists[b])
        assert hinted[b] == ref or min(oracle.sampler.sample_boundary_gaps(x[b], params[b], u[b], hists[b])) < DRAW_GAP
    # PLH_SAMPLE_NUCLEUS_ONLY: no merge launch.  Given wrongly (the greedy,
    # top-k and top_p 0.9 rows are not nucleus rows), those three rows are
    # finished by the general pipeline in the nucleus path: the same ids
    f3 = c.fallback_rows()
    only = _sample(c, x, params, u, ids, off, _native.PLH_SAMPLE_NUCLEUS | _native.PLH_SAMPLE_NUCLEUS_ONLY)
    f4 = c.fallback_rows()
    assert np.array_equal(only, hinted)
    assert f4 - f3 == 3, f4 - f3
    # and given rightly, on the seven nucleus rows alone: the hinted ids
    nuc = [b for b in range(B) if b < 6 or b == 9]
    sub_ids = np.concatenate([hists[b] for b in nuc])
    sub_off = np.concatenate([[0], np.cumsum([hists[b].size for b in nuc])]).astype(np.int64)
    sub = _sample(c, x[nuc], [params[b] for b in nuc], u[nuc], sub_ids, sub_off,
                  _native.PLH_SAMPLE_NUCLEUS | _native.PLH_SAMPLE_NUCLEUS_ONLY)
    assert np.array_equal(sub, hinted[nuc])
    assert c.fallback_rows() == f4


def test_penalize_rejects_in_place_and_overlapping_output():
    """plh_penalize works on a copy (sampling.py:58): an output that overlaps
    the input is an invalid argument, and a disjoint one is penalised once
    per distinct id even when the history repeats ids."""
    c = _native.default_context()
    V, B = 1000, 2
    g = np.random.default_rng(8)
    x = g.normal(0, 2, (B, V)).astype(np.float32)
    ids = np.array([5, 5, 5, 7, 999, 5, 7], dtype=np.int32)
    off = np.array([0, 7, 7], dtype=np.int64)
    pen = np.array([1.5, 1.5])
    d_x = c.to_device(x)
    d_ids, d_off, d_pen = c.to_device(ids), c.to_device(off), c.to_device(pen)
    with pytest.raises(ValueError, match="overlap"):
        c.penalize(d_x.ptr, _native.PLH_F32, V, B, V, d_ids.ptr, d_off.ptr, d_pen.ptr, d_x.ptr, V)
    with pytest.raises(ValueError, match="overlap"):  # shifted by one element into row 0
        c.penalize(d_x.ptr, _native.PLH_F32, V, B, V, d_ids.ptr, d_off.ptr, d_pen.ptr, d_x.ptr + 4, V)
    d_o = c.empty((B, V), np.float32)
    c.penalize(d_x.ptr, _native.PLH_F32, V, B, V, d_ids.ptr, d_off.ptr, d_pen.ptr, d_o.ptr, V)
    got = d_o.download()
    assert np.array_equal(got[0], oracle.apply_repetition_penalty(x[0], ids.tolist(), 1.5))
    assert np.array_equal(got[1], x[1])
    assert np.array_equal(d_x.download(), x)  # the input is untouched
    # interleaved rows of one buffer never touch: x = buf[:, :V], out = buf[:, V:2V]
    buf = np.concatenate([x, np.zeros_like(x)], axis=1)
    d_buf = c.to_device(buf)
    c.penalize(d_buf.ptr, _native.PLH_F32, 2 * V, B, V, d_ids.ptr, d_off.ptr, d_pen.ptr, d_buf.ptr + 4 * V, 2 * V)
    both = d_buf.download()
    assert np.array_equal(both[:, :V], x) and np.array_equal(both[:, V:], got)
    with pytest.raises(ValueError, match="overlap"):  # out's row 0 reaches one element into x's row 1
        c.penalize(d_buf.ptr, _native.PLH_F32, 2 * V, B, V, d_ids.ptr, d_off.ptr, d_pen.ptr,
                   d_buf.ptr + 4 * (V + 1), 2 * V)


def _launch_rows(c, w, rows=None):
    """plh_sample on the context's current stream, not waited for: the
    device ids (their inputs kept alive with them)."""
    from pagellm_amd.sampling import _nucleus_hint, _pack_histories

    x = w["logits"] if rows is None else w["logits"][:rows]
    params = w["params"] if rows is None else w["params"][:rows]
    ctxs = w["contexts"] if rows is None else w["contexts"][:rows]
    u = w["uniforms"] if rows is None else w["uniforms"][:rows]
    B, V = x.shape
    t, k, p, r = _pack_params(params)
    hist_ids, hist_off = _pack_histories(ctxs, params, B, V)
    d = {n: c.to_device(a) for n, a in dict(x=x, t=t, k=k, p=p, r=r, u=u).items()}
    hi = c.to_device(hist_ids) if hist_ids is not None else None
    ho = c.to_device(hist_off) if hist_off is not None else None
    out = c.empty((B,), np.int32)
    c.sample(d["x"].ptr, _native.dtype_code(x.dtype), V, B, V, hi.ptr if hi else None, ho.ptr if ho else None,
             d["t"].ptr, d["k"].ptr, d["p"].ptr, d["r"].ptr, d["u"].ptr, out.ptr, None, _nucleus_hint(t, k, p, V))
    out.keep = (d, hi, ho)
    return out


def test_workspace_calls_on_changing_streams():
    """plh_sample calls of one context share its workspace.  Calls on one
    stream record no event; moving to another stream closes the calls on
    the stream left, and the next call waits for them.  Back-to-back calls
    with no host wait, switching streams between them (and once right after
    the workspace grew), return the ids of calls made one at a time."""
    import torch

    from pagellm_amd import workloads

    c = _native.Context(0)
    try:
        small, big = workloads.zipf32k(), workloads.mixed128k()
        ref_small = _launch_rows(c, small, rows=48).download()
        ref_big = _launch_rows(c, big).download()
        c.close()
        c = _native.Context(0)  # a fresh context: its workspace grows on the way
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        outs = []
        c.set_stream(s1.cuda_stream)
        outs.append((_launch_rows(c, small, rows=48), ref_small))
        outs.append((_launch_rows(c, small, rows=48), ref_small))  # same stream: no event
        c.set_stream(s2.cuda_stream)
        outs.append((_launch_rows(c, big), ref_big))  # grows the workspace after s1's calls
        c.set_stream(s1.cuda_stream)
        outs.append((_launch_rows(c, small, rows=48), ref_small))
        c.set_stream(None)
        outs.append((_launch_rows(c, big), ref_big))
        c.set_stream(s2.cuda_stream)
        outs.append((_launch_rows(c, small, rows=48), ref_small))
        torch.cuda.synchronize()
        for i, (o, ref) in enumerate(outs):
            assert np.array_equal(o.download(), ref), i
    finally:
        c.set_stream(None)
        c.close()


def test_workspace_users_interleaved_on_streams():
    """plh_sample, plh_verify and plh_rmsnorm_lm_head share the context's
    workspace (each grows it to its own size).  Interleaved over three
    streams with no host wait between the calls, every result equals the
    same call made alone on one stream."""
    import torch

    from pagellm_amd import workloads

    g = np.random.default_rng(11)
    zw = workloads.zipf32k()
    sw = workloads.spec32k()
    Bv = 16
    p, q = sw["p"][:Bv], sw["q"][:Bv]
    draft = np.asarray(sw["draft"][:Bv], dtype=np.int32)
    acc_u, res_u = sw["accept_u"][:Bv], sw["resample_u"][:Bv]
    _, k1, V = p.shape
    N, D, Vh = 8, 256, 3000
    h = g.normal(0, 1, (N, D)).astype(np.float32)
    norm = g.normal(1, 0.1, D).astype(np.float32)
    wt = g.normal(0, 0.05, (D, Vh)).astype(np.float32)

    def verify_call(c):
        d = {n: c.to_device(a) for n, a in dict(p=p, q=q, d=draft, a=acc_u, w=res_u).items()}
        tok, nacc = c.empty((Bv, k1), np.int32), c.empty((Bv,), np.int32)
        c.verify(d["p"].ptr, d["q"].ptr, _native.PLH_F64, Bv, k1 - 1, V, d["d"].ptr, d["a"].ptr, d["w"].ptr, 0,
                 tok.ptr, nacc.ptr)
        tok.keep = nacc.keep = d
        return tok, nacc

    def head_call(c):
        d = {n: c.to_device(a) for n, a in dict(h=h, n=norm, w=wt).items()}
        out = c.empty((N, Vh), np.float32)
        c.rmsnorm_lm_head(d["h"].ptr, D, N, D, d["n"].ptr, 1e-6, d["w"].ptr, Vh, Vh, out.ptr, Vh)
        out.keep = d
        return out

    c = _native.Context(0)
    try:
        ref_s = _launch_rows(c, zw, rows=48).download()
        ref_t, ref_n = (a.download() for a in verify_call(c))
        ref_h = head_call(c).download()
    finally:
        c.close()
    c = _native.Context(0)
    try:
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        got = []
        c.set_stream(s1.cuda_stream)
        got.append(("head", head_call(c)))
        c.set_stream(s2.cuda_stream)
        got.append(("verify", verify_call(c)))
        c.set_stream(None)
        got.append(("sample", _launch_rows(c, zw, rows=48)))
        c.set_stream(s1.cuda_stream)
        got.append(("verify", verify_call(c)))
        got.append(("head", head_call(c)))
        c.set_stream(s2.cuda_stream)
        got.append(("sample", _launch_rows(c, zw, rows=48)))
        torch.cuda.synchronize()
        for i, (kind, r) in enumerate(got):
            if kind == "sample":
                assert np.array_equal(r.download(), ref_s), i
            elif kind == "verify":
                assert np.array_equal(r[0].download(), ref_t) and np.array_equal(r[1].download(), ref_n), i
            else:
                assert np.array_equal(r.download(), ref_h), i
    finally:
        c.set_stream(None)
        c.close()
