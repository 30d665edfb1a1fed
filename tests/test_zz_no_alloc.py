"""plh_sample_noalloc (needs an MI355X): the same ids as plh_sample on the
same inputs, over two calls in a row (the second smaller, so the scratch
array still holds the first call's data), through the C ABI; a batch whose
workspace exceeds the scratch array is refused with a clear error.  Runs
last: its name sorts after every other test file."""

from __future__ import annotations

import numpy as np
import pytest

from pagellm_amd import _native, workloads
from pagellm_amd.sampling import _nucleus_hint, _pack_histories, _pack_params

pytestmark = pytest.mark.gpu


def _launch(c, w, noalloc, rows=None):
    """Uploads the rows and launches plh_sample(_noalloc) on the context's
    stream; returns the device ids (not yet waited for)."""
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
    fn = c.sample_noalloc if noalloc else c.sample
    fn(d["x"].ptr, _native.dtype_code(x.dtype), V, B, V, hi.ptr if hi else None, ho.ptr if ho else None,
       d["t"].ptr, d["k"].ptr, d["p"].ptr, d["r"].ptr, d["u"].ptr, out.ptr, None, _nucleus_hint(t, k, p, V))
    out.keep = (d, hi, ho)  # the inputs live as long as the output
    return out


def _call(c, w, noalloc, rows=None):
    return _launch(c, w, noalloc, rows).download()


def test_noalloc_matches_sample_on_two_calls_in_a_row():
    c = _native.Context(0)
    try:
        big = workloads.mixed128k()
        small = workloads.zipf32k()
        ref_big = _call(c, big, False)
        ref_small = _call(c, small, False, rows=40)
        got_big = _call(c, big, True)
        got_small = _call(c, small, True, rows=40)  # smaller: the array still holds the first call's data
        assert np.array_equal(got_big, ref_big)
        assert np.array_equal(got_small, ref_small)
        # and again in the other order, with a third, different batch between
        got_small2 = _call(c, small, True, rows=40)
        got_char = _call(c, workloads.char65(), True)
        assert np.array_equal(got_small2, ref_small)
        assert np.array_equal(got_char, _call(c, workloads.char65(), False))
        # a batch of nucleus rows only (the nucleus kernels, no merge launch)
        nuc = workloads.zipf152k(rows=8)
        assert np.array_equal(_call(c, nuc, True), _call(c, nuc, False))
    finally:
        c.close()


def test_noalloc_orders_calls_on_two_streams():
    """Back-to-back noalloc calls of one context on two streams, with no
    host wait between them: the second waits on the first (both share the
    GPU's scratch array), and both return plh_sample's ids."""
    import torch

    c = _native.Context(0)
    try:
        big = workloads.mixed128k()
        small = workloads.zipf32k()
        ref_big = _call(c, big, False)
        ref_small = _call(c, small, False, rows=40)
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        c.set_stream(s1.cuda_stream)
        o1 = _launch(c, big, True)
        c.set_stream(s2.cuda_stream)
        o2 = _launch(c, small, True, rows=40)
        torch.cuda.synchronize()
        assert np.array_equal(o1.download(), ref_big)
        assert np.array_equal(o2.download(), ref_small)
    finally:
        c.set_stream(None)
        c.close()


def test_noalloc_refuses_a_batch_beyond_its_scratch():
    c = _native.Context(0)
    try:
        B, V = 2048, 131072  # about 260 MB of fast-path workspace
        d_x = c.empty((B, V), np.float32)
        one = c.to_device(np.ones(B))
        k0 = c.to_device(np.zeros(B, dtype=np.int32))
        out = c.empty((B,), np.int32)
        with pytest.raises(ValueError, match="workspace"):
            c.sample_noalloc(d_x.ptr, _native.PLH_F32, V, B, V, None, None, one.ptr, k0.ptr, one.ptr, one.ptr,
                             one.ptr, out.ptr, None, 0)
    finally:
        c.close()
