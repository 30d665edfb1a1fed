"""GPU parity of the logits producer (``plh_rmsnorm_lm_head``) against the
CPU oracle and against torch's float32 product, and the head -> sampler chain
with the logits kept in HBM (needs an MI355X).

Tolerance: float32 products summed in a different order than numpy's BLAS
(or hipBLAS) differ by rounding only, which scales with
``sum_d |a[n, d]| |W[d, v]|`` (``oracle.head_error_bound``); every logit must
be within 1e-5 of that bound (a wrong index or a dropped term is off by
O(1) of it).  The reference's own model tests compare float32 logits at
rtol = atol = 1e-4 (``tests/unit/test_model.py:55``)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from pagellm_amd import head as H

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _case(seed, N, D, V, scale=1.0):
    g = np.random.default_rng(seed)
    h = (scale * g.standard_normal((N, D))).astype(np.float32)
    norm = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
    W = (0.02 * g.standard_normal((D, V))).astype(np.float32)
    return h, norm, W


@pytest.mark.parametrize("N,D,V", [
    (1, 128, 65),        # the reference model's width, the character vocabulary
    (3, 100, 1000),      # D not a multiple of the 32-wide k stage, ragged V tile
    (300, 64, 513),      # two row tiles, the second ragged
    (256, 128, 4096),    # full row tile, V on the vector-load path
    (17, 4096, 300),     # deep k loop
    (5, 1, 7),           # one column of k
])
def test_head_matches_oracle(N, D, V):
    print(f"[head] N={N} D={D} V={V}", flush=True)
    h, norm, W = _case(N * 7 + D, N, D, V)
    got = H.rms_norm_lm_head(h, norm, W, 1e-5)
    ref = oracle.lm_head_logits(h, norm, W, 1e-5)
    bound = oracle.head_error_bound(h, norm, W, 1e-5)
    assert got.shape == (N, V) and got.dtype == np.float32
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= TOL * bound + 1e-30), float(np.max(err / (bound + 1e-30)))
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


def test_tiny_rows_and_eps():
    """Rows of norm ~1e-3 (eps visible), an all-zero row (r = 1/sqrt(eps))."""
    h, norm, W = _case(3, 6, 96, 257, scale=1e-3)
    h[2] = 0.0
    got = H.rms_norm_lm_head(h, norm, W, 1e-5)
    ref = oracle.lm_head_logits(h, norm, W, 1e-5)
    bound = oracle.head_error_bound(h, norm, W, 1e-5)
    assert np.all(np.abs(got - ref) <= TOL * bound + 1e-30)
    assert np.all(got[2] == 0.0)


def test_strided_torch_buffers_and_full_size_against_torch():
    """h, lm_head and out as row-strided views (out a slice of a larger
    buffer, as the sampler's rotating logits sets are), at 256 x 4096 x
    128256, against torch's float32 product on the same device."""
    import torch

    torch.manual_seed(0)
    dev = torch.device("cuda:0")
    N, D, V = 256, 4096, 128256
    hbuf = torch.randn((N, D + 8), device=dev, dtype=torch.float32)
    h = hbuf[:, :D]
    norm = 1 + 0.1 * torch.randn(D, device=dev, dtype=torch.float32)
    W = 0.02 * torch.randn((D, V), device=dev, dtype=torch.float32)
    obuf = torch.full((N, V + 64), float("nan"), device=dev, dtype=torch.float32)
    out = obuf[:, :V]
    print("[head] full size 256x4096x128256", flush=True)
    H.rms_norm_lm_head(h, norm, W, 1e-5, out=out)
    torch.cuda.synchronize()
    assert torch.isnan(obuf[:, V:]).all(), "wrote past the row"
    r = torch.rsqrt((h.double() ** 2).mean(dim=1, keepdim=True) + 1e-5).float()
    a = (h * r) * norm
    ref = a @ W
    bound = a.abs().double() @ W.abs().double()
    err = (out.double() - ref.double()).abs()
    worst = float((err / bound).max())
    print(f"[head] worst error / bound {worst:.3e}", flush=True)
    assert worst <= TOL


def test_logits_stay_on_device_into_the_sampler():
    """LogitsHead output (a torch CUDA tensor) goes straight into
    sample_batch; ids equal the oracle's on the same logits (greedy rows
    exactly; sampled rows except draws within 1e-6 of a CDF boundary)."""
    from pagellm_amd.sampling import SamplingParams, sample_batch

    N, D, V = 12, 256, 32000
    h, norm, W = _case(11, N, D, V)
    head = H.LogitsHead(norm, W, 1e-5)
    logits = head(h)
    params = [SamplingParams(temperature=0.0)] * 4 + [SamplingParams(temperature=0.8, top_k=40)] * 4 + \
        [SamplingParams(temperature=1.0, top_p=0.9)] * 4
    u = np.random.default_rng(3).random(N)
    ids = sample_batch(logits, params, uniforms=u)
    host = logits.cpu().numpy()
    ref = oracle.sample_batch(host, params, u, None)
    for b in range(N):
        if ids[b] != ref[b]:
            assert b >= 4
            gap = oracle.draw_boundary_gap(oracle.probs(host[b], params[b], ()), u[b])
            cut = oracle.top_p_boundary_gap(host[b], params[b], ())
            assert gap < 1e-6 or cut < 1e-12, (b, gap, cut)
    bound = oracle.head_error_bound(h, norm, W, 1e-5)
    assert np.all(np.abs(host - oracle.lm_head_logits(h, norm, W, 1e-5)) <= TOL * bound + 1e-30)
