"""The logits producer on the GPU: the model's final RMSNorm and lm_head.

``Transformer.forward`` ends with ``rms_norm(h, self.w["norm"], eps) @
self.w["lm_head"]`` (``src/pagellm/model/transformer.py:271``, ``rms_norm``
at ``:79-82``), in the model's dtype, float32 by default
(``init_weights``, ``:184-197``).  :func:`rms_norm_lm_head` computes the same
float32 logits with ``plh_rmsnorm_lm_head`` (fp32 matrix cores) and writes
them where the sampler reads them, so that a step's logits never leave HBM:

    head = LogitsHead(w["norm"], w["lm_head"], cfg.norm_eps)   # weights resident
    ids = sampler.sample(head(h), params, rngs, keys)           # no host copy

``h``, the weights and ``out`` may be numpy arrays (uploaded, and the logits
downloaded: the parity path) or torch CUDA float32 tensors (read and written
in place on torch's current stream).
"""

from __future__ import annotations

import numpy as np

from . import _native
from .sampling import _is_torch_cuda

__all__ = ["LogitsHead", "rms_norm_lm_head"]


def _ctx(ctx):
    return ctx if ctx is not None else _native.default_context()


def _check_f32_rows(x, name: str, ndim: int):
    import torch

    if x.dtype != torch.float32:
        raise TypeError(f"{name} must be float32")
    if x.dim() != ndim or (x.numel() and x.stride(-1) != 1):
        raise ValueError(f"{name} must be {ndim}-D with unit stride in its last dimension")


def rms_norm_lm_head(h, norm, lm_head, eps: float = 1e-5, *, out=None, ctx: _native.Context | None = None):
    """``rms_norm(h, norm, eps) @ lm_head`` in float32: h [N, D], norm [D],
    lm_head [D, V] -> logits [N, V].  numpy in, numpy out; or torch CUDA
    tensors in, and the logits in ``out`` (a new tensor when None; a
    row-strided view of a larger buffer is fine)."""
    c = _ctx(ctx)
    if _is_torch_cuda(h):
        import torch

        _check_f32_rows(h, "h", 2)
        _check_f32_rows(norm, "norm", 1)
        _check_f32_rows(lm_head, "lm_head", 2)
        N, D = int(h.shape[0]), int(h.shape[1])
        if int(norm.shape[0]) != D or int(lm_head.shape[0]) != D:
            raise ValueError("norm must be [D] and lm_head [D, V] for h [N, D]")
        V = int(lm_head.shape[1])
        if out is None:
            out = torch.empty((N, V), dtype=torch.float32, device=h.device)
        _check_f32_rows(out, "out", 2)
        if tuple(out.shape) != (N, V):
            raise ValueError(f"out must be [{N}, {V}]")
        c.set_stream(torch.cuda.current_stream(h.device).cuda_stream)
        c.rmsnorm_lm_head(h.data_ptr(), int(h.stride(0)), N, D, norm.data_ptr(), float(eps), lm_head.data_ptr(),
                          int(lm_head.stride(0)), V, out.data_ptr(), int(out.stride(0)))
        return out
    h = np.ascontiguousarray(h, dtype=np.float32)
    norm = np.ascontiguousarray(norm, dtype=np.float32)
    lm_head = np.ascontiguousarray(lm_head, dtype=np.float32)
    if h.ndim != 2 or norm.ndim != 1 or lm_head.ndim != 2:
        raise ValueError("h must be [N, D], norm [D] and lm_head [D, V]")
    N, D = h.shape
    if norm.shape[0] != D or lm_head.shape[0] != D:
        raise ValueError("norm must be [D] and lm_head [D, V] for h [N, D]")
    V = lm_head.shape[1]
    if N == 0:
        return np.zeros((0, V), dtype=np.float32)
    c.set_stream(None)
    d_h = c.scratch_upload("head_h", h)
    d_n = c.scratch_upload("head_norm", norm)
    d_w = c.scratch_upload("head_w", lm_head)
    d_o = c.scratch("head_out", (N, V), np.float32)
    c.rmsnorm_lm_head(d_h.ptr, D, N, D, d_n.ptr, float(eps), d_w.ptr, V, V, d_o.ptr, V)
    return d_o.download()


class LogitsHead:
    """The final norm and lm_head held in HBM; calling it with the last
    hidden states of a step returns that step's float32 logits on the device
    (a torch CUDA tensor), ready for ``BatchSampler.sample`` or
    ``sample_batch``."""

    def __init__(self, norm, lm_head, eps: float = 1e-5, *, device: int = 0, ctx: _native.Context | None = None):
        import torch

        self.ctx = _ctx(ctx)
        dev = torch.device("cuda", device)
        self.norm = torch.as_tensor(np.asarray(norm, dtype=np.float32)).to(dev) if not _is_torch_cuda(norm) else norm
        self.lm_head = (torch.as_tensor(np.ascontiguousarray(lm_head, dtype=np.float32)).to(dev)
                        if not _is_torch_cuda(lm_head) else lm_head)
        self.eps = float(eps)
        self.D, self.V = int(self.lm_head.shape[0]), int(self.lm_head.shape[1])

    def __call__(self, h, out=None):
        import torch

        if not _is_torch_cuda(h):
            h = torch.as_tensor(np.ascontiguousarray(h, dtype=np.float32)).to(self.lm_head.device)
        return rms_norm_lm_head(h, self.norm, self.lm_head, self.eps, out=out, ctx=self.ctx)
