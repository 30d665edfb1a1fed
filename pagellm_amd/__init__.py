"""pagellm_amd: MI355X-native batched sampler for pagellm.

Drop-in replacement for ``pagellm.engine.sampling`` and the accept/resample
step of ``pagellm.engine.speculative``, computed by hand-written gfx950 HIP
kernels behind the C ABI of ``libpagellm_hip.so``.
"""

from .params import SamplingParams, make_rng

__all__ = ["SamplingParams", "make_rng"]
