"""CPU oracle for the pagellm sampler and logits producer: test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the reference results or as the timed
CPU baseline.  The product path (``pagellm_amd``) never imports it.
"""

from .sampler import (  # noqa: F401
    ScriptedRNG,
    apply_repetition_penalty,
    draw,
    draw_boundary_gap,
    probs,
    sample,
    sample_batch,
    top_p_boundary_gap,
    verify,
    verify_batch,
    verify_boundary_gap,
)
from .head import head_error_bound, lm_head_logits, rms_norm  # noqa: F401,E402
