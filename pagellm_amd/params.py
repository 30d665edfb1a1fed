"""Per-request sampling parameters and per-sequence RNG construction.

Host-only objects, kept field-for-field compatible with the reference so
engine, scheduler, protocol and CLI code keep constructing them unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass(frozen=True)
class SamplingParams:
    """Same fields, defaults, validation and ``greedy`` property as
    ``src/pagellm/engine/sampling.py:22-49``.  Floats stay Python floats
    (IEEE double), which is the precision the kernels compute in."""

    max_tokens: int = 64
    temperature: float = 1.0  # 0 => greedy
    top_k: int = 0  # 0 => disabled
    top_p: float = 1.0  # 1 => disabled
    repetition_penalty: float = 1.0  # 1 => disabled; >1 discourages repeats
    seed: int | None = None
    n: int = 1  # parallel samples sharing one prompt
    stop: tuple[str, ...] = field(default_factory=tuple)

    def __post_init__(self) -> None:
        # validation order and messages follow sampling.py:33-45
        if self.max_tokens < 1:
            raise ValueError("max_tokens must be >= 1")
        if self.temperature < 0:
            raise ValueError("temperature must be >= 0")
        if self.top_k < 0:
            raise ValueError("top_k must be >= 0")
        if not 0 < self.top_p <= 1:
            raise ValueError("top_p must be in (0, 1]")
        if self.repetition_penalty <= 0:
            raise ValueError("repetition_penalty must be > 0")
        if self.n < 1:
            raise ValueError("n must be >= 1")

    @property
    def greedy(self) -> bool:
        return self.temperature == 0


def make_rng(seed: int | None, index: int) -> np.random.Generator:
    """``sampling.py:110-111``: one PCG64 stream per (seed, sequence index);
    ``seed=None`` draws OS entropy.  The GPU never generates randomness: the
    host draws uniforms from these generators in the reference's order."""
    return np.random.default_rng(None if seed is None else [seed, index])
