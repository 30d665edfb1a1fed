"""Request parameters from the ``/v1/completions`` wire format to the sampler's ABI.

The validation rules, defaults and error messages are those of
``src/pagellm/serving/protocol.py:31-108`` (a bad value becomes a
:class:`ProtocolError`, HTTP 400, before it reaches the engine), and the
response shapes those of ``:111-127``.  :func:`abi_params` is the step after
parsing: it packs the parsed values into the arrays ``plh_sample`` reads,
float64 for temperature, top_p and repetition_penalty (a JSON number parses to
a Python float, an IEEE double, so the value reaches the kernels unchanged)
and int32 for top_k (any top_k >= V disables the mask, so values above 2^31 - 1
are clamped to 2^31 - 1, which is >= every V the sampler accepts).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Sequence

import numpy as np

from .params import SamplingParams

__all__ = [
    "MAX_N",
    "MAX_STOP_STRINGS",
    "CompletionRequest",
    "ProtocolError",
    "abi_params",
    "choice",
    "completion_chunk",
    "error_body",
    "parse_completion_request",
]

MAX_N = 16
MAX_STOP_STRINGS = 4


class ProtocolError(ValueError):
    """A request the server must reject with HTTP 400."""


@dataclass(frozen=True)
class CompletionRequest:
    prompt: str
    params: SamplingParams
    stream: bool


def _int(body: dict, key: str, default: int, lo: int, hi: int | None = None) -> int:
    """protocol.py:31-39: an int (bool is not one) within [lo, hi]."""
    v = body.get(key, default)
    if isinstance(v, bool) or not isinstance(v, int):
        raise ProtocolError(f"{key} must be an integer")
    if v < lo or (hi is not None and v > hi):
        raise ProtocolError(f"{key} must be " + (f">= {lo}" if hi is None else f"in [{lo}, {hi}]"))
    return v


def _float(body: dict, key: str, default: float) -> float:
    """protocol.py:42-46: a finite int or float (not bool), as a float."""
    v = body.get(key, default)
    if isinstance(v, bool) or not isinstance(v, (int, float)) or not math.isfinite(v):
        raise ProtocolError(f"{key} must be a finite number")
    return float(v)


def _prompt(body: dict) -> str:
    """protocol.py:49-61: one non-empty string, bare or in a one-element list."""
    if "prompt" not in body:
        raise ProtocolError("missing required field: prompt")
    prompt = body["prompt"]
    if isinstance(prompt, list):
        if len(prompt) != 1 or not isinstance(prompt[0], str):
            raise ProtocolError("only a single string prompt is supported")
        prompt = prompt[0]
    if not isinstance(prompt, str):
        raise ProtocolError("prompt must be a string")
    if not prompt:
        raise ProtocolError("prompt must not be empty")
    return prompt


def _stop(body: dict) -> tuple[str, ...]:
    """protocol.py:64-78: None, one non-empty string, or up to four of them."""
    stop = body.get("stop")
    if stop is None:
        return ()
    if isinstance(stop, str):
        stop = [stop]
    ok = isinstance(stop, list) and len(stop) <= MAX_STOP_STRINGS and all(isinstance(s, str) and s for s in stop)
    if not ok:
        raise ProtocolError(
            f"stop must be a non-empty string or a list of up to {MAX_STOP_STRINGS} non-empty strings")
    return tuple(stop)


def parse_completion_request(body: Any) -> CompletionRequest:
    """protocol.py:81-108: validate a decoded JSON body into engine inputs.
    Defaults: max_tokens 16, temperature 1.0, top_k 0, top_p 1.0,
    repetition_penalty 1.0, n 1, no stop strings, no streaming."""
    if not isinstance(body, dict):
        raise ProtocolError("request body must be a JSON object")
    prompt = _prompt(body)
    seed = body.get("seed")
    if seed is not None and (isinstance(seed, bool) or not isinstance(seed, int) or seed < 0):
        raise ProtocolError("seed must be a non-negative integer")
    stream = body.get("stream", False)
    if not isinstance(stream, bool):
        raise ProtocolError("stream must be a boolean")
    try:
        params = SamplingParams(
            max_tokens=_int(body, "max_tokens", 16, 1),
            temperature=_float(body, "temperature", 1.0),
            top_k=_int(body, "top_k", 0, 0),
            top_p=_float(body, "top_p", 1.0),
            repetition_penalty=_float(body, "repetition_penalty", 1.0),
            seed=seed,
            n=_int(body, "n", 1, 1, MAX_N),
            stop=_stop(body),
        )
    except ProtocolError:
        raise
    except ValueError as e:  # the range checks SamplingParams owns
        raise ProtocolError(str(e)) from e
    return CompletionRequest(prompt, params, stream)


def abi_params(params: Sequence[SamplingParams | CompletionRequest]) -> dict[str, np.ndarray]:
    """The per-row parameter arrays of ``plh_sample`` for one batch:
    ``temperature``, ``top_p``, ``repetition_penalty`` float64 [B] and
    ``top_k`` int32 [B]."""
    from .sampling import _pack_params  # the packing every sampler entry point uses

    rows = [r.params if isinstance(r, CompletionRequest) else r for r in params]
    t, k, p, r = _pack_params(rows)
    return {"temperature": t, "top_k": k, "top_p": p, "repetition_penalty": r}


def error_body(message: str, kind: str = "invalid_request_error") -> dict:
    """protocol.py:111-112."""
    return {"error": {"message": message, "type": kind}}


def completion_chunk(rid: str, created: int, model: str, choices: list[dict]) -> dict:
    """protocol.py:115-122: one response object (or one SSE delta)."""
    return {"id": rid, "object": "text_completion", "created": created, "model": model, "choices": choices}


def choice(index: int, text: str, finish_reason: str | None) -> dict:
    """protocol.py:125-126."""
    return {"index": index, "text": text, "logprobs": None, "finish_reason": finish_reason}
