"""Wire-format parameters (``src/pagellm/serving/protocol.py``) down to the
sampler's ABI arrays.  The request bodies are those of the reference's
``tests/unit/test_protocol.py:15-90``; the ABI checks are that every parsed
value reaches the arrays unchanged (float64 bits, int32 top_k)."""

from __future__ import annotations

import math
import struct

import numpy as np
import pytest

from pagellm_amd.wire import (
    MAX_N,
    ProtocolError,
    abi_params,
    choice,
    completion_chunk,
    error_body,
    parse_completion_request,
)


def test_defaults_follow_openai():
    r = parse_completion_request({"prompt": "hi"})
    assert r.prompt == "hi" and r.stream is False
    assert r.params.max_tokens == 16 and r.params.temperature == 1.0 and r.params.n == 1
    assert r.params.stop == () and r.params.seed is None


def test_full_request_is_mapped():
    r = parse_completion_request({
        "prompt": ["ROMEO:"], "max_tokens": 5, "temperature": 0, "top_k": 3, "top_p": 0.9,
        "repetition_penalty": 1.2, "seed": 7, "n": 2, "stop": ["\n", "END"], "stream": True,
    })
    p = r.params
    assert r.prompt == "ROMEO:" and r.stream
    assert (p.max_tokens, p.temperature, p.top_k, p.top_p) == (5, 0.0, 3, 0.9)
    assert (p.repetition_penalty, p.seed, p.n, p.stop) == (1.2, 7, 2, ("\n", "END"))
    assert isinstance(p.temperature, float)


def test_single_stop_string_is_wrapped():
    assert parse_completion_request({"prompt": "a", "stop": "x"}).params.stop == ("x",)


@pytest.mark.parametrize("body", [
    [], {}, {"prompt": 5}, {"prompt": ""}, {"prompt": ["a", "b"]}, {"prompt": [1]},
    {"prompt": "a", "seed": "abc"}, {"prompt": "a", "seed": -1}, {"prompt": "a", "seed": True},
    {"prompt": "a", "seed": 1.5}, {"prompt": "a", "max_tokens": 0}, {"prompt": "a", "max_tokens": True},
    {"prompt": "a", "max_tokens": "10"}, {"prompt": "a", "n": MAX_N + 1}, {"prompt": "a", "temperature": -1},
    {"prompt": "a", "temperature": math.nan}, {"prompt": "a", "temperature": "hot"}, {"prompt": "a", "top_p": 0},
    {"prompt": "a", "top_k": -2}, {"prompt": "a", "repetition_penalty": 0}, {"prompt": "a", "stop": ""},
    {"prompt": "a", "stop": ["a", "b", "c", "d", "e"]}, {"prompt": "a", "stop": [1]},
    {"prompt": "a", "stream": "yes"},
    # beyond the reference's list: infinities, top_p above 1, a bool top_k
    {"prompt": "a", "temperature": math.inf}, {"prompt": "a", "top_p": 1.5}, {"prompt": "a", "top_k": False},
])
def test_invalid_requests_raise_protocol_error(body):
    with pytest.raises(ProtocolError):
        parse_completion_request(body)


def test_response_shapes():
    c = completion_chunk("cmpl-1", 123, "m", [choice(0, "hi", "length")])
    assert c == {"id": "cmpl-1", "object": "text_completion", "created": 123, "model": "m",
                 "choices": [{"index": 0, "text": "hi", "logprobs": None, "finish_reason": "length"}]}
    assert error_body("nope")["error"] == {"message": "nope", "type": "invalid_request_error"}


def _bits(x: float) -> bytes:
    return struct.pack("<d", x)


def test_parsed_values_reach_the_abi_unchanged():
    """Every float reaches the float64 arrays bit for bit (including the
    smallest subnormal and values one ulp from 1); integers given for float
    fields become exact floats; top_k beyond int32 clamps to 2^31 - 1, which
    disables the mask as any top_k >= V does."""
    bodies = [
        {"prompt": "a"},
        {"prompt": "a", "temperature": 0, "top_k": 1},
        {"prompt": "a", "temperature": 5e-324, "top_p": math.nextafter(1.0, 0.0), "repetition_penalty": 1e308},
        {"prompt": "a", "temperature": 0.7, "top_k": 2**31 - 1, "top_p": 5e-324, "repetition_penalty": 1},
        {"prompt": "a", "temperature": 3, "top_k": 2**40, "top_p": 0.95, "repetition_penalty": 1.1},
        {"prompt": "a", "temperature": 1e-300, "top_k": 2**31, "top_p": 0.1 + 0.2},
    ]
    reqs = [parse_completion_request(b) for b in bodies]
    arr = abi_params(reqs)
    assert arr["temperature"].dtype == np.float64 and arr["top_p"].dtype == np.float64
    assert arr["repetition_penalty"].dtype == np.float64 and arr["top_k"].dtype == np.int32
    for b, (body, r) in enumerate(zip(bodies, reqs)):
        for key, default in (("temperature", 1.0), ("top_p", 1.0), ("repetition_penalty", 1.0)):
            want = float(body.get(key, default))
            assert _bits(float(arr[key][b])) == _bits(want), (b, key)
            assert getattr(r.params, key) == want
        want_k = min(body.get("top_k", 0), 2**31 - 1)
        assert int(arr["top_k"][b]) == want_k
    # the same arrays whether given requests or their SamplingParams
    again = abi_params([r.params for r in reqs])
    for key in arr:
        assert np.array_equal(arr[key], again[key])
