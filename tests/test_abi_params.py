"""Request parameters down to the sampler's ABI arrays.

The server's request parser (``src/pagellm/serving/protocol.py:82-108``) is
the reference's own and stays as it is; what this package adds is the
packing of the parsed values into the arrays ``plh_sample`` reads.  The
checks: every float reaches the float64 arrays bit for bit and top_k the
int32 array, clamped to 2^31 - 1."""

from __future__ import annotations

import math
import struct
from dataclasses import dataclass

import numpy as np
import pytest

from pagellm_amd.params import SamplingParams
from pagellm_amd.sampling import abi_params


@dataclass(frozen=True)
class _Parsed:
    """The shape of a parsed request (``protocol.py:75-79``): the sampler
    reads only ``.params``."""

    prompt: str
    params: SamplingParams
    stream: bool = False


def _bits(x: float) -> bytes:
    return struct.pack("<d", x)


_ROWS = [
    {},
    {"temperature": 0.0, "top_k": 1},
    {"temperature": 5e-324, "top_p": math.nextafter(1.0, 0.0), "repetition_penalty": 1e308},
    {"temperature": 0.7, "top_k": 2**31 - 1, "top_p": 5e-324, "repetition_penalty": 1.0},
    {"temperature": 3.0, "top_k": 2**40, "top_p": 0.95, "repetition_penalty": 1.1},
    {"temperature": 1e-300, "top_k": 2**31, "top_p": 0.1 + 0.2},
    {"temperature": float(2**53 + 1), "top_p": 1.0, "repetition_penalty": math.nextafter(1.0, 2.0)},
]


@pytest.mark.parametrize("wrap", [False, True], ids=["params", "parsed-request"])
def test_values_reach_the_abi_unchanged(wrap):
    """Every float reaches the float64 arrays bit for bit (the smallest
    subnormal, one ulp from 1, integers beyond 2^53); top_k beyond int32
    clamps to 2^31 - 1, which disables the mask as any top_k >= V does."""
    sps = [SamplingParams(**kw) for kw in _ROWS]
    rows = [_Parsed("p", sp) for sp in sps] if wrap else sps
    arr = abi_params(rows)
    assert arr["temperature"].dtype == np.float64 and arr["top_p"].dtype == np.float64
    assert arr["repetition_penalty"].dtype == np.float64 and arr["top_k"].dtype == np.int32
    for b, kw in enumerate(_ROWS):
        for key, default in (("temperature", 1.0), ("top_p", 1.0), ("repetition_penalty", 1.0)):
            assert _bits(float(arr[key][b])) == _bits(float(kw.get(key, default))), (b, key)
        assert int(arr["top_k"][b]) == min(kw.get("top_k", 0), 2**31 - 1)


def test_shared_params_objects_pack_like_distinct_ones():
    """A batch of few distinct SamplingParams objects (the engine's usual
    case, one per request) takes the indexed packing; the arrays equal those
    of distinct equal objects."""
    sps = [SamplingParams(**kw) for kw in _ROWS]
    shared = [sps[i % 3] for i in range(40)]
    distinct = [SamplingParams(**_ROWS[i % 3]) for i in range(40)]
    a, b = abi_params(shared), abi_params(distinct)
    for key in a:
        assert a[key].dtype == b[key].dtype and np.array_equal(a[key], b[key])
