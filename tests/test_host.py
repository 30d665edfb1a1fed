"""Host-side logic of the drop-in API (CPU only): argument packing, numpy
indexing semantics for histories, randomness consumption order, workload
generators."""

from __future__ import annotations

import numpy as np
import pytest

from pagellm_amd import sampling as S
from pagellm_amd import workloads as W
from pagellm_amd.params import SamplingParams, make_rng


def test_params_mirror_reference_defaults():
    p = SamplingParams()
    assert (p.max_tokens, p.temperature, p.top_k, p.top_p, p.repetition_penalty, p.seed, p.n, p.stop) == (
        64, 1.0, 0, 1.0, 1.0, None, 1, ())
    assert SamplingParams(temperature=0).greedy and not p.greedy
    with pytest.raises(Exception):
        p.temperature = 2.0  # frozen


def test_make_rng_is_numpy_seed_sequence():
    a = make_rng(7, 3).random(4)
    b = np.random.default_rng([7, 3]).random(4)
    assert np.array_equal(a, b)


def test_history_ids_follow_numpy_indexing():
    assert list(S._history_ids([0, 3, -1, -5], 5)) == [0, 3, 4, 0]
    with pytest.raises(IndexError):
        S._history_ids([5], 5)
    with pytest.raises(IndexError):
        S._history_ids([-6], 5)
    assert S._history_ids([], 5).size == 0


def test_histories_packed_only_for_active_penalty():
    params = [SamplingParams(repetition_penalty=1.0), SamplingParams(repetition_penalty=1.3),
              SamplingParams(repetition_penalty=2.0)]
    ids, off = S._pack_histories([[1, 2], [3, 3, 4], []], params, 3, 10)
    assert list(off) == [0, 0, 3, 3] and list(ids) == [3, 3, 4]
    assert S._pack_histories([[1], [2], [3]], [SamplingParams()] * 3, 3, 10) == (None, None)
    assert S._pack_histories(None, params, 3, 10) == (None, None)


def test_uniforms_one_per_nongreedy_row_in_order():
    params = [SamplingParams(temperature=0), SamplingParams(), SamplingParams(top_p=0.5)]
    rngs = [None, make_rng(1, 0), make_rng(2, 0)]
    u = S._draw_uniforms(params, rngs, 3)
    assert u[0] == 0.0
    assert u[1] == make_rng(1, 0).random() and u[2] == make_rng(2, 0).random()
    with pytest.raises(ValueError):
        S._draw_uniforms([SamplingParams()], [None], 1)


def test_param_packing():
    t, k, p, r = S._pack_params([SamplingParams(temperature=0.6, top_k=40, top_p=0.95, repetition_penalty=1.1),
                                 SamplingParams(top_k=10**12)])
    assert t.dtype == np.float64 and k.dtype == np.int32
    assert list(t) == [0.6, 1.0] and list(k) == [40, 2**31 - 1] and list(p) == [0.95, 1.0]
    assert list(r) == [1.1, 1.0]


def test_float_promotion():
    assert S._as_float_rows(np.zeros(3, np.float32)).dtype == np.float32
    assert S._as_float_rows(np.zeros(3, np.float16)).dtype == np.float64
    assert S._as_float_rows([1, 2, 3]).dtype == np.float64


def test_workload_char65_matches_recipe():
    w = W.char65()
    g = np.random.default_rng(1001)
    assert np.array_equal(w["logits"], g.normal(0.0, 2.0, (16, 65)).astype(np.float32))
    assert np.array_equal(np.stack(w["contexts"]), g.integers(0, 65, (16, 64)))
    assert all(p.greedy for p in w["params"][:4])
    assert all(p == SamplingParams(temperature=0.8, top_k=10, top_p=0.9, repetition_penalty=1.1)
               for p in w["params"][4:])
    assert w["uniforms"][0] == 0.0 and w["uniforms"][5] == make_rng(5, 0).random()


def test_algorithmic_bytes_counts_penalised_histories_only():
    w = dict(logits=np.zeros((4, 100), np.float32), params=[SamplingParams(), SamplingParams(repetition_penalty=2.0)] * 2,
             contexts=[np.arange(10)] * 4)
    assert W.algorithmic_bytes(w) == 4 * 100 * 4 + 2 * 10 * 4 + 4 * 48


def test_mixed_workload_bytes_formula():
    # 256 x 128256 fp32 + 64 penalised rows x 2048 ids + 48 B/row
    assert 256 * 128256 * 4 + 64 * 2048 * 4 + 256 * 48 == 131870720


def test_round_histories_spans_cover_context_and_draft_prefix():
    """Target row (b, i) of a speculative round reads ``ctx_b + drafts_b[:i]``
    (speculative.py:127); sequences with the penalty off read nothing."""
    from pagellm_amd.speculative import _round_histories

    V = 50
    ctxs = [[1, 2, -1], [7, 8], [], [3]]
    params = [SamplingParams(repetition_penalty=1.2), SamplingParams(repetition_penalty=1.0),
              SamplingParams(repetition_penalty=1.1), SamplingParams(repetition_penalty=0.9)]
    d = np.array([[4, 5], [6, 9], [10, 11], [12, 13]], dtype=np.int32)
    ids, spans = _round_histories(ctxs, params, d, V)
    spans = spans.reshape(4, 3, 2)
    for b in range(4):
        for i in range(3):
            got = list(ids[spans[b, i, 0]:spans[b, i, 1]])
            want = [] if params[b].repetition_penalty == 1.0 else \
                [t % V for t in ctxs[b]] + list(d[b, :i])
            assert got == want, (b, i, got, want)
    # nothing to read at all
    assert _round_histories([[], []], [SamplingParams()] * 2, np.zeros((2, 0), np.int32), V) == (None, None)


def test_bulk_uniform_draws_match_scalar_draws():
    """Drawing n uniforms in one call consumes the Generator exactly as n
    calls of ``random()`` do (the speculative round replays this way)."""
    a, b = make_rng(11, 2), make_rng(11, 2)
    x = [a.random() for _ in range(6)]
    assert np.array_equal(np.array(x), b.random(6))
    assert a.bit_generator.state == b.bit_generator.state


def test_nucleus_hint_only_for_high_top_p_rows_without_top_k():
    """The hint is set when some non-greedy row has no top-k (0 or >= V) and
    0.98 <= top_p < 1, with PLH_SAMPLE_NUCLEUS_ONLY when every row is one."""
    from pagellm_amd import _native

    def hint(rows, V=100):
        return S._nucleus_hint(*S._pack_params(rows)[:3], V)

    both = _native.PLH_SAMPLE_NUCLEUS | _native.PLH_SAMPLE_NUCLEUS_ONLY
    assert hint([SamplingParams(top_p=0.99)]) == both
    assert hint([SamplingParams(top_p=0.98, top_k=100)]) == both  # top_k >= V is off
    assert hint([SamplingParams(top_p=0.97)]) == 0
    assert hint([SamplingParams(top_p=1.0)]) == 0
    assert hint([SamplingParams(top_p=0.99, top_k=40)]) == 0
    assert hint([SamplingParams(top_p=0.99, temperature=0.0)]) == 0
    assert hint([SamplingParams(), SamplingParams(top_p=0.995)]) == _native.PLH_SAMPLE_NUCLEUS
    assert hint([SamplingParams(top_p=0.99), SamplingParams(top_p=0.995, temperature=0.7)]) == both


def test_penalised_rows_beyond_the_bitmap_fail_on_the_host_with_the_reason():
    """Penalised histories need V <= 262144 (the kernels' per-row bitmap);
    a larger vocabulary is refused before anything reaches the device, with
    the reason.  Rows without an active penalty are not affected."""
    from pagellm_amd.sampling import MAX_PENALTY_VOCAB, _pack_histories

    V = MAX_PENALTY_VOCAB + 1
    pen, plain = SamplingParams(repetition_penalty=1.1), SamplingParams()
    with pytest.raises(NotImplementedError, match="262144"):
        _pack_histories([[1, 2, 3]], [pen], 1, V)
    assert _pack_histories([[1, 2, 3]], [plain], 1, V) == (None, None)
    assert _pack_histories([[]], [pen], 1, V) == (None, None)
    ids, off = _pack_histories([[1, 2, 3]], [pen], 1, MAX_PENALTY_VOCAB)
    assert list(ids) == [1, 2, 3] and list(off) == [0, 3]
