"""The decoder-state oracle (oracle/kvcache.py) against index formulas and invariants the
reference's operations fix (CPU only)."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import kvcache as kv


def test_split_heads_index_formula():
    """split_heads(x)[b, h, l, d] == x[b, l, h * D + d] (text_decoder.rs:638-643)."""
    rng = np.random.default_rng(0)
    b, length, heads, d = 2, 5, 3, 8
    x = rng.standard_normal((b, length, heads * d)).astype(np.float32)
    s = kv.split_heads(x, heads)
    assert s.shape == (b, heads, length, d)
    for bi, h, li, di in [(0, 0, 0, 0), (1, 2, 4, 7), (0, 1, 3, 5), (1, 0, 2, 6)]:
        assert s[bi, h, li, di] == x[bi, li, h * d + di]


def test_append_is_concatenation_and_commutes_with_split():
    rng = np.random.default_rng(1)
    a, b2, c = (rng.standard_normal((2, t, 24)).astype(np.float32) for t in (3, 1, 4))
    one = kv.self_cache_append(kv.self_cache_append(kv.self_cache_append(None, a), b2), c)
    two = kv.self_cache_append(a, np.concatenate([b2, c], axis=1))
    np.testing.assert_array_equal(one, two)
    np.testing.assert_array_equal(kv.split_heads(one, 3),
                                  np.concatenate([kv.split_heads(x, 3) for x in (a, b2, c)], axis=2))


def test_beam_restore_follows_parents():
    states = [np.full((1, 2), i, np.float32) for i in range(4)]
    out = kv.beam_restore(states, [2, 2, 0, 3])
    assert [int(s[0, 0]) for s in out] == [2, 2, 0, 3]
    assert out[0] is out[1]  # shared, as the reference's refcounted snapshots


@pytest.mark.parametrize("k_transposed", [True, False])
def test_cross_cache_layout(k_transposed):
    rng = np.random.default_rng(2)
    t, heads, d = 7, 2, 8
    k = rng.standard_normal((t, heads * d)).astype(np.float32)
    v = rng.standard_normal((t, heads * d)).astype(np.float32)
    kk, vv = kv.cross_cache_build(k, v, heads, "f32", k_transposed=k_transposed)
    for h, ti, di in [(0, 0, 0), (1, 6, 7), (1, 3, 2)]:
        assert vv[h, ti, di] == v[ti, h * d + di]
        assert (kk[h, di, ti] if k_transposed else kk[h, ti, di]) == k[ti, h * d + di]


def test_round_to_nearest_even():
    # bf16 keeps 8 significant bits: 1 + 2^-8 is a tie between 1 and 1 + 2^-7 -> 1 (even);
    # 1 + 3 * 2^-8 ties between 1 + 2^-7 and 1 + 2^-6 -> 1 + 2^-6 (even)
    x = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, 1 + 2 ** -7], np.float32)
    np.testing.assert_array_equal(kv.round_to(x, "bf16"), [1.0, 1 + 2 ** -6, 1 + 2 ** -7])
    # f16 keeps 11: 1 + 2^-11 ties -> 1
    np.testing.assert_array_equal(kv.round_to(np.array([1 + 2 ** -11], np.float32), "f16"), [1.0])


def test_causal_mask_brute_force():
    """Element by element: -inf exactly where key j > offset + i (text_decoder.rs:902-923)."""
    for q_len, k_len, offset in [(1, 1, 0), (4, 4, 0), (3, 8, 5), (5, 7, 1)]:
        m = kv.causal_mask(q_len, k_len, offset)
        assert m.shape == (q_len, k_len) and m.dtype == np.float32
        for i in range(q_len):
            for j in range(k_len):
                assert (m[i, j] == -np.inf) == (j > offset + i) and (m[i, j] in (0.0, -np.inf))
    # a prompt at offset 0 sees a lower triangle; the steady-state single token sees everything
    assert (np.isneginf(kv.causal_mask(4, 4, 0)) == np.triu(np.ones((4, 4), bool), 1)).all()
    assert not np.isneginf(kv.causal_mask(1, 9, 8)).any()


def test_three_op_attend_against_brute_force_loops():
    """Tiny case by explicit Python loops: masked softmax over keys, then the weighted sum."""
    rng = np.random.default_rng(3)
    b, h, tq, tk, d = 1, 2, 3, 5, 4
    q, k, v = (rng.standard_normal(s).astype(np.float32) for s in
               ((b, h, tq, d), (b, h, tk, d), (b, h, tk, d)))
    mask = kv.causal_mask(tq, tk, 2)
    got = kv.three_op_attend(q, k, v, 0.5, mask)
    for hh in range(h):
        for i in range(tq):
            s = [sum(0.5 * float(q[0, hh, i, t]) * float(k[0, hh, j, t]) for t in range(d))
                 + float(mask[i, j]) for j in range(tk)]
            mx = max(s)
            w = [math.exp(x - mx) for x in s]
            z = sum(w)
            for t in range(d):
                want = sum(w[j] / z * float(v[0, hh, j, t]) for j in range(tk))
                assert abs(got[0, hh, i, t] - want) < 1e-5
    # a fully visible row with all scores equal averages V
    same = kv.three_op_attend(np.zeros((1, 1, 1, d), np.float32), k[:, :1], v[:, :1], 1.0)
    np.testing.assert_allclose(same[0, 0, 0], v[0, 0].mean(axis=0), rtol=1e-6, atol=1e-6)
